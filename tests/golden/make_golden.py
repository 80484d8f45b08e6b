"""Writes the golden vectors of tests/golden/ from the reference's own CPU path.

Runs in the build container only (needs /root/reference and oracle/_ref, built by
`make -C oracle ref` from the reference's cpu_ops.cpp / cpu_kquants.cpp /
cpu_threadpool.cpp). The reference's friday_cpu::rope and
friday_cpu::decodeAttention (cpu_ops.cpp:26-83) produce the expected outputs;
inputs are seeded N(0,1) values rounded to fp16. Output: golden_cpu_path.npz
(inputs and outputs as fp16 bit patterns / fp32 values; data only).

    python tests/golden/make_golden.py
"""
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(HERE, "..", "..", "oracle"))
from py_oracle import RefCpu  # noqa: E402


def f16(rng, shape, scale=1.0):
    return (rng.standard_normal(shape, dtype=np.float32) * np.float32(scale)).astype(np.float16)


def main():
    ref = RefCpu()
    out = {}
    # --- case A: BASELINE config 1 (Qwen2.5-0.5B layer shapes): 14q/2kv, d64, base 1e6, neox,
    # existing context 512, append at 512, attend over 513, scale 1/8 (cpu_backend.cpp:111-117)
    rng = np.random.default_rng(512)
    Hq, Hkv, d, pos = 14, 2, 64, 512
    kv = Hkv * d
    kc = f16(rng, (pos + 1, kv))
    vc = f16(rng, (pos + 1, kv))
    q, k, v = f16(rng, Hq * d), f16(rng, kv), f16(rng, kv)
    qf, kf = q.astype(np.float32), k.astype(np.float32)
    ref.rope(qf, kf, d, Hq, Hkv, pos, 1e6, 1)
    kcf, vcf = kc.astype(np.float32), vc.astype(np.float32)
    kcf[pos], vcf[pos] = kf, v.astype(np.float32)
    o = ref.decode(qf, kcf, vcf, pos + 1, Hq, Hkv, d, threads=4)
    out.update(a_q=q.view(np.uint16), a_k=k.view(np.uint16), a_v=v.view(np.uint16), a_kcache=kc.view(np.uint16),
               a_vcache=vc.view(np.uint16), a_q_rot=qf, a_k_rot=kf, a_out=o,
               a_meta=np.array([Hq, Hkv, d, pos], np.int32))
    # --- case B: Llama-3 style interleaved RoPE with rope_freqs, 32q/8kv d128 at pos 4095
    rng = np.random.default_rng(4095)
    Hq, Hkv, d, pos = 32, 8, 128, 4095
    ff = rng.uniform(1.0, 8.0, d // 2).astype(np.float32)
    q, k = f16(rng, Hq * d, 3.0), f16(rng, Hkv * d, 3.0)
    qf, kf = q.astype(np.float32), k.astype(np.float32)
    ref.rope(qf, kf, d, Hq, Hkv, pos, 5e5, 0, ff)
    out.update(b_q=q.view(np.uint16), b_k=k.view(np.uint16), b_ff=ff, b_q_rot=qf, b_k_rot=kf,
               b_meta=np.array([Hq, Hkv, d, pos], np.int32))
    # --- case C: decode at the reference kernel-test shapes (40q/8kv d128, q = 2 N(0,1)) with a NaN
    # key row and a x30 outlier row, S = 120
    rng = np.random.default_rng(7)
    Hq, Hkv, d, S = 40, 8, 128, 120
    kc = f16(rng, (S, Hkv * d))
    kc[17] = np.float16(np.nan)
    kc[100] = (kc[100].astype(np.float32) * 30).astype(np.float16)
    vc = f16(rng, (S, Hkv * d))
    q = f16(rng, Hq * d, 2.0)
    o = ref.decode(q.astype(np.float32), kc.astype(np.float32), vc.astype(np.float32), S, Hq, Hkv, d, threads=4)
    out.update(c_q=q.view(np.uint16), c_kcache=kc.view(np.uint16), c_vcache=vc.view(np.uint16), c_out=o,
               c_meta=np.array([Hq, Hkv, d, S], np.int32))
    path = os.path.join(HERE, "golden_cpu_path.npz")
    np.savez_compressed(path, **out)
    print(path, os.path.getsize(path), "bytes")


if __name__ == "__main__":
    main()
