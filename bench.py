#!/usr/bin/env python3
"""Benchmark of the KV-cache path on one MI355X (BASELINE.json metric and configs).

A step is one decode token through all layers of the headline workload
(Qwen2.5-32B attention shapes, 40 query / 8 kv heads,
head_dim 128, fp16 KV, context 32768 after the append, 64 layers' caches
resident in HBM): per layer, RoPE + KV append at position S-1 followed by
split-K decode attention with the log-sum-exp merge. The 64-layer step is
captured once into a HIP graph (as the reference captures its decode layers
into a CUDA graph, transformer.cpp:1465-1483) and replayed.

Prints ONE JSON line. `value` is the K/V bytes the attention must read per
layer-step (2*S*Hkv*d*2) divided by the measured time per layer-step (append +
attention), in GB/s. The same line carries the per-layer-step time, the decode
kernel's roofline record (HIP events around every decode launch inside the
timed graph replays) and the reference CPU attention timed on this host.
"""
from __future__ import annotations

import argparse
import ctypes as C
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "friday-inference-engine_amd"))

METRIC = "decode-attn µs/layer-step + KV GB/s (% HBM peak) at 32k ctx, 40q/8kv d128"
HBM_PEAK_GBS = 8000.0


def log(msg):
    print(msg, file=sys.stderr, flush=True)


def cpu_baseline(S, Hq, Hkv, d, budget_s):
    """Reference CPU decode attention (cpu_ops.cpp:45-83) on a bounded sample."""
    import numpy as np

    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import py_oracle

    ncpu = os.cpu_count() or 1
    threads = max(1, min(16, ncpu, Hq))  # per-head parallelism; the box's CPU share is 16
    rng = np.random.default_rng(0)
    kv_dim = Hkv * d
    kc = rng.standard_normal((S, kv_dim), dtype=np.float32).astype(np.float16).astype(np.float32)
    vc = rng.standard_normal((S, kv_dim), dtype=np.float32).astype(np.float16).astype(np.float32)
    q = rng.standard_normal(Hq * d, dtype=np.float32).astype(np.float16).astype(np.float32)
    if py_oracle.ref_available():
        ref = py_oracle.RefCpu()
        kind = "reference"
        run = lambda: ref.decode(q, kc, vc, S, Hq, Hkv, d, threads=threads)
        what = "oracle/_ref: the reference's cpu_ops.cpp decodeAttention compiled from source"
    else:
        orc = py_oracle.Oracle()
        kind, threads = "port", 1
        qh, kh, vh = (a.astype(np.float16) for a in (q, kc, vc))
        run = lambda: orc.decode(qh, kh, vh, S, Hq, Hkv, d)
        what = "oracle/fa_oracle.c restatement of cpu_ops.cpp decodeAttention (single thread)"
    run()  # warm the pool and the pages
    n, t0 = 0, time.perf_counter()
    while True:
        run()
        n += 1
        el = time.perf_counter() - t0
        if el >= budget_s or n >= 200:
            break
    us = el / n * 1e6
    gbs = 2 * S * kv_dim * 4 / (us * 1e-6) / 1e9
    return {"value": round(us, 1), "unit": "us/layer-step", "cores": threads, "kind": kind,
            "kv_gbs_fp32": round(gbs, 2),
            "sample": f"{n} calls of one layer (ctx {S}, {Hq}q/{Hkv}kv d{d}, fp32 cache of fp16 values), "
                      f"{el:.1f} s; {what}; host logical CPUs {ncpu}"}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--ctx", type=int, default=32768)
    ap.add_argument("--layers", type=int, default=64)
    ap.add_argument("--heads", type=int, default=40)
    ap.add_argument("--kv-heads", type=int, default=8)
    ap.add_argument("--head-dim", type=int, default=128)
    ap.add_argument("--cpu-seconds", type=float, default=12.0)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-check", action="store_true")
    ap.add_argument("--merge", choices=("step", "fused", "kernel"), default="step",
                    help="step: RoPE+append+decode+merge in one launch per layer; fused: append launch + "
                         "decode with last-workgroup merge; kernel: append + decode + merge kernel")
    args = ap.parse_args()

    if args.gpus != 1:
        print(f"bench.py measures one GPU only (got --gpus {args.gpus}): the KV-cache path is built and "
              f"measured on a single MI355X; multi-GPU sharding is a design note, not a run.", file=sys.stderr)
        sys.exit(2)

    import numpy as np

    import friday_attn as fa

    lib = fa.load()
    bk = C.CDLL(os.path.join(ROOT, "friday-inference-engine_amd", "lib", "libfa_benchkit.so"))
    bk.fabk_fill_normal_f16.argtypes = [C.c_void_p, C.c_size_t, C.c_uint32, C.c_float, C.c_void_p]
    if fa.Hip.device_count() < 1:
        raise SystemExit("no HIP device")

    S, L, Hq, Hkv, d = args.ctx, args.layers, args.heads, args.kv_heads, args.head_dim
    kv_dim = Hkv * d
    layer_elems = S * kv_dim
    log(f"[bench] config3 S={S} layers={L} {Hq}q/{Hkv}kv d{d}: allocating "
        f"{2 * L * layer_elems * 2 / 2**30:.2f} GiB of KV cache")
    stream = fa.Stream()
    kcache = fa.DeviceBuffer(L * layer_elems * 2)
    vcache = fa.DeviceBuffer(L * layer_elems * 2)
    bk.fabk_fill_normal_f16(kcache.ptr, L * layer_elems, 1, 1.0, stream.s)
    bk.fabk_fill_normal_f16(vcache.ptr, L * layer_elems, 2, 1.0, stream.s)
    rng = np.random.default_rng(0)
    f16 = lambda shape: rng.standard_normal(shape, dtype=np.float32).astype(np.float16).view(np.uint16)
    qs = fa.DeviceBuffer.from_array(f16((L, Hq * d)))
    ks = fa.DeviceBuffer.from_array(f16((L, kv_dim)))
    vs = fa.DeviceBuffer.from_array(f16((L, kv_dim)))
    outs = fa.DeviceBuffer(L * Hq * d * 2)
    table = fa.DeviceBuffer(fa.rope_table_bytes(S, d))
    fa.rope_table_upload(table, S, d, 1e6)
    dpos = fa.DeviceBuffer.from_array(np.array([S - 1], np.int32))
    ws = fa.DeviceBuffer(fa.splitAttentionWorkspaceBytes(Hq, S))
    fa.decodeWorkspaceInit(ws, stream=stream.s)
    launch = fa.launchDecodeAttentionSplit if args.merge == "kernel" else fa.launchDecodeAttentionFused
    stream.synchronize()

    def step():
        for l in range(L):
            kl = kcache.ptr + l * layer_elems * 2
            vl = vcache.ptr + l * layer_elems * 2
            ql = qs.ptr + l * Hq * d * 2
            if args.merge == "step":
                fa.decodeStep(ql, ks.ptr + l * kv_dim * 2, vs.ptr + l * kv_dim * 2, kl, vl, outs.ptr + l * Hq * d * 2,
                              dpos, 0, S, Hq, Hkv, d, table, 1, ws, stream.s)
                continue
            fa.ropeStoreKv(ql, ks.ptr + l * kv_dim * 2, vs.ptr + l * kv_dim * 2, kl, vl, dpos, 0, 1, d, Hq, Hkv,
                           S, table, 1, stream.s)
            decode(l)

    def decode(l):
        kl = kcache.ptr + l * layer_elems * 2
        vl = vcache.ptr + l * layer_elems * 2
        ql = qs.ptr + l * Hq * d * 2
        launch(ql, kl, vl, outs.ptr + l * Hq * d * 2, 0, dpos, S, Hq, Hkv, d, ws, stream.s)

    def timed(graph, steps, warmup):
        for _ in range(warmup):
            graph.launch()
        stream.synchronize()
        t_start, t_end = fa.Event(), fa.Event()
        w0 = time.perf_counter()
        t_start.record(stream.s)
        for _ in range(steps):
            graph.launch()
        t_end.record(stream.s)
        stream.synchronize()
        return t_start.elapsed_ms(t_end) / steps, time.perf_counter() - w0

    # timed region 1: the whole step (append + attention, all layers)
    ms_step, wall = timed(fa.Graph(stream, step), args.steps, args.warmup)
    # timed region 2: the dominant kernel alone (decode attention of all layers, back to back)
    ms_dec, _ = timed(fa.Graph(stream, lambda: [decode(l) for l in range(L)]), args.steps, args.warmup)
    dec_mean = ms_dec * 1e3 / L

    us_layer = ms_step * 1e3 / L
    kv_bytes = 2 * S * kv_dim * 2
    kv_gbs = kv_bytes / (us_layer * 1e-6) / 1e9
    ach = kv_bytes / (dec_mean * 1e-6) / 1e9
    log(f"[bench] merge={args.merge} min_chunk={os.environ.get('FRIDAY_ATTN_MIN_CHUNK', 'default')} "
        f"max_splits={os.environ.get('FRIDAY_ATTN_MAX_SPLITS', 'default')}")
    log(f"[bench] {ms_step:.3f} ms/step, {us_layer:.2f} us/layer-step, decode call {dec_mean:.2f} us, "
        f"wall {wall:.2f} s")

    check = None
    if not args.no_check:
        sys.path.insert(0, os.path.join(ROOT, "oracle"))
        from py_oracle import Oracle

        q0 = qs.download(Hq * d, np.uint16)
        k0 = kcache.download((S, kv_dim), np.uint16)
        v0 = vcache.download((S, kv_dim), np.uint16)
        got = outs.download(Hq * d, np.uint16).view(np.float16).astype(np.float32)
        ref = Oracle().decode(q0, k0, v0, S, Hq, Hkv, d)
        err = np.abs(got - ref)
        ok = bool(np.all(err <= 2e-3 + 1e-2 * np.abs(ref)))
        check = {"layer0_vs_oracle_max_abs": float(err.max()), "pass": ok}
        log(f"[bench] layer 0 vs oracle: max_abs {err.max():.2e} {'PASS' if ok else 'FAIL'}")

    cpu = None
    if not args.no_cpu:
        log("[bench] timing the reference CPU attention ...")
        cpu = cpu_baseline(S, Hq, Hkv, d, args.cpu_seconds)

    rec = {
        "metric": METRIC,
        "value": round(kv_gbs, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp16",
        "data": "synthetic: device-generated N(0,1) fp16 K/V caches, seeded N(0,1) q/k/v",
        "config": {"workload": f"BASELINE config 3: decode step (RoPE+KV append, split-K GQA attention + LSE merge) "
                               f"over {L} layers, ctx {S} after append, {Hq}q/{Hkv}kv d{d}, fp16 KV, batch 1, "
                               f"HIP graph replay",
                   "layers": L, "ctx": S, "num_heads": Hq, "num_kv_heads": Hkv, "head_dim": d},
        "us_per_layer_step": round(us_layer, 3),
        "hbm_frac_step": round(kv_gbs / HBM_PEAK_GBS, 4),
        "tokens_per_s": round(1e3 / ms_step, 2),
        "decode_call_us": round(dec_mean, 3),
        "roofline": {"bound": "hbm", "kernel": ("fa_decode_kernel + fa_merge_kernel (friday_attn_decode_attention_split)"
                                if args.merge == "kernel" else
                                "fa_decode_kernel (friday_attn_decode_attention_fused, last-workgroup merge)"),
                     "achieved": round(ach, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(ach / HBM_PEAK_GBS, 4), "traffic": None,
                     "algorithmic_bytes_per_launch": kv_bytes},
        "cpu_baseline": cpu,
        "check": check,
    }
    print(json.dumps(rec), flush=True)


if __name__ == "__main__":
    main()
