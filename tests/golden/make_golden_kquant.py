"""Writes tests/golden/golden_kquant.npz from the reference's own CPU K-quant path.

Runs in the build container only (needs oracle/_ref, built by `make -C oracle ref` from the
reference's cpu_kquants.cpp). For every weight kind: random rows as the reference GEMM test
makes them, two fp16 activation rows, and the reference's quantizeActivation (q, d),
dequantizeRow and gemvRowsScalar outputs (cpu_kquants.cpp:75-139, 227-280, 437-455). Data only.

    python tests/golden/make_golden_kquant.py
"""
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(HERE, "..", "..", "oracle"))
sys.path.insert(0, os.path.join(HERE, ".."))
from py_oracle import RefCpu  # noqa: E402
from fa_helpers import KQ_KINDS, kq_random_weights  # noqa: E402


def main():
    ref = RefCpu()
    out = {}
    K, N, T = 512, 8, 2
    for kind, (name, _, _, _) in KQ_KINDS.items():
        rng = np.random.default_rng(20261110 + kind)
        W = kq_random_weights(rng, kind, N, K)
        x = (rng.standard_normal((T, K), dtype=np.float32) * 2).astype(np.float16)
        x[1, :32] = 0  # an all-zero block: d = 0, q = 0
        deq = np.stack([ref.dequantize_row(name, W[n], K) for n in range(N)])
        qs, ds, ys = [], [], []
        for t in range(T):
            q, d = ref.quantize_activation(x[t].astype(np.float32))
            qs.append(q)
            ds.append(d)
            ys.append(ref.gemv_rows_scalar(name, W, x[t].astype(np.float32), K, N))
        out[f"k{kind}_w"] = W
        out[f"k{kind}_x"] = x.view(np.uint16)
        out[f"k{kind}_xq"] = np.stack(qs)
        out[f"k{kind}_xd"] = np.stack(ds)
        out[f"k{kind}_deq"] = deq
        out[f"k{kind}_y"] = np.stack(ys)
    np.savez_compressed(os.path.join(HERE, "golden_kquant.npz"), **out)
    print("wrote", os.path.join(HERE, "golden_kquant.npz"))


if __name__ == "__main__":
    main()
