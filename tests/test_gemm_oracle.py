"""CPU tests pinning the prefill-GEMM oracle (oracle/gemm_oracle.c).

What pins it (none of these restate the oracle's own formulas):
  * golden vectors written from the reference's own cpu_kquants.cpp
    (tests/golden/golden_kquant.npz): quantizeActivation and dequantizeRow bit-exact,
    gemvRowsScalar within fp32 summation-order rounding;
  * the live reference build in oracle/_ref, when present, on fresh seeds;
  * an fp64 product of the dequantised operands (the sums are exact integers times
    scales, so only fp32 rounding separates them);
  * closed forms of the epilogue (storeY, prefill_kernels.cu:155-171): NaN -> 0,
    +-65504 clamp, residual added after the bias, in fp16.
"""
import os

import numpy as np
import pytest

from fa_helpers import KQ_KINDS, kq_random_weights

HERE = os.path.dirname(os.path.abspath(__file__))
GOLD = np.load(os.path.join(HERE, "golden", "golden_kquant.npz"))


def _ref():
    from py_oracle import RefCpu, ref_available
    if not ref_available():
        pytest.skip("oracle/_ref not built (needs /root/reference at build time)")
    return RefCpu()


@pytest.mark.parametrize("kind", sorted(KQ_KINDS))
def test_golden_quantize_dequant_gemv(oracle, kind):
    W, x = GOLD[f"k{kind}_w"], GOLD[f"k{kind}_x"]
    T, K = x.shape
    N = W.shape[0]
    xq, xd = oracle.quantize_q8_rows(x)
    assert np.array_equal(xq, GOLD[f"k{kind}_xq"])
    assert np.array_equal(xd.view(np.uint32), GOLD[f"k{kind}_xd"].view(np.uint32))
    deq = np.stack([oracle.dequant_row(kind, W[n], K) for n in range(N)])
    assert np.array_equal(deq.view(np.uint32), GOLD[f"k{kind}_deq"].view(np.uint32))
    _, raw = oracle.gemm_q8(kind, W, xq, xd, T, K, N)
    y = GOLD[f"k{kind}_y"]
    scale = np.sqrt(np.mean(y.astype(np.float64) ** 2))
    assert np.max(np.abs(raw - y)) <= 1e-5 * scale


@pytest.mark.parametrize("kind", sorted(KQ_KINDS))
def test_vs_reference_build(oracle, kind):
    ref = _ref()
    name = KQ_KINDS[kind][0]
    rng = np.random.default_rng(99 + kind)
    K, N = 768, 24
    W = kq_random_weights(rng, kind, N, K)
    x = (rng.standard_normal(K, dtype=np.float32) * 3).astype(np.float16)
    x[64:96] = 0
    x[200] = np.float16(60000.0)  # a block whose amax dwarfs the rest
    q, d = ref.quantize_activation(x.astype(np.float32))
    xq, xd = oracle.quantize_q8_rows(x.view(np.uint16)[None])
    assert np.array_equal(xq[0], q) and np.array_equal(xd[0].view(np.uint32), d.view(np.uint32))
    for n in range(0, N, 5):
        assert np.array_equal(oracle.dequant_row(kind, W[n], K).view(np.uint32),
                              ref.dequantize_row(name, W[n], K).view(np.uint32))
    _, raw = oracle.gemm_q8(kind, W, xq, xd, 1, K, N)
    y = ref.gemv_rows_scalar(name, W, x.astype(np.float32), K, N)
    assert np.max(np.abs(raw[0] - y)) <= 1e-5 * np.sqrt(np.mean(y.astype(np.float64) ** 2))


@pytest.mark.parametrize("kind", sorted(KQ_KINDS))
def test_gemm_vs_fp64_dequant_product(oracle, kind):
    rng = np.random.default_rng(7 * kind)
    T, K, N = 5, 512, 12
    W = kq_random_weights(rng, kind, N, K)
    x = (rng.standard_normal((T, K), dtype=np.float32)).astype(np.float16)
    xq, xd = oracle.quantize_q8_rows(x.view(np.uint16))
    _, raw = oracle.gemm_q8(kind, W, xq, xd, T, K, N)
    # exact weights in fp64 from the block integers (not from the fp32 dequant formula)
    wt = np.zeros((N, K))
    for n in range(N):
        for b in range(K // 32):
            q, ws, wm = oracle.kq_block(kind, W[n], b)
            half = np.arange(32) // 16
            wt[n, 32 * b:32 * b + 32] = ws.astype(np.float64)[half] * q - wm.astype(np.float64)[half]
    xa = xq.astype(np.float64) * np.repeat(xd.astype(np.float64), 32, axis=1)
    exact = xa @ wt.T
    assert np.max(np.abs(raw - exact)) <= 1e-5 * np.sqrt(np.mean(exact ** 2))


def test_quantize_closed_forms(oracle):
    x = np.zeros((1, 64), np.float16)
    x[0, :32] = np.linspace(-3, 3, 32)
    xq, xd = oracle.quantize_q8_rows(x.view(np.uint16))
    assert xd[0, 1] == 0 and not xq[0, 32:].any()          # zero block: d = 0, q = 0
    assert xq[0, 0] == -127 and xq[0, 31] == 127             # the amax elements map to -+127
    assert np.float32(xd[0, 0]) == np.float32(3.0) / np.float32(127.0)
    # q = rne(x / d): |x - q d| <= d / 2
    err = np.abs(x[0, :32].astype(np.float32) - xq[0, :32] * xd[0, 0])
    assert np.all(err <= xd[0, 0] / 2 * (1 + 1e-6))


def test_epilogue_closed_forms(oracle):
    kind, T, K, N = 6, 2, 256, 4
    rng = np.random.default_rng(5)
    W = kq_random_weights(rng, kind, N, K)
    x = rng.standard_normal((T, K), dtype=np.float32).astype(np.float16)
    xq, xd = oracle.quantize_q8_rows(x.view(np.uint16))
    Y0, raw = oracle.gemm_q8(kind, W, xq, xd, T, K, N)
    h = lambda v: np.float32(v).astype(np.float16)  # noqa: E731
    assert np.array_equal(Y0, raw.astype(np.float16).view(np.uint16))     # plain: fp16 rounding
    bias = np.array([0.5, np.nan, 1e6, -1e6], np.float32)
    res = np.zeros((T, N), np.float16)
    res[:, 0] = np.float16(np.nan)
    res[:, 1] = np.float16(2.0)
    Y, _ = oracle.gemm_q8(kind, W, xq, xd, T, K, N, bias=bias, res=res.view(np.uint16))
    yf = Y.view(np.float16).astype(np.float32)
    for t in range(T):
        y0 = np.float32(h(raw[t, 0]))
        assert yf[t, 0] == np.float32(h(np.float32(h(y0 + np.float32(0.5)))))  # NaN residual counts 0
        assert yf[t, 1] == np.float32(h(np.float32(h(raw[t, 1])) + np.float32(2.0)))  # NaN bias counts 0
        assert yf[t, 2] == 65504.0 and yf[t, 3] == -65504.0                  # clamped to the fp16 range
