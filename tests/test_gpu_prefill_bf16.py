"""GPU parity of the bf16 causal prefill (friday_attn_prefill_attention_bf16).

No counterpart in the reference (its caches are fp16); the oracle is the same causal
decode restatement with bf16 inputs widened exactly and the output rounded to bf16
(or_prefill_attention_bf16), itself pinned against the fp16 path and float64 in
tests/test_oracle.py.

Tolerance (bf16 mode): |got - ref| <= 4e-3 + 2^-6 |ref| elementwise and rel-L2 < 5e-3.
The fp16 bar (2e-3 abs) is below one bf16 step at |x| >= 0.5 (2^-8 relative), so it
cannot hold for bf16 outputs. The budget: the two sides may round the output one bf16
step apart (<= 2^-7 relative), and the kernel's PV weights are rounded to bf16
(relative error <= 2^-9 each, normalised by the sum of the same rounded weights).
"""
import numpy as np
import pytest

from fa_helpers import assert_close, bf16, bf16_as_f32

pytestmark = pytest.mark.gpu

BF_ATOL = 4e-3
BF_RTOL = 2.0**-6
BF_REL_L2 = 5e-3
NAN_BF16 = np.uint16(0x7FC0)


def close(got, ref, what):
    return assert_close(got, ref, what, atol=BF_ATOL, rtol=BF_RTOL, rel_l2=BF_REL_L2)


def run_bf16(fa, q, k, v, T, p0, Hq, Hkv, d):
    dq, dk, dv = (fa.DeviceBuffer.from_array(a) for a in (q, k, v))
    out = fa.DeviceBuffer(q.nbytes)
    out.fill_bytes(0xFF)
    dpos = fa.DeviceBuffer.from_array(np.array([p0], np.int32))
    fa.launchPrefillAttentionBf16(dq, dk, dv, out, T, dpos, Hq, Hkv, d)
    fa.Hip.sync()
    return bf16_as_f32(out.download((T, Hq * d), np.uint16))


def cache(rng, rows, kv_dim):
    return bf16(rng, (rows, kv_dim)), bf16(rng, (rows, kv_dim))


@pytest.mark.parametrize("Hq,Hkv,d,T,p0", [(32, 8, 128, 1, 0), (32, 8, 128, 13, 0), (32, 8, 128, 70, 100),
                                           (16, 16, 128, 9, 31), (14, 2, 64, 40, 0), (14, 2, 64, 129, 300),
                                           (48, 1, 128, 33, 10), (40, 8, 128, 300, 700)])
def test_shapes(gpu, oracle, Hq, Hkv, d, T, p0):
    """Every row vs the bf16 oracle; the cache ends at p0 + T (the last stage's copies stop there)."""
    fa = gpu
    rng = np.random.default_rng(5000 + T * 7 + p0)
    q = bf16(rng, (T, Hq * d))
    k, v = cache(rng, p0 + T, Hkv * d)
    got = run_bf16(fa, q, k, v, T, p0, Hq, Hkv, d)
    mx, rel = close(got, oracle.prefill_bf16(q, k, v, T, p0, Hq, Hkv, d), f"bf16 {Hq}/{Hkv} d{d} T={T} p0={p0}")
    print(f"bf16 prefill {Hq}/{Hkv} d{d} T={T} p0={p0}: max_abs {mx:.3e} rel_l2 {rel:.3e}")


@pytest.mark.parametrize("p0", [0, 1024, 2048, 4096, 7680])  # every p0 bench.py measures
def test_config4_chunk(gpu, oracle, p0):
    """Config 4 shapes (40q/8kv d128, 512-token chunk) in bf16: all 512 rows vs the oracle."""
    fa = gpu
    Hq, Hkv, d, T = 40, 8, 128, 512
    rng = np.random.default_rng(p0 + 40)
    q = bf16(rng, (T, Hq * d))
    k, v = cache(rng, p0 + T, Hkv * d)
    got = run_bf16(fa, q, k, v, T, p0, Hq, Hkv, d)
    ref = oracle.prefill_all(q, k, v, T, p0, Hq, Hkv, d, bf16=True)
    mx, rel = close(got, ref, f"bf16 config4 p0={p0}, all {T} rows")
    print(f"bf16 config4 p0={p0}: {T} rows, max_abs {mx:.3e} rel_l2 {rel:.3e}")


def test_long_prefix(gpu, oracle):
    """A ragged chunk after a 60k-token prefix: sampled rows vs the oracle."""
    fa = gpu
    Hq, Hkv, d, T, p0 = 10, 2, 128, 77, 60000
    rng = np.random.default_rng(61)
    q = bf16(rng, (T, Hq * d))
    k, v = cache(rng, p0 + T, Hkv * d)
    got = run_bf16(fa, q, k, v, T, p0, Hq, Hkv, d)
    for t in (0, 1, 15, 16, 76):
        close(got[t], oracle.prefill_bf16(q[t:t + 1], k, v, 1, p0 + t, Hq, Hkv, d)[0], f"bf16 long t={t}")


def test_single_token_is_v0(gpu):
    """T = 1, p0 = 0: the only key is position 0 -> out = v0 bit for bit (weight 1 exactly)."""
    fa = gpu
    Hq, Hkv, d = 32, 8, 128
    rng = np.random.default_rng(62)
    q = bf16(rng, (1, Hq * d))
    k, v = cache(rng, 4, Hkv * d)
    got = run_bf16(fa, q, k, v, 1, 0, Hq, Hkv, d)
    exp = np.concatenate([bf16_as_f32(v[0, (h // 4) * d:(h // 4 + 1) * d]) for h in range(Hq)])
    assert np.array_equal(got[0], exp)


def test_wide_range_values(gpu, oracle):
    """bf16 keeps the fp32 exponent range: q and V of magnitude 1e4 and 1e-4 (outside
    or below fp16's normal range) give finite outputs on the oracle's scale."""
    fa = gpu
    Hq, Hkv, d, T, p0 = 16, 4, 128, 40, 90
    rng = np.random.default_rng(63)
    q = bf16(rng, (T, Hq * d), 0.05)
    k = bf16(rng, (p0 + T, Hkv * d))
    v = bf16(rng, (p0 + T, Hkv * d), 1e4)
    got = run_bf16(fa, q, k, v, T, p0, Hq, Hkv, d)
    ref = oracle.prefill_bf16(q, k, v, T, p0, Hq, Hkv, d)
    assert_close(got / 1e4, ref / 1e4, "bf16 V x 1e4", atol=BF_ATOL, rtol=BF_RTOL, rel_l2=BF_REL_L2)
    v = bf16(rng, (p0 + T, Hkv * d), 1e-4)
    got = run_bf16(fa, q, k, v, T, p0, Hq, Hkv, d)
    ref = oracle.prefill_bf16(q, k, v, T, p0, Hq, Hkv, d)
    assert_close(got * 1e4, ref * 1e4, "bf16 V x 1e-4", atol=BF_ATOL, rtol=BF_RTOL, rel_l2=BF_REL_L2)


def test_causal_invariance(gpu):
    """Rows after a query's position must not influence it (bit-identical output)."""
    fa = gpu
    Hq, Hkv, d, T, p0 = 40, 8, 128, 64, 50
    rng = np.random.default_rng(64)
    q = bf16(rng, (T, Hq * d))
    k, v = cache(rng, p0 + T, Hkv * d)
    a = run_bf16(fa, q, k, v, T, p0, Hq, Hkv, d)
    k2, v2 = k.copy(), v.copy()
    k2[p0 + 20:] = bf16(rng, k2[p0 + 20:].shape, 5.0)
    v2[p0 + 20:] = bf16(rng, v2[p0 + 20:].shape, 5.0)
    b = run_bf16(fa, q, k2, v2, T, p0, Hq, Hkv, d)
    assert np.array_equal(a[:20], b[:20])
    assert not np.array_equal(a[21:], b[21:])


@pytest.mark.parametrize("d", [128, 64])
def test_nan_scores(gpu, oracle, d):
    """NaN rule as in the fp16 path: a NaN K row is excluded; a token whose q is all NaN
    weighs its visible keys uniformly; outputs stay finite."""
    fa = gpu
    Hq, Hkv, T, p0 = 40, 8, 300, 200
    rng = np.random.default_rng(65 + d)
    q = bf16(rng, (T, Hq * d))
    k, v = cache(rng, p0 + T, Hkv * d)
    k[50, :] = NAN_BF16
    k[p0 + 10, :] = NAN_BF16
    for t in (0, 3, 130, 299):
        q[t, :] = NAN_BF16
    got = run_bf16(fa, q, k, v, T, p0, Hq, Hkv, d)
    assert np.isfinite(got).all()
    close(got, oracle.prefill_bf16(q, k, v, T, p0, Hq, Hkv, d), f"bf16 NaN d{d}")


def test_fp16_entry_unchanged_by_bf16_calls(gpu, oracle):
    """The two element types share the kernel source: interleaved calls keep the fp16
    entry's results identical."""
    from fa_helpers import as_f32, f16
    fa = gpu
    Hq, Hkv, d, T, p0 = 32, 8, 128, 70, 100
    rng = np.random.default_rng(66)
    q16, k16, v16 = f16(rng, (T, Hq * d)), f16(rng, (p0 + T, Hkv * d)), f16(rng, (p0 + T, Hkv * d))
    qb, kb = bf16(rng, (T, Hq * d)), bf16(rng, (p0 + T, Hkv * d))
    vb = bf16(rng, (p0 + T, Hkv * d))

    def fp16_call():
        dq, dk, dv = (fa.DeviceBuffer.from_array(a) for a in (q16, k16, v16))
        out = fa.DeviceBuffer(q16.nbytes)
        dpos = fa.DeviceBuffer.from_array(np.array([p0], np.int32))
        fa.launchPrefillAttention(dq, dk, dv, out, T, dpos, Hq, Hkv, d)
        fa.Hip.sync()
        return as_f32(out.download((T, Hq * d), np.uint16))

    a = fp16_call()
    run_bf16(fa, qb, kb, vb, T, p0, Hq, Hkv, d)
    assert np.array_equal(a, fp16_call())
    assert_close(a, oracle.prefill(q16, k16, v16, T, p0, Hq, Hkv, d), "fp16 after bf16")
