"""GPU parity of causal prefill attention (launchPrefillAttention semantics) on MFMA.

Mirrors tests/kernels/test_prefill_attention.cu: the same (nh, nkv, T, p0, int8)
cases with max_ctx 1024; row t must equal decode attention at S = p0 + t + 1
(the oracle computes exactly that, in the reference CPU order). Adds benchmark
config 4 (40q/8kv, T = 512, p0 up to 7680) on sampled rows and the causal
invariance: K/V rows after a query's position do not change its output.
"""
import numpy as np
import pytest

from fa_helpers import as_f32, assert_close, f16

pytestmark = pytest.mark.gpu

REF_CASES = [(32, 8, 1, 0, False), (32, 8, 13, 0, False), (32, 8, 70, 100, False), (40, 8, 37, 5, True),
             (32, 8, 70, 300, True), (16, 16, 9, 31, False), (64, 8, 20, 64, True)]


def make_cache(rng, max_ctx, kv_dim, q8):
    if q8:
        k8 = rng.integers(-127, 128, (max_ctx, kv_dim), dtype=np.int8)
        v8 = rng.integers(-127, 128, (max_ctx, kv_dim), dtype=np.int8)
        ks = rng.uniform(0.005, 0.03, (max_ctx, kv_dim // 32)).astype(np.float16).view(np.uint16)
        vs = rng.uniform(0.005, 0.03, (max_ctx, kv_dim // 32)).astype(np.float16).view(np.uint16)
        return k8, v8, ks, vs
    return f16(rng, (max_ctx, kv_dim)), f16(rng, (max_ctx, kv_dim)), None, None


def run_prefill(fa, q, k, v, ks, vs, T, p0, Hq, Hkv, d):
    dq = fa.DeviceBuffer.from_array(q)
    dk, dv = fa.DeviceBuffer.from_array(k), fa.DeviceBuffer.from_array(v)
    dks = fa.DeviceBuffer.from_array(ks) if ks is not None else None
    dvs = fa.DeviceBuffer.from_array(vs) if vs is not None else None
    out = fa.DeviceBuffer(q.nbytes)
    out.fill_bytes(0xFF)
    dpos = fa.DeviceBuffer.from_array(np.array([p0], np.int32))
    fa.launchPrefillAttention(dq, dk, dv, out, T, dpos, Hq, Hkv, d, k_scale=dks, v_scale=dvs)
    fa.Hip.sync()
    return as_f32(out.download((T, Hq * d), np.uint16))


@pytest.mark.parametrize("Hq,Hkv,T,p0,q8", REF_CASES)
def test_reference_prefill_cases(gpu, oracle, Hq, Hkv, T, p0, q8):
    fa = gpu
    d, max_ctx = 128, 1024
    rng = np.random.default_rng(20261110 + T + p0)
    q = f16(rng, (T, Hq * d))
    k, v, ks, vs = make_cache(rng, max_ctx, Hkv * d, q8)
    got = run_prefill(fa, q, k, v, ks, vs, T, p0, Hq, Hkv, d)
    ref = oracle.prefill_q8(q, k, ks, v, vs, T, p0, Hq, Hkv, d) if q8 else oracle.prefill(q, k, v, T, p0, Hq, Hkv, d)
    assert_close(got, ref, f"prefill {Hq}/{Hkv} T={T} p0={p0} q8={q8}")


@pytest.mark.parametrize("q8", [False, True])
@pytest.mark.parametrize("Hq,Hkv,d,T,p0", [(14, 2, 64, 40, 0), (14, 2, 64, 129, 300), (48, 1, 128, 33, 10)])
def test_other_shapes(gpu, oracle, Hq, Hkv, d, T, p0, q8):
    """The cache ends at p0 + T: the last stage's copies stop at its last row."""
    fa = gpu
    rng = np.random.default_rng(T * 7 + p0)
    max_ctx = p0 + T
    q = f16(rng, (T, Hq * d))
    k, v, ks, vs = make_cache(rng, max_ctx, Hkv * d, q8)
    got = run_prefill(fa, q, k, v, ks, vs, T, p0, Hq, Hkv, d)
    ref = oracle.prefill_q8(q, k, ks, v, vs, T, p0, Hq, Hkv, d) if q8 else oracle.prefill(q, k, v, T, p0, Hq, Hkv, d)
    assert_close(got, ref, f"prefill {Hq}/{Hkv} d{d} T={T} p0={p0} q8={q8}")


@pytest.mark.parametrize("p0", [0, 1024, 2048, 7680])
def test_config4_chunk_q8(gpu, oracle, p0):
    """Config 4 on an int8 cache: all 512 rows vs the int8 oracle prefill (prefill_all, bit-identical to
    or_prefill_attention_q8; row t = the int8
    decode at S = p0 + t + 1)."""
    fa = gpu
    Hq, Hkv, d, T = 40, 8, 128, 512
    rng = np.random.default_rng(p0 + 8)
    q = f16(rng, (T, Hq * d))
    k, v, ks, vs = make_cache(rng, p0 + T, Hkv * d, True)
    got = run_prefill(fa, q, k, v, ks, vs, T, p0, Hq, Hkv, d)
    ref = oracle.prefill_all(q, k, v, T, p0, Hq, Hkv, d, ks=ks, vs=vs)
    mx, rel = assert_close(got, ref, f"config4 q8 p0={p0}, all {T} rows")
    print(f"config4 q8 p0={p0}: {T} rows, max_abs {mx:.3e} rel_l2 {rel:.3e}")


def test_q8_scales_off_dword_alignment(gpu, oracle):
    """Scale arrays 2 bytes off 4-byte alignment (the scales are read as 2-byte values): same results."""
    fa = gpu
    Hq, Hkv, d, T, p0 = 32, 8, 128, 70, 300
    rng = np.random.default_rng(17)
    q = f16(rng, (T, Hq * d))
    k, v, ks, vs = make_cache(rng, p0 + T, Hkv * d, True)
    dq, dk, dv = (fa.DeviceBuffer.from_array(a) for a in (q, k, v))
    dks, dvs = fa.DeviceBuffer(ks.nbytes + 4), fa.DeviceBuffer(vs.nbytes + 4)
    dks.upload(ks, offset=2)
    dvs.upload(vs, offset=2)
    out = fa.DeviceBuffer(q.nbytes)
    dpos = fa.DeviceBuffer.from_array(np.array([p0], np.int32))
    fa.launchPrefillAttention(dq, dk, dv, out, T, dpos, Hq, Hkv, d, k_scale=dks.ptr + 2, v_scale=dvs.ptr + 2)
    fa.Hip.sync()
    got = as_f32(out.download((T, Hq * d), np.uint16))
    assert_close(got, oracle.prefill_q8(q, k, ks, v, vs, T, p0, Hq, Hkv, d), "prefill q8 misaligned scales")


@pytest.mark.parametrize("p0", [0, 1024, 2048, 4096, 7680])  # every p0 bench.py measures
def test_config4_chunk(gpu, oracle, p0):
    """benchmark config 4: 40q/8kv d128, 512-token chunk after p0 cached tokens; all 512 rows
    vs the oracle prefill (prefill_all, bit-identical to or_prefill_attention: row t = the decode at S = p0 + t + 1)."""
    fa = gpu
    Hq, Hkv, d, T = 40, 8, 128, 512
    rng = np.random.default_rng(p0 + 4)
    q = f16(rng, (T, Hq * d))
    k, v, _, _ = make_cache(rng, p0 + T, Hkv * d, False)
    got = run_prefill(fa, q, k, v, None, None, T, p0, Hq, Hkv, d)
    ref = oracle.prefill_all(q, k, v, T, p0, Hq, Hkv, d)
    mx, rel = assert_close(got, ref, f"config4 p0={p0}, all {T} rows")
    print(f"config4 p0={p0}: {T} rows, max_abs {mx:.3e} rel_l2 {rel:.3e}")


# T for each row-tile share the launcher picks at 32q/8kv (ceil(T * 4 * 8 / 4096) tiles per
# workgroup): (1,0), (1,1), (2,1), (2,2), (3,2), (3,3)
SHARE_T = [100, 200, 300, 500, 600, 700]


@pytest.mark.parametrize("q8", [False, True])
@pytest.mark.parametrize("T", SHARE_T)
def test_every_row_share(gpu, oracle, T, q8):
    """Every row-tile share of the workgroup (which sets how the waves split the stage copies,
    including a group without rows) on a ragged prefix; sampled rows vs the decode oracle."""
    fa = gpu
    Hq, Hkv, d, p0 = 32, 8, 128, 37
    rng = np.random.default_rng(900 + T + q8)
    q = f16(rng, (T, Hq * d))
    k, v, ks, vs = make_cache(rng, p0 + T, Hkv * d, q8)
    got = run_prefill(fa, q, k, v, ks, vs, T, p0, Hq, Hkv, d)
    for t in sorted(set([0, 1, 90, T // 2, T - 2, T - 1] + list(rng.choice(T, 4, replace=False)))):
        S = p0 + t + 1
        ref = oracle.decode_q8(q[t], k, ks, v, vs, S, Hq, Hkv, d) if q8 else oracle.decode(q[t], k, v, S, Hq, Hkv, d)
        assert_close(got[t], ref, f"share T={T} q8={q8} t={t}")


@pytest.mark.parametrize("Hq,Hkv,d,T,p0,q8", [(10, 2, 128, 77, 100000, False), (10, 2, 128, 77, 60000, True),
                                               (14, 2, 64, 200, 30000, False),
                                               (10, 2, 128, 2048, 100, False), (10, 2, 128, 2047, 9, True)])
def test_long_prefix(gpu, oracle, Hq, Hkv, d, T, p0, q8):
    """A ragged chunk after a long cached prefix (up to 100k positions), and chunks of about
    2k tokens: sampled rows vs the decode oracle at S = p0 + t + 1."""
    fa = gpu
    rng = np.random.default_rng(p0 + T)
    q = f16(rng, (T, Hq * d))
    k, v, ks, vs = make_cache(rng, p0 + T, Hkv * d, q8)
    got = run_prefill(fa, q, k, v, ks, vs, T, p0, Hq, Hkv, d)
    for t in sorted(set([0, 1, 15, 16, T - 1] + list(rng.choice(T, 3, replace=False)))):
        S = p0 + t + 1
        ref = oracle.decode_q8(q[t], k, ks, v, vs, S, Hq, Hkv, d) if q8 else oracle.decode(q[t], k, v, S, Hq, Hkv, d)
        assert_close(got[t], ref, f"long prefix p0={p0} t={t} q8={q8}")


def test_causal_invariance(gpu):
    """Rows after a query's position must not influence it (bit-identical output)."""
    fa = gpu
    Hq, Hkv, d, T, p0 = 40, 8, 128, 64, 50
    rng = np.random.default_rng(12)
    q = f16(rng, (T, Hq * d))
    k, v, _, _ = make_cache(rng, p0 + T, Hkv * d, False)
    a = run_prefill(fa, q, k, v, None, None, T, p0, Hq, Hkv, d)
    k2, v2 = k.copy(), v.copy()
    k2[p0 + 20:] = f16(rng, k2[p0 + 20:].shape, 5.0)
    v2[p0 + 20:] = f16(rng, v2[p0 + 20:].shape, 5.0)
    b = run_prefill(fa, q, k2, v2, None, None, T, p0, Hq, Hkv, d)
    assert np.array_equal(a[:20], b[:20])
    assert not np.array_equal(a[21:], b[21:])


def test_single_token_first_position(gpu):
    """T = 1, p0 = 0: the only key is position 0 -> out = v0 exactly."""
    fa = gpu
    Hq, Hkv, d = 32, 8, 128
    rng = np.random.default_rng(13)
    q = f16(rng, (1, Hq * d))
    k, v, _, _ = make_cache(rng, 4, Hkv * d, False)
    got = run_prefill(fa, q, k, v, None, None, 1, 0, Hq, Hkv, d)
    exp = np.concatenate([as_f32(v[0, (h // 4) * d:(h // 4 + 1) * d]) for h in range(Hq)])
    assert np.array_equal(got[0], exp)


@pytest.mark.parametrize("d,q8", [(128, False), (64, False), (128, True)])
def test_nan_scores(gpu, oracle, d, q8):
    """A NaN score becomes -1e30 (attention.cu NaN rule, as in decode): a NaN K row is
    excluded, and a token whose q is all NaN sees every score at -1e30 -> uniform weights
    over its visible keys (mean of V). Several stages, NaN rows before and inside the chunk."""
    fa = gpu
    Hq, Hkv, T, p0 = 40, 8, 300, 200
    rng = np.random.default_rng(77 + d)
    q = f16(rng, (T, Hq * d))
    k, v, ks, vs = make_cache(rng, p0 + T, Hkv * d, q8)
    nan16 = np.float16(np.nan).view(np.uint16)
    if not q8:
        k[50, :] = nan16
        k[p0 + 10, :] = nan16
    for t in (0, 3, 130, 299):
        q[t, :] = nan16
    got = run_prefill(fa, q, k, v, ks, vs, T, p0, Hq, Hkv, d)
    ref = oracle.prefill_q8(q, k, ks, v, vs, T, p0, Hq, Hkv, d) if q8 else oracle.prefill(q, k, v, T, p0, Hq, Hkv, d)
    assert np.isfinite(got).all()
    assert_close(got, ref, f"prefill NaN d{d} q8={q8}")
