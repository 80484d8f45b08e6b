"""CPU pinning of the oracle (oracle/fa_oracle.c) -- no GPU needed.

Every oracle function is checked against something it does not restate:
  * the committed golden vectors written by the reference's own CPU path
    (tests/golden/make_golden.py: friday_cpu::rope / decodeAttention compiled
    from cpu_ops.cpp), bit for bit;
  * the live reference build in oracle/_ref when present (build container);
  * numpy's IEEE fp16 conversion and torch's bf16 conversion, exhaustively or
    on large samples;
  * float64 brute force and closed forms of the softmax rules.
"""
import os

import numpy as np
import pytest

from fa_helpers import bf16, bf16_as_f32, f16

HERE = os.path.dirname(os.path.abspath(__file__))
GOLDEN = os.path.join(HERE, "golden", "golden_cpu_path.npz")


@pytest.fixture(scope="module")
def golden():
    return np.load(GOLDEN, allow_pickle=False)


def h(bits):
    return np.asarray(bits, np.uint16).view(np.float16).astype(np.float32)


# ---------------------------------------------------------------- fp16 rules
def test_half_to_float_exhaustive(oracle):
    bits = np.arange(65536, dtype=np.uint16)
    got = oracle.h2f(bits)
    exp = bits.view(np.float16).astype(np.float32)
    same = (got.view(np.uint32) == exp.view(np.uint32)) | (np.isnan(got) & np.isnan(exp))
    assert same.all()


def test_float_to_half_rne(oracle):
    rng = np.random.default_rng(1)
    x = np.concatenate([rng.standard_normal(100000).astype(np.float32) * s for s in (1e-7, 1e-5, 1e-2, 1, 300, 6e4)])
    halves = np.arange(0, 0x7C00, dtype=np.uint16).view(np.float16).astype(np.float64)
    mids = ((halves[:-1] + halves[1:]) / 2).astype(np.float32)  # exact ties -> even
    x = np.concatenate([x, mids, -mids, np.float32([65504, 65519.99, 65520, 1e9, 0.0, -0.0])])
    with np.errstate(over="ignore"):
        exp = x.astype(np.float16).view(np.uint16)
    assert np.array_equal(oracle.f2h(x), exp)


def test_round_to_half_rules(oracle):
    assert oracle.round_to_half(float("nan")) == 0.0            # NaN -> 0
    assert oracle.round_to_half(1e9) == 65504.0                 # clamp before rounding
    assert oracle.round_to_half(-70000.0) == -65504.0
    assert oracle.round_to_half(1.0 + 2 ** -11) == 1.0          # tie to even
    assert oracle.round_to_half(1.0 + 3 * 2 ** -11) == 1.0 + 2 ** -9


# ---------------------------------------------------------------- golden vectors (reference CPU path)
def test_golden_rope_neox_config1(oracle, golden):
    Hq, Hkv, d, pos = golden["a_meta"]
    q, k, v = golden["a_q"].copy()[None], golden["a_k"].copy()[None], golden["a_v"].copy()[None]
    cs = oracle.rope_table(pos + 1, d, 1e6)
    kc = np.zeros((pos + 1, Hkv * d), np.uint16)
    vc = kc.copy()
    oracle.rope_append(q, k, v, kc, vc, cs, pos, Hq, Hkv, d, True)
    assert np.array_equal(h(q[0]).view(np.uint32), golden["a_q_rot"].view(np.uint32))
    assert np.array_equal(h(k[0]).view(np.uint32), golden["a_k_rot"].view(np.uint32))
    assert np.array_equal(kc[pos], k[0]) and np.array_equal(vc[pos], v[0])


def test_golden_decode_config1(oracle, golden):
    """Append at 512 then attend over 513 (cpu_backend.cpp:111-117): bit-exact."""
    Hq, Hkv, d, pos = golden["a_meta"]
    q, k, v = golden["a_q"].copy()[None], golden["a_k"].copy()[None], golden["a_v"].copy()[None]
    kc, vc = golden["a_kcache"].copy(), golden["a_vcache"].copy()
    cs = oracle.rope_table(pos + 1, d, 1e6)
    oracle.rope_append(q, k, v, kc, vc, cs, pos, Hq, Hkv, d, True)
    out = oracle.decode(q[0], kc, vc, pos + 1, Hq, Hkv, d)
    assert np.array_equal(out.view(np.uint32), golden["a_out"].view(np.uint32))


def test_golden_rope_interleaved_freq_factors(oracle, golden):
    Hq, Hkv, d, pos = golden["b_meta"]
    q, k = golden["b_q"].copy()[None], golden["b_k"].copy()[None]
    cs = oracle.rope_table(pos + 1, d, 5e5, golden["b_ff"])
    oracle.rope_append(q, k, k.copy(), None, None, cs, pos, Hq, Hkv, d, False)
    assert np.array_equal(h(q[0]).view(np.uint32), golden["b_q_rot"].view(np.uint32))
    assert np.array_equal(h(k[0]).view(np.uint32), golden["b_k_rot"].view(np.uint32))


def test_golden_decode_nan_and_outlier(oracle, golden):
    Hq, Hkv, d, S = golden["c_meta"]
    out = oracle.decode(golden["c_q"], golden["c_kcache"], golden["c_vcache"], S, Hq, Hkv, d)
    assert np.array_equal(out.view(np.uint32), golden["c_out"].view(np.uint32))


# ---------------------------------------------------------------- live reference build (build container only)
def _ref():
    from py_oracle import RefCpu, ref_available
    if not ref_available():
        pytest.skip("oracle/_ref not built (needs /root/reference at build time)")
    return RefCpu()


@pytest.mark.parametrize("Hq,Hkv,d,S,threads", [(14, 2, 64, 513, 1), (40, 8, 128, 1000, 7), (32, 8, 128, 1, 3),
                                                 (16, 16, 128, 77, 2)])
def test_decode_bitexact_vs_reference_build(oracle, Hq, Hkv, d, S, threads):
    ref = _ref()
    rng = np.random.default_rng(S)
    kc, vc, q = f16(rng, (S, Hkv * d)), f16(rng, (S, Hkv * d)), f16(rng, Hq * d, 2.0)
    a = oracle.decode(q, kc, vc, S, Hq, Hkv, d)
    b = ref.decode(h(q), h(kc), h(vc), S, Hq, Hkv, d, threads=threads)
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))


@pytest.mark.parametrize("pos,neox", [(0, 1), (1, 0), (777, 1), (32767, 1), (32767, 0)])
def test_rope_bitexact_vs_reference_build(oracle, pos, neox):
    ref = _ref()
    Hq, Hkv, d = 40, 8, 128
    rng = np.random.default_rng(pos + neox)
    q, k = f16(rng, (1, Hq * d), 4.0), f16(rng, (1, Hkv * d), 4.0)
    qf, kf = h(q[0]).copy(), h(k[0]).copy()
    ref.rope(qf, kf, d, Hq, Hkv, pos, 1e6, neox)
    cs = oracle.rope_table(pos + 1, d, 1e6)
    oracle.rope_append(q, k, k.copy(), None, None, cs, pos, Hq, Hkv, d, neox)
    assert np.array_equal(h(q[0]).view(np.uint32), qf.view(np.uint32))
    assert np.array_equal(h(k[0]).view(np.uint32), kf.view(np.uint32))


# ---------------------------------------------------------------- mathematics
@pytest.mark.parametrize("Hq,Hkv,d,S", [(4, 2, 64, 1), (8, 2, 128, 17), (6, 3, 64, 64), (40, 8, 128, 200)])
def test_decode_vs_float64(oracle, Hq, Hkv, d, S):
    rng = np.random.default_rng(S * 3 + d)
    kc, vc, q = f16(rng, (S, Hkv * d)), f16(rng, (S, Hkv * d)), f16(rng, Hq * d, 2.0)
    got = oracle.decode(q, kc, vc, S, Hq, Hkv, d)
    exact = oracle.decode_f64(q, kc, vc, S, Hq, Hkv, d)
    # independent numpy restatement of softmax attention for the float64 path
    qh, kh, vh = h(q).reshape(Hq, d), h(kc).reshape(S, Hkv, d), h(vc).reshape(S, Hkv, d)
    G = Hq // Hkv
    for hh in range(Hq):
        s = kh[:, hh // G, :].astype(np.float64) @ qh[hh].astype(np.float64) / np.sqrt(d)
        w = np.exp(s - s.max())
        w /= w.sum()
        np.testing.assert_allclose(exact[hh * d:(hh + 1) * d], w @ vh[:, hh // G, :], rtol=1e-9, atol=1e-12)
    np.testing.assert_allclose(got, exact, atol=2e-3, rtol=1e-2)
    assert np.all(np.abs(got - exact) <= np.abs(exact) * 2 ** -10 + 1e-6)  # fp32 math + one fp16 rounding


def test_decode_closed_forms(oracle):
    rng = np.random.default_rng(4)
    Hq, Hkv, d, S = 8, 2, 64, 50
    kc, vc, q = f16(rng, (S, Hkv * d)), f16(rng, (S, Hkv * d)), f16(rng, Hq * d)
    # S = 1: out = v0
    out = oracle.decode(q, kc, vc, 1, Hq, Hkv, d)
    assert np.array_equal(out, np.concatenate([h(vc[0, (i // 4) * d:(i // 4 + 1) * d]) for i in range(Hq)]))
    # all-NaN q: every score -1e30 -> uniform weights -> mean of V (cpu_ops.cpp:63-71)
    qn = np.full(Hq * d, np.float16(np.nan).view(np.uint16), np.uint16)
    out = oracle.decode(qn, kc, vc, S, Hq, Hkv, d)
    mean = h(vc).reshape(S, Hkv, d).mean(0)
    np.testing.assert_allclose(out.reshape(Hq, d), np.repeat(mean, 4, 0), atol=2e-3)
    # a key with margin > 50: weight 1 on it, exactly
    qd = np.ones(Hq * d, np.float16).view(np.uint16)
    kd = np.zeros((S, Hkv * d), np.float16)
    kd[9] = 8.0
    out = oracle.decode(qd, kd.view(np.uint16), vc, S, Hq, Hkv, d)
    assert np.array_equal(out, np.concatenate([h(vc[9, (i // 4) * d:(i // 4 + 1) * d]) for i in range(Hq)]))


def test_split_partition_invariance(oracle):
    rng = np.random.default_rng(8)
    Hq, Hkv, d, S = 40, 8, 128, 1000
    kc, vc, q = f16(rng, (S, Hkv * d)), f16(rng, (S, Hkv * d)), f16(rng, Hq * d, 2.0)
    base = oracle.decode(q, kc, vc, S, Hq, Hkv, d)
    for ns in (1, 2, 7, 32, 128):
        np.testing.assert_allclose(oracle.decode_split(q, kc, vc, S, Hq, Hkv, d, ns), base, atol=2e-3, rtol=1e-2)


def test_lse_merge_forms(oracle):
    rng = np.random.default_rng(9)
    o = rng.standard_normal((1, 64)).astype(np.float32)
    # one split: o / l
    np.testing.assert_allclose(oracle.lse_merge(o, np.float32([3.0]), np.float32([2.5])),
                               [oracle.round_to_half(x) for x in o[0] / 2.5])
    # a split 60 below the max contributes nothing (cut-off at -50)
    o2 = np.vstack([o, 1e3 * np.ones((1, 64), np.float32)])
    got = oracle.lse_merge(o2, np.float32([3.0, -57.0]), np.float32([2.5, 1.0]))
    np.testing.assert_array_equal(got, [oracle.round_to_half(x) for x in o[0] / 2.5])


def test_prefill_is_causal_decode(oracle):
    rng = np.random.default_rng(10)
    Hq, Hkv, d, T, p0 = 16, 4, 64, 9, 20
    kc, vc, q = f16(rng, (p0 + T, Hkv * d)), f16(rng, (p0 + T, Hkv * d)), f16(rng, (T, Hq * d))
    out = oracle.prefill(q, kc, vc, T, p0, Hq, Hkv, d)
    for t in range(T):
        assert np.array_equal(out[t], oracle.decode(q[t], kc, vc, p0 + t + 1, Hq, Hkv, d))
    kc2 = kc.copy()
    kc2[p0 + 5:] = f16(rng, kc2[p0 + 5:].shape, 9.0)
    out2 = oracle.prefill(q, kc2, vc, T, p0, Hq, Hkv, d)
    assert np.array_equal(out[:5], out2[:5])


# ---------------------------------------------------------------- bf16 rules
def test_bf16_to_float_exhaustive(oracle):
    import torch
    bits = np.arange(65536, dtype=np.uint16)
    got = np.array([oracle.lib.or_bf16_to_float(int(b)) for b in bits], np.float32)
    exp = torch.from_numpy(bits.view(np.int16).copy()).view(torch.bfloat16).float().numpy()
    same = (got.view(np.uint32) == exp.view(np.uint32)) | (np.isnan(got) & np.isnan(exp))
    assert same.all()


def test_float_to_bf16_rne(oracle):
    """torch's float -> bfloat16 (round to nearest even) on random bit patterns, ties,
    the neighbours of ties, subnormals, infinities and NaN."""
    import torch
    rng = np.random.default_rng(41)
    x = rng.integers(0, 2**32, 200000, dtype=np.uint64).astype(np.uint32)
    base = rng.integers(0, 2**16, 2000, dtype=np.uint64).astype(np.uint32) << 16
    ties = np.concatenate([base | 0x8000, base | 0x7FFF, base | 0x8001, base | 0x10000 | 0x8000])
    edges = np.array([0, 0x80000000, 1, 0x007FFFFF, 0x7F7FFFFF, 0x7F7F8000, 0x7F800000, 0xFF800000, 0x7FC00000,
                      0x7F800001, 0x3F808000, 0x3F818000], np.uint32)
    bits = np.concatenate([x, ties.astype(np.uint32), edges])
    f = bits.view(np.float32)
    got = np.array([oracle.lib.or_float_to_bf16(float(v)) for v in f], np.uint16)
    exp = torch.from_numpy(f.copy()).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    nan = np.isnan(f)
    assert np.array_equal(got[~nan], exp[~nan])
    assert np.isnan(bf16_as_f32(got[nan])).all()
    assert oracle.lib.or_round_to_bf16(float("nan")) == 0.0


def _bf16_bits_exact(x):
    """bf16 bits of float32 values that bf16 holds exactly (the low 16 bits are zero)."""
    b = np.asarray(x, np.float32).view(np.uint32)
    assert not (b & 0xFFFF).any()
    return (b >> 16).astype(np.uint16)


def _dual_values(rng, shape):
    """Values exact in fp16 and in bf16 (m * 2^-6, |m| < 256): fp16 bits, bf16 bits."""
    m = rng.integers(-255, 256, shape).astype(np.float32) * np.float32(2.0**-6)
    return m.astype(np.float16).view(np.uint16), _bf16_bits_exact(m)


def test_prefill_bf16_matches_fp16_path_on_shared_values(oracle):
    """On inputs that fp16 and bf16 both hold exactly, the two prefills accumulate the same
    fp32 values in the same order: they differ only in the final rounding. So the bf16
    output is the bf16 rounding of the fp16 output wherever that fp16 value is not a
    bf16 midpoint (double rounding fp32 -> fp16 -> bf16 only differs there). A transposed
    operand, a wrong cache or head index, or a wrong widening would break this."""
    rng = np.random.default_rng(42)
    Hq, Hkv, d, T, p0 = 12, 4, 64, 7, 30
    q16, qb = _dual_values(rng, (T, Hq * d))
    k16, kb = _dual_values(rng, (p0 + T, Hkv * d))
    v16, vb = _dual_values(rng, (p0 + T, Hkv * d))
    o16 = oracle.prefill(q16, k16, v16, T, p0, Hq, Hkv, d)
    ob = oracle.prefill_bf16(qb, kb, vb, T, p0, Hq, Hkv, d)
    rounded = np.array([oracle.lib.or_round_to_bf16(float(v)) for v in o16.ravel()], np.float32).reshape(o16.shape)
    # fp16 outputs that sit exactly halfway between two bf16 values: there the fp32 value
    # may lie on either side, so the bf16 output is either neighbour
    tie = (o16.view(np.uint32) & 0xFFFF) == 0x8000
    assert np.array_equal(rounded[~tie], ob[~tie])
    lo = (o16.view(np.uint32) & 0xFFFF0000).view(np.float32)
    hi = ((o16.view(np.uint32) & 0xFFFF0000) + 0x10000).view(np.float32)
    assert ((ob[tie] == lo[tie]) | (ob[tie] == hi[tie])).all()
    _bf16_bits_exact(ob)  # every output is a bf16 value


def test_prefill_bf16_f64_brute_force(oracle):
    """Against float64 attention over the widened bf16 inputs: the oracle's only errors
    are fp32 accumulation and the final bf16 rounding (half a bf16 step, 2^-9 relative)."""
    rng = np.random.default_rng(43)
    Hq, Hkv, d, T, p0 = 8, 2, 128, 5, 60
    q, k, v = bf16(rng, (T, Hq * d)), bf16(rng, (p0 + T, Hkv * d)), bf16(rng, (p0 + T, Hkv * d))
    got = oracle.prefill_bf16(q, k, v, T, p0, Hq, Hkv, d)
    qf, kf, vf = (bf16_as_f32(a).astype(np.float64) for a in (q, k, v))
    G = Hq // Hkv
    for t in range(T):
        S = p0 + t + 1
        for hh in range(Hq):
            kv = hh // G
            s = kf[:S, kv * d:(kv + 1) * d] @ qf[t, hh * d:(hh + 1) * d] / np.sqrt(d)
            w = np.exp(s - s.max())
            ref = (w / w.sum()) @ vf[:S, kv * d:(kv + 1) * d]
            np.testing.assert_allclose(got[t, hh * d:(hh + 1) * d], ref, rtol=2.0**-8, atol=1e-5)


def test_store_kv_q8_rules(oracle):
    rng = np.random.default_rng(11)
    kv_dim = 64
    k = f16(rng, (1, kv_dim), 3.0)
    v = f16(rng, (1, kv_dim), 3.0)
    k[0, :32] = 0
    k8 = np.zeros((1, kv_dim), np.int8)
    v8 = k8.copy()
    ks = np.zeros((1, 2), np.uint16)
    vs = ks.copy()
    oracle.store_kv_q8(k, v, k8, ks, v8, vs, 0, kv_dim)
    assert (k8[0, :32] == 0).all() and ks[0, 0] == 0           # zero block: scale 0, values 0
    for blk, (x8, sc, src) in enumerate([(k8, ks, k), (v8, vs, v)]):
        for b in range(2):
            x = h(src[0, b * 32:(b + 1) * 32]).astype(np.float64)
            amax = np.abs(x).max()
            dh = np.float16(np.float32(amax) / np.float32(127.0))
            assert sc[0, b] == dh.view(np.uint16)
            if amax == 0:
                continue
            deq = x8[0, b * 32:(b + 1) * 32].astype(np.float64) * float(dh)
            assert np.all(np.abs(deq - x) <= float(dh) * 0.5 * (1 + 1e-6) + float(dh) * 127 * 2 ** -11)
            assert np.abs(x8[0, b * 32:(b + 1) * 32]).max() == 127 or float(dh) * 127 > amax


def test_paged_gather(oracle):
    rng = np.random.default_rng(12)
    kv_dim, S, page = 32, 50, 16
    rows = f16(rng, (S, kv_dim))
    nb = (S + page - 1) // page
    perm = rng.permutation(nb).astype(np.int32)
    pool = np.zeros((nb, page, kv_dim), np.uint16)
    for j in range(nb):
        n = min(page, S - j * page)
        pool[perm[j], :n] = rows[j * page:j * page + n]
    assert np.array_equal(oracle.paged_gather(pool, perm, S, page, kv_dim), rows)


@pytest.mark.parametrize("Hq,Hkv,d,T,p0", [(8, 2, 64, 37, 21), (40, 8, 128, 40, 300), (16, 1, 128, 3, 0),
                                            (48, 3, 64, 20, 5)])
def test_blocked_prefill_equals_row_by_row(oracle, Hq, Hkv, d, T, p0):
    """The blocked evaluator the GPU tests use for whole config-4 chunks (prefill_all:
    or_prefill_widen + or_prefill_rows_f32 over threaded row blocks) gives the row-by-row
    oracle prefill bit for bit: fp16, int8 and bf16 caches, with a NaN key row, an all-NaN
    query row, an outlier key and a score block boundary inside the rows."""
    from fa_helpers import f16

    rng = np.random.default_rng(11 + T)
    S = p0 + T
    q = f16(rng, (T, Hq * d))
    k, v = f16(rng, (S, Hkv * d)), f16(rng, (S, Hkv * d))
    k[S // 2] = 0x7E00  # NaN key row
    k[S // 3, :d] = np.float16(40.0).view(np.uint16)  # outlier key of kv head 0
    q[T // 2] = 0x7E00  # every score of this row NaN
    for blk, workers in ((16, 16), (5, 3), (1, 2)):
        want = oracle.prefill(q, k, v, T, p0, Hq, Hkv, d)
        got = oracle.prefill_all(q, k, v, T, p0, Hq, Hkv, d, block=blk, workers=workers)
        assert np.array_equal(want.view(np.uint32), got.view(np.uint32)), f"fp16 block={blk}"
        wb = oracle.prefill_bf16(q, k, v, T, p0, Hq, Hkv, d)
        gb = oracle.prefill_all(q, k, v, T, p0, Hq, Hkv, d, bf16=True, block=blk, workers=workers)
        assert np.array_equal(wb.view(np.uint32), gb.view(np.uint32)), f"bf16 block={blk}"
    k8 = rng.integers(-127, 128, (S, Hkv * d), dtype=np.int8)
    v8 = rng.integers(-127, 128, (S, Hkv * d), dtype=np.int8)
    ks = rng.uniform(0.001, 0.02, (S, Hkv * d // 32)).astype(np.float16).view(np.uint16)
    vs = rng.uniform(0.001, 0.02, (S, Hkv * d // 32)).astype(np.float16).view(np.uint16)
    wq = oracle.prefill_q8(q, k8, ks, v8, vs, T, p0, Hq, Hkv, d)
    gq = oracle.prefill_all(q, k8, v8, T, p0, Hq, Hkv, d, ks=ks, vs=vs, block=7, workers=4)
    assert np.array_equal(wq.view(np.uint32), gq.view(np.uint32))


def test_blocked_prefill_long_prefix(oracle):
    """Several 256-position score blocks and a long prefix (the config-4 regime), against the
    row-by-row oracle on a few rows."""
    from fa_helpers import f16

    rng = np.random.default_rng(3)
    Hq, Hkv, d, T, p0 = 40, 8, 128, 24, 1500
    q = f16(rng, (T, Hq * d))
    k, v = f16(rng, (p0 + T, Hkv * d)), f16(rng, (p0 + T, Hkv * d))
    got = oracle.prefill_all(q, k, v, T, p0, Hq, Hkv, d)
    want = oracle.prefill(q, k, v, T, p0, Hq, Hkv, d)
    assert np.array_equal(want.view(np.uint32), got.view(np.uint32))
