"""CPU pinning of the oracle (oracle/fa_oracle.c) -- no GPU needed.

Every oracle function is checked against something it does not restate:
  * the committed golden vectors written by the reference's own CPU path
    (tests/golden/make_golden.py: friday_cpu::rope / decodeAttention compiled
    from cpu_ops.cpp), bit for bit;
  * the live reference build in oracle/_ref when present (build container);
  * numpy's IEEE fp16 conversion, exhaustively;
  * float64 brute force and closed forms of the softmax rules.
"""
import os

import numpy as np
import pytest

from fa_helpers import f16

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
