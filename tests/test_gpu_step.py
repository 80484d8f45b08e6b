"""GPU parity of the one-launch decode layer-step (RoPE + KV append + split-K decode + merge).

Bar: cache rows and rotated q bit-exact vs the oracle append; attention output
bit-identical to the two-launch sequence (rope_store_kv, then the fused split
decode) and within tolerance of the oracle; paged step bit-identical to the
contiguous step per sequence.
"""
import numpy as np
import pytest

from fa_helpers import as_f32, assert_close, f16

pytestmark = pytest.mark.gpu


def run_step_vs_two_launch(fa, oracle, Hq, Hkv, d, S, max_ctx, base, neox, devpos, seed):
    rng = np.random.default_rng(seed)
    kv_dim = Hkv * d
    kc = f16(rng, (max_ctx, kv_dim))
    vc = f16(rng, (max_ctx, kv_dim))
    q, k, v = f16(rng, (1, Hq * d), 2.0), f16(rng, (1, kv_dim)), f16(rng, (1, kv_dim))
    pos = S - 1
    table = fa.rope_table_host(max_ctx, d, base)
    dt = fa.DeviceBuffer.from_array(table)
    dpos = fa.DeviceBuffer.from_array(np.array([pos], np.int32))
    ws_bytes = fa.splitAttentionWorkspaceBytes(Hq, max_ctx)

    # one launch
    b1 = {n: fa.DeviceBuffer.from_array(a) for n, a in dict(q=q, k=k, v=v, kc=kc, vc=vc).items()}
    out1 = fa.DeviceBuffer(q.nbytes)
    ws1 = fa.DeviceBuffer(ws_bytes)
    fa.decodeWorkspaceInit(ws1)
    fa.decodeStep(b1["q"], b1["k"], b1["v"], b1["kc"], b1["vc"], out1, dpos if devpos else None,
                  0 if devpos else pos, max_ctx, Hq, Hkv, d, dt, neox, ws1)
    # two launches
    b2 = {n: fa.DeviceBuffer.from_array(a) for n, a in dict(q=q, k=k, v=v, kc=kc, vc=vc).items()}
    out2 = fa.DeviceBuffer(q.nbytes)
    ws2 = fa.DeviceBuffer(ws_bytes)
    fa.decodeWorkspaceInit(ws2)
    fa.ropeStoreKv(b2["q"], b2["k"], b2["v"], b2["kc"], b2["vc"], dpos if devpos else None, 0 if devpos else pos, 1,
                   d, Hq, Hkv, max_ctx, dt, neox)
    fa.launchDecodeAttentionFused(b2["q"], b2["kc"], b2["vc"], out2, 0 if devpos else S, dpos if devpos else None,
                                  max_ctx, Hq, Hkv, d, ws2)
    fa.Hip.sync()

    qr, kr = q.copy(), k.copy()
    oracle.rope_append(qr, kr, v, kc, vc, table, pos, Hq, Hkv, d, neox)
    assert np.array_equal(b1["kc"].download(kc.shape, np.uint16), kc), "k cache after step"
    assert np.array_equal(b1["vc"].download(vc.shape, np.uint16), vc), "v cache after step"
    assert np.array_equal(b1["q"].download(q.shape, np.uint16), qr), "rotated q written back"
    assert np.array_equal(b1["k"].download(k.shape, np.uint16), k), "k input left unrotated"
    g1 = out1.download(Hq * d, np.uint16)
    g2 = out2.download(Hq * d, np.uint16)
    assert np.array_equal(g1, g2), "step differs from the two-launch sequence"
    assert_close(as_f32(g1), oracle.decode(qr[0], kc, vc, S, Hq, Hkv, d), f"step S={S}")
    return ws1


@pytest.mark.parametrize("Hq,Hkv,d,S,max_ctx,base,neox,devpos", [
    (14, 2, 64, 513, 1024, 1e6, 1, True),       # config 1: append at 512, attend 513
    (32, 8, 128, 4096, 4096, 5e5, 0, True),     # config 2 shapes, interleaved pairs
    (40, 8, 128, 32768, 32768, 1e6, 1, True),   # config 3 headline
    (40, 8, 128, 1, 64, 1e6, 1, False),         # first token
    (40, 8, 128, 300, 512, 1e6, 1, False),
    (64, 4, 128, 2000, 2048, 1e6, 1, True),     # G = 16
    (48, 1, 128, 999, 1024, 1e4, 0, True),      # G = 48: three head blocks
])
def test_step_matches_two_launches(gpu, oracle, Hq, Hkv, d, S, max_ctx, base, neox, devpos):
    run_step_vs_two_launch(gpu, oracle, Hq, Hkv, d, S, max_ctx, base, neox, devpos, seed=S + Hq)


@pytest.mark.parametrize("over,neox", [(0, 1), (3, 0)])
def test_step_position_past_cache(gpu, over, neox):
    """*d_pos >= max_ctx: the separate append skips the token (q stays unrotated, no row is
    written), then attention covers the max_ctx cached rows. The step does the same, bit for
    bit."""
    fa = gpu
    Hq, Hkv, d, max_ctx = 40, 8, 128, 4096
    rng = np.random.default_rng(77 + over)
    kv_dim = Hkv * d
    kc, vc = f16(rng, (max_ctx, kv_dim)), f16(rng, (max_ctx, kv_dim))
    q, k, v = f16(rng, (1, Hq * d)), f16(rng, (1, kv_dim)), f16(rng, (1, kv_dim))
    dt = fa.DeviceBuffer.from_array(fa.rope_table_host(max_ctx, d, 1e6))
    dpos = fa.DeviceBuffer.from_array(np.array([max_ctx + over], np.int32))
    ws_bytes = fa.splitAttentionWorkspaceBytes(Hq, max_ctx)
    outs, bufs = [], []
    for fused in (True, False):
        b = {n: fa.DeviceBuffer.from_array(a) for n, a in dict(q=q, k=k, v=v, kc=kc, vc=vc).items()}
        out, ws = fa.DeviceBuffer(q.nbytes), fa.DeviceBuffer(ws_bytes)
        fa.decodeWorkspaceInit(ws)
        if fused:
            fa.decodeStep(b["q"], b["k"], b["v"], b["kc"], b["vc"], out, dpos, 0, max_ctx, Hq, Hkv, d, dt, neox, ws)
        else:
            fa.ropeStoreKv(b["q"], b["k"], b["v"], b["kc"], b["vc"], dpos, 0, 1, d, Hq, Hkv, max_ctx, dt, neox)
            fa.launchDecodeAttentionFused(b["q"], b["kc"], b["vc"], out, 0, dpos, max_ctx, Hq, Hkv, d, ws)
        outs.append(out)
        bufs.append(b)
    fa.Hip.sync()
    for name, b in zip(("step", "two launches"), bufs):
        assert np.array_equal(b["q"].download(q.shape, np.uint16), q), f"{name}: q changed"
        assert np.array_equal(b["kc"].download(kc.shape, np.uint16), kc), f"{name}: k cache changed"
        assert np.array_equal(b["vc"].download(vc.shape, np.uint16), vc), f"{name}: v cache changed"
    g1, g2 = (o.download(Hq * d, np.uint16) for o in outs)
    assert np.array_equal(g1, g2), "step differs from the two-launch sequence"


def test_step_workspace_rearms(gpu, oracle):
    """Counters return to zero: consecutive steps on one workspace keep the bits."""
    fa = gpu
    Hq, Hkv, d, max_ctx = 40, 8, 128, 4096
    rng = np.random.default_rng(21)
    kv_dim = Hkv * d
    kc, vc = f16(rng, (max_ctx, kv_dim)), f16(rng, (max_ctx, kv_dim))
    table = fa.DeviceBuffer.from_array(fa.rope_table_host(max_ctx, d, 1e6))
    ws = fa.DeviceBuffer(fa.splitAttentionWorkspaceBytes(Hq, max_ctx))
    fa.decodeWorkspaceInit(ws)
    dkc, dvc = fa.DeviceBuffer.from_array(kc), fa.DeviceBuffer.from_array(vc)
    out = fa.DeviceBuffer(Hq * d * 2)
    for pos in (1000, 1001, 1002, 3000):
        q, k, v = f16(rng, (1, Hq * d)), f16(rng, (1, kv_dim)), f16(rng, (1, kv_dim))
        dq, dk, dv = (fa.DeviceBuffer.from_array(a) for a in (q, k, v))
        dpos = fa.DeviceBuffer.from_array(np.array([pos], np.int32))
        fa.decodeStep(dq, dk, dv, dkc, dvc, out, dpos, 0, max_ctx, Hq, Hkv, d, table, 1, ws)
        fa.Hip.sync()
        qr = q.copy()
        oracle.rope_append(qr, k.copy(), v, kc, vc, table.download((max_ctx, d // 2, 2), np.float32), pos, Hq, Hkv,
                           d, 1)
        assert_close(as_f32(out.download(Hq * d, np.uint16)), oracle.decode(qr[0], kc, vc, pos + 1, Hq, Hkv, d),
                     f"pos {pos}")


def test_paged_step_matches_contiguous_step(gpu):
    """benchmark config 5 in one launch: every sequence equals the contiguous step bit for bit."""
    from test_gpu_paged import build_paged
    fa = gpu
    Hq, Hkv, d, nseq, PAGE = 40, 8, 128, 9, 16
    kv_dim = Hkv * d
    rng = np.random.default_rng(55)
    lens = [int(x) for x in rng.integers(256, 5000, nseq)]  # after the append
    max_seq = 5120
    seqs, table, k_pool, v_pool = build_paged(rng, lens, kv_dim, max_seq)
    q, k, v = f16(rng, (nseq, Hq * d)), f16(rng, (nseq, kv_dim)), f16(rng, (nseq, kv_dim))
    rope = fa.DeviceBuffer.from_array(fa.rope_table_host(max_seq, d, 1e6))
    bufs = {n: fa.DeviceBuffer.from_array(a) for n, a in
            dict(q=q, k=k, v=v, kp=k_pool, vp=v_pool, t=table, l=np.array(lens, np.int32)).items()}
    out = fa.DeviceBuffer(q.nbytes)
    ws = fa.DeviceBuffer(fa.pagedWorkspaceBytes(nseq, Hq, max_seq))
    fa.decodeWorkspaceInit(ws)
    fa.pagedDecodeStep(bufs["q"], bufs["k"], bufs["v"], bufs["kp"], bufs["vp"], out, bufs["t"], table.shape[1],
                       bufs["l"], nseq, max_seq, Hq, Hkv, d, rope, 1, ws)
    fa.Hip.sync()
    got = out.download((nseq, Hq * d), np.uint16)
    got_kp = bufs["kp"].download(k_pool.shape, np.uint16)
    for b, S in enumerate(lens):
        kc = np.zeros((max_seq, kv_dim), np.uint16)
        vc = np.zeros_like(kc)
        kc[:S], vc[:S] = seqs[b]
        dq, dk, dv = (fa.DeviceBuffer.from_array(a) for a in (q[b:b + 1], k[b:b + 1], v[b:b + 1]))
        dkc, dvc = fa.DeviceBuffer.from_array(kc), fa.DeviceBuffer.from_array(vc)
        o1 = fa.DeviceBuffer(Hq * d * 2)
        w1 = fa.DeviceBuffer(fa.splitAttentionWorkspaceBytes(Hq, max_seq))
        fa.decodeWorkspaceInit(w1)
        dpos = fa.DeviceBuffer.from_array(np.array([S - 1], np.int32))
        fa.decodeStep(dq, dk, dv, dkc, dvc, o1, dpos, 0, max_seq, Hq, Hkv, d, rope, 1, w1)
        fa.Hip.sync()
        assert np.array_equal(got[b], o1.download(Hq * d, np.uint16)), f"seq {b} S={S}"
        row = dkc.download((max_seq, kv_dim), np.uint16)[S - 1]
        assert np.array_equal(got_kp[table[b, (S - 1) // PAGE], (S - 1) % PAGE], row), f"k row seq {b}"


@pytest.mark.parametrize("Hq,Hkv,d,S,max_ctx,neox,devpos", [
    (40, 8, 128, 32768, 32768, 1, True),   # headline shape, int8 KV
    (32, 8, 128, 1000, 1024, 0, False),    # interleaved pairs
    (14, 2, 64, 513, 1024, 1, True),       # d = 64
    (40, 8, 128, 1, 64, 1, True),          # first token
])
def test_step_q8_matches_three_launches(gpu, oracle, Hq, Hkv, d, S, max_ctx, neox, devpos):
    """int8 KV (--kv q8): one launch == ropeStoreKv without caches + storeKvQ8 + fused split
    decode with scales (transformer.cpp:1035-1040, 1049-1051), bit for bit, including the
    quantized cache row and its scales; and within tolerance of the oracle."""
    fa = gpu
    rng = np.random.default_rng(S + 7)
    kv_dim = Hkv * d
    kf, vf = f16(rng, (max_ctx, kv_dim)), f16(rng, (max_ctx, kv_dim))
    k8, v8 = np.zeros((max_ctx, kv_dim), np.int8), np.zeros((max_ctx, kv_dim), np.int8)
    ks, vs = np.zeros((max_ctx, kv_dim // 32), np.uint16), np.zeros((max_ctx, kv_dim // 32), np.uint16)
    oracle.store_kv_q8(kf, vf, k8, ks, v8, vs, 0, kv_dim)
    q, k, v = f16(rng, (1, Hq * d), 2.0), f16(rng, (1, kv_dim)), f16(rng, (1, kv_dim))
    pos = S - 1
    table = fa.rope_table_host(max_ctx, d, 1e6)
    dt = fa.DeviceBuffer.from_array(table)
    dpos = fa.DeviceBuffer.from_array(np.array([pos], np.int32))
    ws_bytes = fa.splitAttentionWorkspaceBytes(Hq, max_ctx)
    P, pp = (dpos, 0) if devpos else (None, pos)

    b1 = {n: fa.DeviceBuffer.from_array(a) for n, a in dict(q=q, k=k, v=v, k8=k8, ks=ks, v8=v8, vs=vs).items()}
    out1, ws1 = fa.DeviceBuffer(q.nbytes), fa.DeviceBuffer(ws_bytes)
    fa.decodeWorkspaceInit(ws1)
    fa.decodeStepQ8(b1["q"], b1["k"], b1["v"], b1["k8"], b1["ks"], b1["v8"], b1["vs"], out1, P, pp, max_ctx, Hq, Hkv,
                    d, dt, neox, ws1)

    b2 = {n: fa.DeviceBuffer.from_array(a) for n, a in dict(q=q, k=k, v=v, k8=k8, ks=ks, v8=v8, vs=vs).items()}
    out2, ws2 = fa.DeviceBuffer(q.nbytes), fa.DeviceBuffer(ws_bytes)
    fa.decodeWorkspaceInit(ws2)
    fa.ropeStoreKv(b2["q"], b2["k"], b2["v"], None, None, P, pp, 1, d, Hq, Hkv, max_ctx, dt, neox)
    fa.storeKvQ8(b2["k"], b2["v"], b2["k8"], b2["ks"], b2["v8"], b2["vs"], P, pp, 1, kv_dim, max_ctx)
    fa.launchDecodeAttentionFused(b2["q"], b2["k8"], b2["v8"], out2, 0 if devpos else S, P, max_ctx, Hq, Hkv, d, ws2,
                                  k_scale=b2["ks"], v_scale=b2["vs"])
    fa.Hip.sync()

    for n, a in dict(k8=k8, ks=ks, v8=v8, vs=vs).items():
        assert np.array_equal(b1[n].download(a.shape, a.dtype), b2[n].download(a.shape, a.dtype)), n
    assert np.array_equal(b1["q"].download(q.shape, np.uint16), b2["q"].download(q.shape, np.uint16)), "rotated q"
    g1, g2 = out1.download(Hq * d, np.uint16), out2.download(Hq * d, np.uint16)
    assert np.array_equal(g1, g2), "int8 step differs from the three-launch sequence"
    # oracle: rope (q, k), int8 append at pos, int8 decode over S
    qr, kr, vr = q.copy(), k.copy(), v.copy()
    oracle.rope_append(qr, kr, vr, None, None, table, pos, Hq, Hkv, d, neox)
    oracle.store_kv_q8(kr, vr, k8, ks, v8, vs, pos, kv_dim)
    assert np.array_equal(b1["k8"].download(k8.shape, np.int8), k8), "int8 k row vs oracle"
    assert np.array_equal(b1["vs"].download(vs.shape, np.uint16), vs), "v scales vs oracle"
    assert_close(as_f32(g1), oracle.decode_q8(qr[0], k8, ks, v8, vs, S, Hq, Hkv, d), f"q8 step S={S}")


@pytest.mark.parametrize("Hq,Hkv,d,S,max_ctx", [
    (40, 8, 128, 32768, 32768),   # headline: 32 splits, short merge
    (40, 8, 128, 1, 4096),        # one split: the decode workgroup writes out
    (32, 8, 128, 20000, 20480),   # more than 8 splits per group
    (14, 2, 64, 513, 1024),       # d = 64
    (48, 1, 128, 2048, 2048),     # G = 48: three head blocks
])
def test_step_quant_matches_step_plus_quantize(gpu, oracle, Hq, Hkv, d, S, max_ctx):
    """friday_attn_decode_step_quant = decode step + quantizeQ8 of its output, bit for bit."""
    fa = gpu
    rng = np.random.default_rng(S + Hq)
    kv_dim = Hkv * d
    kc, vc = f16(rng, (max_ctx, kv_dim)), f16(rng, (max_ctx, kv_dim))
    q, k, v = f16(rng, (1, Hq * d), 2.0), f16(rng, (1, kv_dim)), f16(rng, (1, kv_dim))
    dt = fa.DeviceBuffer.from_array(fa.rope_table_host(max_ctx, d, 1e6))
    dpos = fa.DeviceBuffer.from_array(np.array([S - 1], np.int32))
    ws_bytes = fa.splitAttentionWorkspaceBytes(Hq, max_ctx)
    outs = []
    for fused in (True, False):
        b = {n: fa.DeviceBuffer.from_array(a) for n, a in dict(q=q, k=k, v=v, kc=kc, vc=vc).items()}
        out = fa.DeviceBuffer(q.nbytes)
        oq, od = fa.DeviceBuffer(Hq * d), fa.DeviceBuffer(Hq * d // 32 * 4)
        ws = fa.DeviceBuffer(ws_bytes)
        fa.decodeWorkspaceInit(ws)
        if fused:
            fa.decodeStepQuant(b["q"], b["k"], b["v"], b["kc"], b["vc"], out, oq, od, dpos, 0, max_ctx, Hq, Hkv, d,
                               dt, 1, ws)
        else:
            fa.decodeStep(b["q"], b["k"], b["v"], b["kc"], b["vc"], out, dpos, 0, max_ctx, Hq, Hkv, d, dt, 1, ws)
            fa.quantizeQ8Rows(out, 1, Hq * d, oq, od)
        fa.Hip.sync()
        outs.append((out.download(Hq * d, np.uint16), oq.download(Hq * d, np.int8),
                     od.download(Hq * d // 32, np.float32)))
    (o1, q1, d1), (o2, q2, d2) = outs
    assert np.array_equal(o1, o2), "attention output"
    assert np.array_equal(q1, q2), "int8 codes"
    assert np.array_equal(d1.view(np.uint32), d2.view(np.uint32)), "scales"
    oq_ref, od_ref = oracle.quantize_q8_rows(o1[None])
    assert np.array_equal(q1, oq_ref[0]) and np.array_equal(d1.view(np.uint32), od_ref[0].view(np.uint32))
