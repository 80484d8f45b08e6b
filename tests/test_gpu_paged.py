"""GPU parity of paged multi-sequence append + decode (benchmark config 5).

16-token pages with physical ids from a seeded permutation, one block table row
per sequence. Bar: every sequence bit-identical to the contiguous-cache split
decode over the same logical rows, and within tolerance of the CPU oracle.
"""
import numpy as np
import pytest

from fa_helpers import as_f32, assert_close, f16

pytestmark = pytest.mark.gpu
PAGE = 16


def build_paged(rng, lens, kv_dim, max_seq):
    """Contiguous per-sequence rows and the same rows scattered into a page pool."""
    max_blocks = (max_seq + PAGE - 1) // PAGE
    nblocks = [(s + PAGE - 1) // PAGE for s in lens]
    total = sum(nblocks)
    perm = rng.permutation(total).astype(np.int32)
    table = np.full((len(lens), max_blocks), -1, np.int32)
    k_pool = np.zeros((total, PAGE, kv_dim), np.uint16)
    v_pool = np.zeros_like(k_pool)
    seqs = []
    at = 0
    for b, s in enumerate(lens):
        kc, vc = f16(rng, (s, kv_dim)), f16(rng, (s, kv_dim))
        seqs.append((kc, vc))
        for j in range(nblocks[b]):
            phys = perm[at]
            at += 1
            table[b, j] = phys
            rows = slice(j * PAGE, min(s, (j + 1) * PAGE))
            n = rows.stop - rows.start
            k_pool[phys, :n] = kc[rows]
            v_pool[phys, :n] = vc[rows]
    return seqs, table, k_pool, v_pool


def contiguous_decode(fa, q, kc, vc, S, Hq, Hkv, d, max_seq):
    dq, dk, dv = (fa.DeviceBuffer.from_array(a) for a in (q, kc, vc))
    out = fa.DeviceBuffer(q.nbytes)
    ws = fa.DeviceBuffer(fa.splitAttentionWorkspaceBytes(Hq, max_seq))
    dpos = fa.DeviceBuffer.from_array(np.array([S - 1], np.int32))
    fa.launchDecodeAttentionSplit(dq, dk, dv, out, 0, dpos, max_seq, Hq, Hkv, d, ws)
    fa.Hip.sync()
    return out.download(q.size, np.uint16)


@pytest.mark.parametrize("nseq,lo,hi,Hq,Hkv,d", [(6, 1, 3000, 40, 8, 128), (16, 256, 4096, 40, 8, 128),
                                                 (5, 17, 700, 14, 2, 64),
                                                 (4, 6000, 40000, 10, 2, 128)])  # 47..128 splits: general merge
def test_paged_matches_contiguous(gpu, oracle, nseq, lo, hi, Hq, Hkv, d):
    fa = gpu
    rng = np.random.default_rng(nseq * 1000 + hi)
    kv_dim = Hkv * d
    lens = [int(x) for x in rng.integers(lo, hi + 1, nseq)]
    max_seq = max(lens) + 5
    seqs, table, k_pool, v_pool = build_paged(rng, lens, kv_dim, max_seq)
    q = f16(rng, (nseq, Hq * d))
    dq = fa.DeviceBuffer.from_array(q)
    dk, dv = fa.DeviceBuffer.from_array(k_pool), fa.DeviceBuffer.from_array(v_pool)
    dt = fa.DeviceBuffer.from_array(table)
    dl = fa.DeviceBuffer.from_array(np.array(lens, np.int32))
    out = fa.DeviceBuffer(q.nbytes)
    ws = fa.DeviceBuffer(fa.pagedWorkspaceBytes(nseq, Hq, max_seq))
    fa.decodeWorkspaceInit(ws)
    fa.launchPagedDecodeAttention(dq, dk, dv, out, dt, table.shape[1], dl, nseq, max_seq, Hq, Hkv, d, ws)
    fa.Hip.sync()
    got = out.download((nseq, Hq * d), np.uint16)
    for b, S in enumerate(lens):
        kc, vc = seqs[b]
        cont = contiguous_decode(fa, q[b], kc, vc, S, Hq, Hkv, d, max_seq)
        assert np.array_equal(got[b], cont), f"seq {b} (S={S}) differs from the contiguous result"
        assert_close(as_f32(got[b]), oracle.decode(q[b], kc, vc, S, Hq, Hkv, d), f"seq {b} S={S}")


def test_config5_exact_draw(gpu, oracle):
    """benchmark config 5 exactly as bench.py draws it (seed 5): 16 sequences with S ~ U[256,
    16384] (sum 117,916), 16-token pages at a seeded permutation of the pool; the one-launch
    paged step (append at S-1 + decode) against the contiguous step of every sequence, bit
    for bit, and the oracle."""
    fa = gpu
    B, Hq, Hkv, d, max_seq = 16, 40, 8, 128, 16384
    kv_dim = Hkv * d
    rng = np.random.default_rng(5)
    lens = rng.integers(256, 16384 + 1, B).astype(np.int32)
    assert int(lens.sum()) == 117916
    nblk = [(int(s) + PAGE - 1) // PAGE for s in lens]
    perm = rng.permutation(sum(nblk)).astype(np.int32)
    data = np.random.default_rng(55)
    table = np.full((B, max_seq // PAGE), -1, np.int32)
    k_pool = np.zeros((sum(nblk), PAGE, kv_dim), np.uint16)
    v_pool = np.zeros_like(k_pool)
    seqs, at = [], 0
    for b, S in enumerate(lens):
        kc, vc = f16(data, (int(S), kv_dim)), f16(data, (int(S), kv_dim))
        seqs.append((kc, vc))
        for j in range(nblk[b]):
            table[b, j] = perm[at]
            rows = slice(j * PAGE, min(int(S), (j + 1) * PAGE))
            k_pool[perm[at], :rows.stop - rows.start] = kc[rows]
            v_pool[perm[at], :rows.stop - rows.start] = vc[rows]
            at += 1
    q, kn, vn = f16(data, (B, Hq * d)), f16(data, (B, kv_dim)), f16(data, (B, kv_dim))
    rope = fa.rope_table_host(max_seq, d, 1e6)
    drope = fa.DeviceBuffer.from_array(rope)
    dq, dk, dv = (fa.DeviceBuffer.from_array(a) for a in (q, kn, vn))
    dkp, dvp = fa.DeviceBuffer.from_array(k_pool), fa.DeviceBuffer.from_array(v_pool)
    dt, dl = fa.DeviceBuffer.from_array(table), fa.DeviceBuffer.from_array(lens)
    out = fa.DeviceBuffer(q.nbytes)
    ws = fa.DeviceBuffer(fa.pagedWorkspaceBytes(B, Hq, max_seq))
    fa.decodeWorkspaceInit(ws)
    fa.pagedDecodeStep(dq, dk, dv, dkp, dvp, out, dt, table.shape[1], dl, B, max_seq, Hq, Hkv, d, drope, 1, ws)
    fa.Hip.sync()
    got = out.download((B, Hq * d), np.uint16)
    for b, S in enumerate(int(x) for x in lens):
        kc, vc = seqs[b]
        # the contiguous one-launch step over the same rows (its row S-1 is overwritten by the append)
        c = {n: fa.DeviceBuffer.from_array(a) for n, a in dict(q=q[b:b + 1], k=kn[b:b + 1], v=vn[b:b + 1], kc=kc,
                                                                 vc=vc).items()}
        cout = fa.DeviceBuffer(Hq * d * 2)
        cws = fa.DeviceBuffer(fa.splitAttentionWorkspaceBytes(Hq, max_seq))
        fa.decodeWorkspaceInit(cws)
        cpos = fa.DeviceBuffer.from_array(np.array([S - 1], np.int32))
        fa.decodeStep(c["q"], c["k"], c["v"], c["kc"], c["vc"], cout, cpos, 0, max_seq, Hq, Hkv,
                      d, drope, 1, cws)
        fa.Hip.sync()
        assert np.array_equal(got[b], cout.download(Hq * d, np.uint16)), f"seq {b} (S={S}) differs from the contiguous step"
        if b % 5 == 0:  # the oracle at a third of the sequences (the contiguous step is checked against it elsewhere)
            qr, kr = q[b:b + 1].copy(), kn[b:b + 1].copy()
            kc2, vc2 = kc.copy(), vc.copy()
            oracle.rope_append(qr, kr, vn[b:b + 1], kc2, vc2, rope, S - 1, Hq, Hkv, d, 1)
            assert_close(as_f32(got[b]), oracle.decode(qr[0], kc2, vc2, S, Hq, Hkv, d), f"config 5 seq {b} S={S}")


def test_paged_append_then_decode(gpu, oracle):
    """Append one token per sequence through the block table, then decode; caches bit-exact."""
    fa = gpu
    Hq, Hkv, d, nseq = 40, 8, 128, 7
    kv_dim = Hkv * d
    rng = np.random.default_rng(77)
    lens = [int(x) for x in rng.integers(1, 900, nseq)]   # lengths AFTER the append
    max_seq = 1024
    seqs, table, k_pool, v_pool = build_paged(rng, lens, kv_dim, max_seq)
    q = f16(rng, (nseq, Hq * d))
    k = f16(rng, (nseq, kv_dim))
    v = f16(rng, (nseq, kv_dim))
    rope = fa.rope_table_host(max_seq, d, 1e6)
    bufs = {n: fa.DeviceBuffer.from_array(a) for n, a in
            dict(q=q, k=k, v=v, kp=k_pool, vp=v_pool, t=table, l=np.array(lens, np.int32), r=rope).items()}
    fa.pagedRopeStoreKv(bufs["q"], bufs["k"], bufs["v"], bufs["kp"], bufs["vp"], bufs["t"], table.shape[1],
                        bufs["l"], nseq, d, Hq, Hkv, max_seq, bufs["r"], 1)
    out = fa.DeviceBuffer(q.nbytes)
    ws = fa.DeviceBuffer(fa.pagedWorkspaceBytes(nseq, Hq, max_seq))
    fa.decodeWorkspaceInit(ws)
    fa.launchPagedDecodeAttention(bufs["q"], bufs["kp"], bufs["vp"], out, bufs["t"], table.shape[1], bufs["l"],
                                  nseq, max_seq, Hq, Hkv, d, ws)
    fa.Hip.sync()
    got_kp = bufs["kp"].download(k_pool.shape, np.uint16)
    got_vp = bufs["vp"].download(v_pool.shape, np.uint16)
    got = as_f32(out.download((nseq, Hq * d), np.uint16))
    for b, S in enumerate(lens):
        kc, vc = seqs[b]
        qb, kb = q[b:b + 1].copy(), k[b:b + 1].copy()
        oracle.rope_append(qb, kb, v[b:b + 1], kc, vc, rope, S - 1, Hq, Hkv, d, 1)
        pos = S - 1
        phys = table[b, pos // PAGE]
        assert np.array_equal(got_kp[phys, pos % PAGE], kc[pos]), f"k row seq {b}"
        assert np.array_equal(got_vp[phys, pos % PAGE], vc[pos]), f"v row seq {b}"
        assert_close(got[b], oracle.decode(qb[0], kc, vc, S, Hq, Hkv, d), f"paged seq {b}")


def test_paged_empty_sequence(gpu, oracle):
    """A sequence of length 0 in the batch: no positions, so its output is zero (the combine
    rule out = L > 1e-12 ? O / L : 0); the other sequences are unaffected."""
    fa = gpu
    Hq, Hkv, d = 40, 8, 128
    rng = np.random.default_rng(404)
    lens = [0, 5, 1000, 0]
    max_seq = 1024
    seqs, table, k_pool, v_pool = build_paged(rng, lens, Hkv * d, max_seq)
    q = f16(rng, (len(lens), Hq * d))
    dq = fa.DeviceBuffer.from_array(q)
    dk, dv = fa.DeviceBuffer.from_array(k_pool), fa.DeviceBuffer.from_array(v_pool)
    dt = fa.DeviceBuffer.from_array(table)
    dl = fa.DeviceBuffer.from_array(np.array(lens, np.int32))
    out = fa.DeviceBuffer(q.nbytes)
    out.fill_bytes(0xFF)
    ws = fa.DeviceBuffer(fa.pagedWorkspaceBytes(len(lens), Hq, max_seq))
    fa.decodeWorkspaceInit(ws)
    fa.launchPagedDecodeAttention(dq, dk, dv, out, dt, table.shape[1], dl, len(lens), max_seq, Hq, Hkv, d, ws)
    fa.Hip.sync()
    got = out.download((len(lens), Hq * d), np.uint16)
    for b, S in enumerate(lens):
        if S == 0:
            assert (got[b] == 0).all(), f"empty sequence {b}: output not zero"
        else:
            kc, vc = seqs[b]
            assert np.array_equal(got[b], contiguous_decode(fa, q[b], kc, vc, S, Hq, Hkv, d, max_seq)), f"seq {b}"


def test_merge_forms_share_a_workspace(gpu):
    """The two fused-merge forms advance each group's arrival counter and its base together.
    Two paged calls on one workspace (same batch, so the same counter slots) alternate: long
    sequences, whose grid exceeds the resident workgroups (the last arriver merges), and the
    same sequences cut to 200 positions with max_seq_len 256 (192 workgroups: fixed mergers).
    Every call is bit-identical to the same call on a fresh workspace, and the short one to
    the separate merge kernel of the contiguous path."""
    fa = gpu
    Hq, Hkv, d, nseq = 40, 8, 128, 12
    rng = np.random.default_rng(77)
    kv_dim = Hkv * d
    lens = [int(x) for x in rng.integers(3000, 9000, nseq)]
    short = [min(s, 200) for s in lens]
    max_seq = 9000
    seqs, table, k_pool, v_pool = build_paged(rng, lens, kv_dim, max_seq)
    q = f16(rng, (nseq, Hq * d))
    dq = fa.DeviceBuffer.from_array(q)
    dk, dv = fa.DeviceBuffer.from_array(k_pool), fa.DeviceBuffer.from_array(v_pool)
    dt = fa.DeviceBuffer.from_array(table)
    dl_long = fa.DeviceBuffer.from_array(np.array(lens, np.int32))
    dl_short = fa.DeviceBuffer.from_array(np.array(short, np.int32))

    def paged(ws, dl, ms):
        out = fa.DeviceBuffer(q.nbytes)
        fa.launchPagedDecodeAttention(dq, dk, dv, out, dt, table.shape[1], dl, nseq, ms, Hq, Hkv, d, ws)
        fa.Hip.sync()
        return out.download((nseq, Hq * d), np.uint16)

    def fresh():
        ws = fa.DeviceBuffer(fa.pagedWorkspaceBytes(nseq, Hq, max_seq))
        fa.decodeWorkspaceInit(ws)
        return ws

    ref_long = paged(fresh(), dl_long, max_seq)
    ref_short = paged(fresh(), dl_short, 256)
    for b in (0, nseq - 1):
        kc, vc = seqs[b]
        assert np.array_equal(ref_short[b], contiguous_decode(fa, q[b], kc[:short[b]], vc[:short[b]], short[b], Hq, Hkv,
                                                             d, 256)), f"seq {b}: paged short call differs"
    shared = fresh()
    for it in range(4):
        assert np.array_equal(paged(shared, dl_long, max_seq), ref_long), f"long call {it} on the shared workspace differs"
        assert np.array_equal(paged(shared, dl_short, 256), ref_short), f"short call {it} on the shared workspace differs"


def test_paged_long_splits_block_table_fallback(gpu, oracle):
    """Splits of more than 64 tiles per wave (4480 positions at S = 140000 with 8 kv heads)
    take the page numbers past the 64th tile from the block table directly instead of from
    the per-wave page list: bit-identical to the contiguous path and close to the oracle."""
    fa = gpu
    Hq, Hkv, d = 8, 8, 128
    rng = np.random.default_rng(140)
    kv_dim = Hkv * d
    lens = [140000, 131200]
    max_seq = 140000
    seqs, table, k_pool, v_pool = build_paged(rng, lens, kv_dim, max_seq)
    q = f16(rng, (len(lens), Hq * d))
    dq = fa.DeviceBuffer.from_array(q)
    dk, dv = fa.DeviceBuffer.from_array(k_pool), fa.DeviceBuffer.from_array(v_pool)
    del k_pool, v_pool
    dt = fa.DeviceBuffer.from_array(table)
    dl = fa.DeviceBuffer.from_array(np.array(lens, np.int32))
    out = fa.DeviceBuffer(q.nbytes)
    ws = fa.DeviceBuffer(fa.pagedWorkspaceBytes(len(lens), Hq, max_seq))
    fa.decodeWorkspaceInit(ws)
    fa.launchPagedDecodeAttention(dq, dk, dv, out, dt, table.shape[1], dl, len(lens), max_seq, Hq, Hkv, d, ws)
    fa.Hip.sync()
    got = out.download((len(lens), Hq * d), np.uint16)
    dk.free()
    dv.free()
    for b, S in enumerate(lens):
        kc, vc = seqs[b]
        assert np.array_equal(got[b], contiguous_decode(fa, q[b], kc, vc, S, Hq, Hkv, d, max_seq)), f"seq {b} S={S}"
        assert_close(as_f32(got[b]), oracle.decode(q[b], kc, vc, S, Hq, Hkv, d), f"seq {b} S={S}")
