"""friday_attn_decode_step_noalloc (the entry point that allocates nothing: its split
counters and partials live in the library's per-GPU device scratch) against
friday_attn_decode_step with a caller workspace: cache rows, rotated q and output bit for
bit, on calls in a row with smaller inputs and other head counts. Argument checks need no GPU."""
import ctypes as C

import numpy as np
import pytest

from fa_helpers import f16


def run_pair(fa, Hq, Hkv, d, S, max_ctx, seed):
    rng = np.random.default_rng(seed)
    kv_dim = Hkv * d
    kc, vc = f16(rng, (max_ctx, kv_dim)), f16(rng, (max_ctx, kv_dim))
    q, k, v = f16(rng, (1, Hq * d), 2.0), f16(rng, (1, kv_dim)), f16(rng, (1, kv_dim))
    dt = fa.DeviceBuffer.from_array(fa.rope_table_host(max_ctx, d, 1e6))
    dpos = fa.DeviceBuffer.from_array(np.array([S - 1], np.int32))
    res = []
    for noalloc in (False, True):
        b = {n: fa.DeviceBuffer.from_array(a) for n, a in dict(q=q, k=k, v=v, kc=kc, vc=vc).items()}
        out = fa.DeviceBuffer(q.nbytes)
        out.fill_bytes(0xFF)
        if noalloc:
            fa.decodeStepNoAlloc(b["q"], b["k"], b["v"], b["kc"], b["vc"], out, dpos, 0, max_ctx, Hq, Hkv, d, dt, 1)
        else:
            ws = fa.DeviceBuffer(fa.splitAttentionWorkspaceBytes(Hq, max_ctx))
            fa.decodeWorkspaceInit(ws)
            fa.decodeStep(b["q"], b["k"], b["v"], b["kc"], b["vc"], out, dpos, 0, max_ctx, Hq, Hkv, d, dt, 1, ws)
        fa.Hip.sync()
        res.append((out.download(Hq * d, np.uint16), b["q"].download(q.shape, np.uint16),
                    b["kc"].download(kc.shape, np.uint16), b["vc"].download(vc.shape, np.uint16)))
    for name, x, y in zip(("out", "q", "k cache", "v cache"), res[0], res[1]):
        assert np.array_equal(x, y), f"{name} differs (Hq={Hq} Hkv={Hkv} d={d} S={S})"


@pytest.mark.gpu
def test_noalloc_matches_workspace_step(gpu):
    # headline shape at 32k (32 splits, distributed merge), then a smaller call that
    # reuses the scratch the first one left behind; then a model with one query head per
    # kv head (32 counter slots, more than the 14 heads of the call before it) and the
    # headline shape again: calls with different head counts share the scratch
    run_pair(gpu, 40, 8, 128, 32768, 32768, seed=1)
    run_pair(gpu, 14, 2, 64, 513, 1024, seed=2)
    run_pair(gpu, 32, 32, 128, 4096, 4096, seed=3)
    run_pair(gpu, 40, 8, 128, 2000, 4096, seed=4)


def test_noalloc_argument_checks(fa):
    L = fa.load()
    FAKE = 0x1000
    # more than the 4 MiB scratch: 8192 query heads (counters alone take 2 MiB)
    rc = L.friday_attn_decode_step_noalloc(FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, 0, 4096, 8192, 8, 128, FAKE, 1,
                                           None)
    assert rc == fa.FA_ERR_WORKSPACE
    assert "4194304" in fa.load().friday_attn_last_error().decode()
    rc = L.friday_attn_decode_step_noalloc(FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, None, 5000, 4096, 40, 8, 128, FAKE, 1,
                                           None)
    assert rc == fa.FA_ERR_INVALID
    rc = L.friday_attn_decode_step_noalloc(FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, 0, 4096, 40, 8, 96, FAKE, 1, None)
    assert rc == fa.FA_ERR_UNSUPPORTED


def _inputs(fa, Hq, Hkv, d, max_ctx, seed):
    rng = np.random.default_rng(seed)
    kv_dim = Hkv * d
    return dict(q=f16(rng, (1, Hq * d), 2.0), k=f16(rng, (1, kv_dim)), v=f16(rng, (1, kv_dim)),
                kc=f16(rng, (max_ctx, kv_dim)), vc=f16(rng, (max_ctx, kv_dim)))


def _reference_step(fa, host, Hq, Hkv, d, max_ctx, dt, dpos):
    b = {n: fa.DeviceBuffer.from_array(a) for n, a in host.items()}
    out = fa.DeviceBuffer(host["q"].nbytes)
    ws = fa.DeviceBuffer(fa.splitAttentionWorkspaceBytes(Hq, max_ctx))
    fa.decodeWorkspaceInit(ws)
    fa.decodeStep(b["q"], b["k"], b["v"], b["kc"], b["vc"], out, dpos, 0, max_ctx, Hq, Hkv, d, dt, 1, ws)
    fa.Hip.sync()
    return out.download(Hq * d, np.uint16), b["q"].download(host["q"].shape, np.uint16)


@pytest.mark.gpu
def test_noalloc_on_created_streams(gpu):
    """Calls on two created streams in turn (each synchronised before the next), against the
    workspace step: the scratch is not tied to the stream of the first call."""
    fa = gpu
    Hq, Hkv, d, max_ctx, S = 40, 8, 128, 8192, 8000
    dt = fa.DeviceBuffer.from_array(fa.rope_table_host(max_ctx, d, 1e6))
    dpos = fa.DeviceBuffer.from_array(np.array([S - 1], np.int32))
    for i, st in enumerate((fa.Stream(), fa.Stream(), fa.Stream())):
        host = _inputs(fa, Hq, Hkv, d, max_ctx, seed=20 + i)
        ref_out, ref_q = _reference_step(fa, host, Hq, Hkv, d, max_ctx, dt, dpos)
        b = {n: fa.DeviceBuffer.from_array(a) for n, a in host.items()}
        out = fa.DeviceBuffer(host["q"].nbytes)
        fa.decodeStepNoAlloc(b["q"], b["k"], b["v"], b["kc"], b["vc"], out, dpos, 0, max_ctx, Hq, Hkv, d, dt, 1,
                             stream=st.s)
        st.synchronize()
        assert np.array_equal(out.download(Hq * d, np.uint16), ref_out), f"stream {i}: output"
        assert np.array_equal(b["q"].download(host["q"].shape, np.uint16), ref_q), f"stream {i}: rotated q"
        st.destroy()


@pytest.mark.gpu
def test_noalloc_captured_and_replayed(gpu):
    """A noalloc call captured into a HIP graph, replayed four times with the program's own
    eager work (fresh inputs copied in, synchronisation) between replays: every replay equals
    the workspace step on the same inputs, bit for bit."""
    fa = gpu
    Hq, Hkv, d, max_ctx = 40, 8, 128, 4096
    dt = fa.DeviceBuffer.from_array(fa.rope_table_host(max_ctx, d, 1e6))
    dpos = fa.DeviceBuffer(4)
    host = _inputs(fa, Hq, Hkv, d, max_ctx, seed=31)
    b = {n: fa.DeviceBuffer.from_array(a) for n, a in host.items()}
    out = fa.DeviceBuffer(host["q"].nbytes)
    st = fa.Stream()
    dpos.upload(np.array([100], np.int32))
    graph = fa.Graph(st, lambda: fa.decodeStepNoAlloc(b["q"], b["k"], b["v"], b["kc"], b["vc"], out, dpos, 0,
                                                      max_ctx, Hq, Hkv, d, dt, 1, stream=st.s))
    try:
        for rep, S in enumerate((4096, 4096, 1500, 257)):
            dpos.upload(np.array([S - 1], np.int32))
            for n, a in host.items():  # the step rotates q and writes row S-1 in place
                b[n].upload(a)
            out.fill_bytes(0xFF)
            graph.launch()
            st.synchronize()
            ref_out, ref_q = _reference_step(fa, host, Hq, Hkv, d, max_ctx, dt, dpos)
            assert np.array_equal(out.download(Hq * d, np.uint16), ref_out), f"replay {rep} (S={S}): output"
            assert np.array_equal(b["q"].download(host["q"].shape, np.uint16), ref_q), f"replay {rep}: q"
    finally:
        graph.destroy()
        st.destroy()
