"""The decode placement and merge forms give the same bits.

friday_attn_set_decode_form switches, for the process, how fp16 contiguous decode launches
place their workgroups (groups' splits on one XCD, or one split's groups on one XCD) and how
the fused merge collects the splits (device-coherent counter, or flag words in the XCD's
L2). The merge arithmetic and the split partition are the same in every form, so the
fused decode and the decode step must give identical output, rotated q and cache rows in
each form, on fresh and on reused workspaces, when forms alternate on one workspace, and
when the split count changes between launches (the flags' tags must not match an earlier
launch's). The oracle pins the default form elsewhere (test_gpu_decode.py, test_gpu_step.py)."""
import numpy as np
import pytest

from fa_helpers import f16

import os

# Built while GPU use was closed: the form has not run on a GPU yet, so the round's
# `pytest -m gpu -x` skips it (a first failure would hide every later test) unless
# FRIDAY_ATTN_TEST_NEW_FORMS=1 asks for it.
pytestmark = [pytest.mark.gpu,
              pytest.mark.skipif(os.environ.get("FRIDAY_ATTN_TEST_NEW_FORMS") != "1",
                                 reason="the XCD-local merge and split-major forms has not yet run on a GPU (FRIDAY_ATTN_TEST_NEW_FORMS=1 runs it)")]

FORMS = ((0, 0), (1, 0), (0, 1))  # (local_merge, split_major)


@pytest.fixture
def forms(gpu):
    yield gpu
    gpu.setDecodeForm(-1, -1, -1)


def fused(fa, q, kc, vc, S, Hq, Hkv, d, max_ctx, ws, pos):
    out = fa.DeviceBuffer(q.nbytes)
    out.fill_bytes(0xFF)
    pos.upload(np.array([S - 1], np.int32))
    fa.launchDecodeAttentionFused(q, kc, vc, out, 0, pos, max_ctx, Hq, Hkv, d, ws)
    fa.Hip.sync()
    r = out.download(Hq * d, np.uint16)
    out.free()
    return r


@pytest.mark.parametrize("Hq,Hkv,d", [(40, 8, 128), (32, 8, 128), (16, 16, 128), (64, 8, 64), (14, 2, 64)])
def test_fused_forms_identical(forms, Hq, Hkv, d):
    fa = forms
    max_ctx = 8192
    rng = np.random.default_rng(Hq * 100 + Hkv)
    kv_dim = Hkv * d
    q = fa.DeviceBuffer.from_array(f16(rng, (1, Hq * d), 2.0))
    kc = fa.DeviceBuffer.from_array(f16(rng, (max_ctx, kv_dim)))
    vc = fa.DeviceBuffer.from_array(f16(rng, (max_ctx, kv_dim)))
    pos = fa.DeviceBuffer(4)
    lengths = (8192, 8192, 300, 4097, 129, 8000, 8000)
    want = {}
    fa.setDecodeForm(0, 0, 0)
    ws0 = fa.DeviceBuffer(fa.splitAttentionWorkspaceBytes(Hq, max_ctx))
    fa.decodeWorkspaceInit(ws0)
    for S in set(lengths):
        want[S] = fused(fa, q, kc, vc, S, Hq, Hkv, d, max_ctx, ws0, pos)
    shared = fa.DeviceBuffer(fa.splitAttentionWorkspaceBytes(Hq, max_ctx))
    fa.decodeWorkspaceInit(shared)
    for form in FORMS:
        fa.setDecodeForm(*form, 0)
        own = fa.DeviceBuffer(fa.splitAttentionWorkspaceBytes(Hq, max_ctx))
        fa.decodeWorkspaceInit(own)
        print(f"[forms] fused {Hq}q/{Hkv}kv d{d} form {form}", flush=True)
        for i, S in enumerate(lengths):
            assert np.array_equal(fused(fa, q, kc, vc, S, Hq, Hkv, d, max_ctx, own, pos), want[S]), \
                f"form {form} S={S} (launch {i}, own workspace)"
            # forms alternate on one workspace: each launch leaves counter and base in step
            assert np.array_equal(fused(fa, q, kc, vc, S, Hq, Hkv, d, max_ctx, shared, pos), want[S]), \
                f"form {form} S={S} (launch {i}, shared workspace)"
        assert fa.decodeWorkspaceStatus(own) == fa.FA_OK
        own.free()
    assert fa.decodeWorkspaceStatus(shared) == fa.FA_OK


def test_step_forms_identical(forms):
    """The decode step (RoPE, append, attention, merge, rotated q written back) at the
    headline shape, 32k and a shorter context: output, q and both cache rows per form."""
    fa = forms
    Hq, Hkv, d, max_ctx = 40, 8, 128, 32768
    rng = np.random.default_rng(11)
    kv_dim = Hkv * d
    host = dict(q=f16(rng, (1, Hq * d), 2.0), k=f16(rng, (1, kv_dim)), v=f16(rng, (1, kv_dim)),
                kc=f16(rng, (max_ctx, kv_dim)), vc=f16(rng, (max_ctx, kv_dim)))
    dt = fa.DeviceBuffer.from_array(fa.rope_table_host(max_ctx, d, 1e6))
    dpos = fa.DeviceBuffer(4)
    ws = fa.DeviceBuffer(fa.splitAttentionWorkspaceBytes(Hq, max_ctx))
    fa.decodeWorkspaceInit(ws)
    b = {n: fa.DeviceBuffer.from_array(a) for n, a in host.items()}
    out = fa.DeviceBuffer(host["q"].nbytes)
    res = {}
    for S in (32768, 5000):
        for form in FORMS:
            print(f"[forms] step S={S} form {form}", flush=True)
            fa.setDecodeForm(*form, 0)
            for n, a in host.items():
                b[n].upload(a)
            dpos.upload(np.array([S - 1], np.int32))
            out.fill_bytes(0xFF)
            fa.decodeStep(b["q"], b["k"], b["v"], b["kc"], b["vc"], out, dpos, 0, max_ctx, Hq, Hkv, d, dt, 1, ws)
            fa.Hip.sync()
            row = slice(S - 1, S)
            got = (out.download(Hq * d, np.uint16), b["q"].download(host["q"].shape, np.uint16),
                   b["kc"].download(host["kc"].shape, np.uint16)[row], b["vc"].download(host["vc"].shape, np.uint16)[row])
            if S not in res:
                res[S] = got
            else:
                for name, x, y in zip(("out", "q", "k row", "v row"), got, res[S]):
                    assert np.array_equal(x, y), f"step S={S} form {form}: {name} differs from form (0, 0)"
    assert fa.decodeWorkspaceStatus(ws) == fa.FA_OK

