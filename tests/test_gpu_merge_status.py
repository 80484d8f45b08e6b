"""The fused merge's bounded wait reports its failure instead of merging partial results.

The host forces the failure: it presets every group's base in the workspace ahead of its
arrival counter, so the count the mergers wait for can never arrive. Every merger then
waits out its bound (1 s of the real-time clock, so the launch takes about that long),
sets the workspace's sticky error word and writes nothing: the output keeps the bytes it
had. friday_attn_decode_workspace_status reports FA_ERR_TIMEOUT until
friday_attn_decode_workspace_init clears it, after which the same call gives the same
bits as on a fresh workspace. No kernel faults or hangs: every wave exits."""
import numpy as np
import pytest

from fa_helpers import f16

pytestmark = pytest.mark.gpu

COUNTER_SLOT = 256  # bytes between the groups' counter slots; the base sits 128 B into a slot


def test_merge_timeout_is_reported_and_recoverable(gpu):
    fa = gpu
    Hq, Hkv, d, S = 40, 8, 128, 4096  # 32 splits per group, fixed mergers (one workgroup per CU)
    rng = np.random.default_rng(5)
    kv_dim = Hkv * d
    q, kc, vc = f16(rng, (1, Hq * d)), f16(rng, (S, kv_dim)), f16(rng, (S, kv_dim))
    dq, dk, dv = (fa.DeviceBuffer.from_array(a) for a in (q, kc, vc))
    out = fa.DeviceBuffer(Hq * d * 2)
    ws = fa.DeviceBuffer(fa.splitAttentionWorkspaceBytes(Hq, S))

    fresh = fa.DeviceBuffer(ws.nbytes)
    fa.decodeWorkspaceInit(fresh)
    fa.launchDecodeAttentionFused(dq, dk, dv, out, S, None, S, Hq, Hkv, d, fresh)
    fa.Hip.sync()
    want = out.download(Hq * d, np.uint16)
    assert fa.decodeWorkspaceStatus(fresh) == fa.FA_OK

    fa.decodeWorkspaceInit(ws)
    fa.Hip.sync()
    for g in range(Hkv):  # one group per kv head (G = 5 <= 16)
        ws.upload(np.array([1000], np.uint32), offset=g * COUNTER_SLOT + 128)
    out.fill_bytes(0xFF)
    print(f"[merge-timeout] forced wait on {Hkv} groups, S={S}", flush=True)
    fa.launchDecodeAttentionFused(dq, dk, dv, out, S, None, S, Hq, Hkv, d, ws)
    fa.Hip.sync()
    assert fa.decodeWorkspaceStatus(ws) == fa.FA_ERR_TIMEOUT
    assert "initialise" in fa.load().friday_attn_last_error().decode()
    assert np.all(out.download(Hq * d, np.uint16) == 0xFFFF), "a merger that gave up wrote output"

    fa.decodeWorkspaceInit(ws)
    assert fa.decodeWorkspaceStatus(ws) == fa.FA_OK
    fa.launchDecodeAttentionFused(dq, dk, dv, out, S, None, S, Hq, Hkv, d, ws)
    fa.Hip.sync()
    assert np.array_equal(out.download(Hq * d, np.uint16), want)
    assert fa.decodeWorkspaceStatus(ws) == fa.FA_OK
