"""HIP graph capture of the per-layer decode path, replayed at advancing positions.

The reference captures its decode layers into a CUDA graph once and replays it for every
token, the position coming from the device int d_pos_ (transformer.cpp:1457-1483); inside a
layer it runs RoPE + append + split attention (:1046-1051), quantizeQ8 of the attention
output and the O-projection gemvQ8 with the residual in place (:1057-1059). Here the same
layer is captured once (friday_attn_decode_step, friday_quantize_q8_rows,
friday_gemv_q8) and replayed for several tokens, with eager host work (new inputs, d_pos
update, synchronisation) between the replays; every replay must equal the same calls run
eagerly on a twin set of buffers, bit for bit (cache rows, attention output, residual).
The int8-KV variant (friday_attn_decode_step_q8) is replayed the same way.
"""
import numpy as np
import pytest

from fa_helpers import f16, kq_random_weights

pytestmark = pytest.mark.gpu

Hq, Hkv, d, MAX_CTX, P0 = 40, 8, 128, 2048, 1000
H = Hq * d  # model width of the O-projection (K = N = 5120, Qwen2.5-32B)


def make_layer(fa, rng, q8):
    kv = Hkv * d
    st = {}
    if q8:
        st["kc"] = fa.DeviceBuffer.from_array(rng.integers(-127, 128, (MAX_CTX, kv), dtype=np.int8))
        st["vc"] = fa.DeviceBuffer.from_array(rng.integers(-127, 128, (MAX_CTX, kv), dtype=np.int8))
        sc = rng.uniform(0.005, 0.03, (MAX_CTX, kv // 32)).astype(np.float16).view(np.uint16)
        st["ks"] = fa.DeviceBuffer.from_array(sc)
        st["vs"] = fa.DeviceBuffer.from_array(sc[::-1].copy())
    else:
        st["kc"] = fa.DeviceBuffer.from_array(f16(rng, (MAX_CTX, kv)))
        st["vc"] = fa.DeviceBuffer.from_array(f16(rng, (MAX_CTX, kv)))
    st["q"], st["k"], st["v"] = fa.DeviceBuffer(H * 2), fa.DeviceBuffer(kv * 2), fa.DeviceBuffer(kv * 2)
    st["ctx"] = fa.DeviceBuffer(H * 2)
    st["x"] = fa.DeviceBuffer.from_array(f16(rng, H))  # residual stream, updated in place
    st["xq"], st["xd"] = fa.DeviceBuffer(H), fa.DeviceBuffer(H // 32 * 4)
    st["pos"] = fa.DeviceBuffer.from_array(np.array([P0], np.int32))
    ws_bytes = fa.splitAttentionWorkspaceBytes(Hq, MAX_CTX)
    st["ws"] = fa.DeviceBuffer(ws_bytes)
    fa.decodeWorkspaceInit(st["ws"])
    return st


def layer_calls(fa, st, W, rope, q8, stream):
    if q8:
        fa.decodeStepQ8(st["q"], st["k"], st["v"], st["kc"], st["ks"], st["vc"], st["vs"], st["ctx"], st["pos"], 0,
                        MAX_CTX, Hq, Hkv, d, rope, 1, st["ws"], stream=stream)
    else:
        fa.decodeStep(st["q"], st["k"], st["v"], st["kc"], st["vc"], st["ctx"], st["pos"], 0, MAX_CTX, Hq, Hkv, d,
                      rope, 1, st["ws"], stream=stream)
    fa.quantizeQ8Rows(st["ctx"], 1, H, st["xq"], st["xd"], stream=stream)
    fa.gemvQ8(fa.Q4_K, W, st["xq"], st["xd"], H, H, st["x"], stream=stream, res=st["x"])


@pytest.mark.parametrize("q8", [False, True])
def test_decode_layer_graph_replay(gpu, q8):
    fa = gpu
    rng = np.random.default_rng(1457 + q8)
    W = fa.DeviceBuffer.from_array(kq_random_weights(rng, fa.Q4_K, H, H))
    rope = fa.DeviceBuffer(fa.rope_table_bytes(MAX_CTX, d))
    fa.rope_table_upload(rope, MAX_CTX, d, 1e6)
    seed = int(rng.integers(1 << 30))
    g_st = make_layer(fa, np.random.default_rng(seed), q8)  # replayed
    e_st = make_layer(fa, np.random.default_rng(seed), q8)  # eager twin (same initial contents)
    fa.Hip.sync()
    stream = fa.Stream()
    graph = fa.Graph(stream, lambda: layer_calls(fa, g_st, W, rope, q8, stream.s))
    kvb = Hkv * d * (1 if q8 else 2)
    for step in range(4):
        pos = P0 + step
        q, k, v = f16(rng, H), f16(rng, Hkv * d), f16(rng, Hkv * d)
        for st in (g_st, e_st):
            st["q"].upload(q)
            st["k"].upload(k)
            st["v"].upload(v)
            st["pos"].upload(np.array([pos], np.int32))
        graph.launch()
        stream.synchronize()
        layer_calls(fa, e_st, W, rope, q8, None)
        fa.Hip.sync()
        for name, n, dt in (("ctx", H, np.uint16), ("x", H, np.uint16), ("q", H, np.uint16)):
            a, b = g_st[name].download(n, dt), e_st[name].download(n, dt)
            assert np.array_equal(a, b), f"replay {step}: {name} differs"
        a = g_st["kc"].download(kvb, np.uint8, offset=pos * kvb)
        b = e_st["kc"].download(kvb, np.uint8, offset=pos * kvb)
        assert np.array_equal(a, b), f"replay {step}: appended k row differs"
        assert a.any(), "the appended row was written"
