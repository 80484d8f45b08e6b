"""GPU parity of decode attention (launchDecodeAttention / DevPos / Split) vs the CPU oracle.

Mirrors tests/kernels/test_decode_attention.cu of the reference (Qwen2.5-32B
shapes 40q/8kv d128, q = 2*N(0,1), seq in {1, 2, 17, 255, 256, 257, 300, 1000,
2048}, single-pass and split-K with host and device lengths) and adds the
the benchmark configs and the closed-form cases of the softmax rules.
"""
import numpy as np
import pytest

from fa_helpers import as_f32, assert_close, f16

pytestmark = pytest.mark.gpu


class Cache:
    """Device copies of q and one layer's K/V cache plus output/workspace buffers."""

    def __init__(self, fa, q, kc, vc, Hq, max_ctx):
        self.fa = fa
        self.q = fa.DeviceBuffer.from_array(q)
        self.k = fa.DeviceBuffer.from_array(kc)
        self.v = fa.DeviceBuffer.from_array(vc)
        self.out = fa.DeviceBuffer(q.nbytes)
        self.pos = fa.DeviceBuffer(4)
        self.ws = fa.DeviceBuffer(fa.splitAttentionWorkspaceBytes(Hq, max_ctx))
        self.wsf = fa.DeviceBuffer(fa.splitAttentionWorkspaceBytes(Hq, max_ctx))
        fa.decodeWorkspaceInit(self.wsf)
        self.n = q.size

    def result(self):
        self.fa.Hip.sync()
        return as_f32(self.out.download(self.n, np.uint16))


def run_all_paths(fa, c, S, Hq, Hkv, d, max_ctx):
    """Single-pass, split with host length, split with device position."""
    outs = {}
    c.out.fill_bytes(0xFF)
    fa.launchDecodeAttention(c.q, c.k, c.v, c.out, S, Hq, Hkv, d)
    outs["single"] = c.result()
    c.pos.upload(np.array([S - 1], np.int32))
    c.out.fill_bytes(0xFF)
    fa.launchDecodeAttentionDevPos(c.q, c.k, c.v, c.out, c.pos, max_ctx, Hq, Hkv, d)
    outs["single_devpos"] = c.result()
    for mode in ("host", "devpos"):
        c.out.fill_bytes(0xFF)
        fa.launchDecodeAttentionSplit(c.q, c.k, c.v, c.out, S if mode == "host" else 0,
                                      c.pos if mode == "devpos" else None, max_ctx, Hq, Hkv, d, c.ws)
        outs["split_" + mode] = c.result()
        c.out.fill_bytes(0xFF)
        fa.launchDecodeAttentionFused(c.q, c.k, c.v, c.out, S if mode == "host" else 0,
                                      c.pos if mode == "devpos" else None, max_ctx, Hq, Hkv, d, c.wsf)
        outs["fused_" + mode] = c.result()
        assert np.array_equal(outs["fused_" + mode], outs["split_" + mode]), "fused merge differs from merge kernel"
    return outs


def test_reference_decode_matrix(gpu, oracle):
    """test_decode_attention.cu:43-97: 40/8 heads, d128, max_ctx 2048, q = 2 N(0,1)."""
    fa = gpu
    Hq, Hkv, d, max_ctx = 40, 8, 128, 2048
    rng = np.random.default_rng(7)
    kc = f16(rng, (max_ctx, Hkv * d))
    vc = f16(rng, (max_ctx, Hkv * d))
    q = f16(rng, Hq * d, 2.0)
    c = Cache(fa, q, kc, vc, Hq, max_ctx)
    for S in (1, 2, 17, 255, 256, 257, 300, 1000, 2048):
        print(f"decode S={S}", flush=True)
        ref = oracle.decode(q, kc, vc, S, Hq, Hkv, d)
        for name, got in run_all_paths(fa, c, S, Hq, Hkv, d, max_ctx).items():
            assert_close(got, ref, f"S={S} {name}")


@pytest.mark.parametrize("Hq,Hkv,d,S", [(14, 2, 64, 513), (32, 8, 128, 4096), (40, 8, 128, 5000),
                                         (16, 16, 128, 333), (64, 8, 128, 777), (40, 2, 128, 1500),
                                         (48, 1, 64, 900)])
def test_shapes(gpu, oracle, Hq, Hkv, d, S):
    """GQA groups 1..48 (head blocks of 16), d 64/128, odd lengths."""
    fa = gpu
    rng = np.random.default_rng(S)
    max_ctx = S + 37
    kc = f16(rng, (max_ctx, Hkv * d))
    vc = f16(rng, (max_ctx, Hkv * d))
    q = f16(rng, Hq * d)
    c = Cache(fa, q, kc, vc, Hq, max_ctx)
    ref = oracle.decode(q, kc, vc, S, Hq, Hkv, d)
    for name, got in run_all_paths(fa, c, S, Hq, Hkv, d, max_ctx).items():
        assert_close(got, ref, f"{Hq}/{Hkv} d{d} S={S} {name}")


@pytest.mark.parametrize("S", [1024, 4096, 8192])
def test_config2_outliers(gpu, oracle, S):
    """benchmark config 2: 32q/8kv d128, ~1% of cached K rows x30 (FP32-safe softmax)."""
    fa = gpu
    Hq, Hkv, d = 32, 8, 128
    rng = np.random.default_rng(1000 + S)
    kf = rng.standard_normal((S, Hkv * d), dtype=np.float32)
    rows = rng.choice(S, size=max(1, S // 100), replace=False)
    kf[rows] *= 30.0
    kc = kf.astype(np.float16).view(np.uint16)
    vc = f16(rng, (S, Hkv * d))
    q = f16(rng, Hq * d)
    c = Cache(fa, q, kc, vc, Hq, S)
    ref = oracle.decode(q, kc, vc, S, Hq, Hkv, d)
    c.pos.upload(np.array([S - 1], np.int32))
    fa.launchDecodeAttentionSplit(c.q, c.k, c.v, c.out, 0, c.pos, S, Hq, Hkv, d, c.ws)
    assert_close(c.result(), ref, f"config2 S={S}")


@pytest.mark.parametrize("S", [16384, 32768])
def test_config3_long_context(gpu, oracle, S):
    """benchmark config 3 (headline): 40q/8kv d128 at 16k / 32k, split-K + LSE merge."""
    fa = gpu
    Hq, Hkv, d = 40, 8, 128
    rng = np.random.default_rng(S)
    kc = f16(rng, (S, Hkv * d))
    vc = f16(rng, (S, Hkv * d))
    q = f16(rng, Hq * d)
    c = Cache(fa, q, kc, vc, Hq, S)
    ref = oracle.decode(q, kc, vc, S, Hq, Hkv, d)
    c.pos.upload(np.array([S - 1], np.int32))
    fa.launchDecodeAttentionSplit(c.q, c.k, c.v, c.out, 0, c.pos, S, Hq, Hkv, d, c.ws)
    split = c.result()
    assert_close(split, ref, f"config3 S={S}")
    for rep in range(3):  # counters re-arm: repeated fused calls give the same bits
        fa.launchDecodeAttentionFused(c.q, c.k, c.v, c.out, 0, c.pos, S, Hq, Hkv, d, c.wsf)
        assert np.array_equal(c.result(), split), f"fused call {rep}"


@pytest.mark.parametrize("S", [131072, 100003])
def test_max_context_many_splits(gpu, oracle, S):
    """A 128k-position cache (Qwen2.5's longest context) with 2 kv heads of group 5: 128 splits
    of 1024 positions at S = 131072 and 112 of 896 at S = 100003, so the merge takes its
    general path (more than 32 splits). Host-length, device-position and fused-merge calls
    give the same bits, and match the oracle."""
    fa = gpu
    Hq, Hkv, d, max_ctx = 10, 2, 128, 131072
    rng = np.random.default_rng(S)
    kc = f16(rng, (S, Hkv * d))
    vc = f16(rng, (S, Hkv * d))
    q = f16(rng, Hq * d)
    c = Cache(fa, q, kc, vc, Hq, max_ctx)
    ref = oracle.decode(q, kc, vc, S, Hq, Hkv, d)
    fa.launchDecodeAttentionSplit(c.q, c.k, c.v, c.out, S, None, max_ctx, Hq, Hkv, d, c.ws)
    host = c.result()
    assert_close(host, ref, f"max context S={S}")
    c.pos.upload(np.array([S - 1], np.int32))
    c.out.fill_bytes(0xFF)
    fa.launchDecodeAttentionSplit(c.q, c.k, c.v, c.out, 0, c.pos, max_ctx, Hq, Hkv, d, c.ws)
    assert np.array_equal(c.result(), host), "device-position call differs from host-length call"
    for rep in range(2):
        c.out.fill_bytes(0xFF)
        fa.launchDecodeAttentionFused(c.q, c.k, c.v, c.out, 0, c.pos, max_ctx, Hq, Hkv, d, c.wsf)
        assert np.array_equal(c.result(), host), f"fused call {rep} differs from the merge kernel"


def test_closed_forms(gpu, oracle):
    """Exact cases fixed by the softmax rules (cpu_ops.cpp:45-83)."""
    fa = gpu
    Hq, Hkv, d, S = 8, 2, 128, 300
    rng = np.random.default_rng(3)
    kc = f16(rng, (S, Hkv * d))
    vc = f16(rng, (S, Hkv * d))
    q = f16(rng, Hq * d)
    c = Cache(fa, q, kc, vc, Hq, S)
    # S = 1: weight 1 -> out = v0 exactly
    for name, got in run_all_paths(fa, c, 1, Hq, Hkv, d, S).items():
        exp = np.concatenate([as_f32(vc[0, (h // 4) * d:(h // 4 + 1) * d]) for h in range(Hq)])
        assert np.array_equal(got, exp), name
    # identical K rows -> uniform weights -> mean of V
    kc2 = np.tile(kc[:1], (S, 1))
    c.k.upload(kc2)
    ref = oracle.decode(q, kc2, vc, S, Hq, Hkv, d)
    for name, got in run_all_paths(fa, c, S, Hq, Hkv, d, S).items():
        assert_close(got, ref, f"equal rows {name}")
    # one dominant key (score margin > 50): out = v of that row exactly
    kd = np.zeros((S, Hkv * d), np.float32)
    qd = np.zeros(Hq * d, np.float32)
    qd[:] = 1.0
    kd[123, :] = 8.0   # q.k/sqrt(d) = 8*128/11.3 = 90.5 vs 0 elsewhere
    kc3 = kd.astype(np.float16).view(np.uint16)
    q3 = qd.astype(np.float16).view(np.uint16)
    c.k.upload(kc3)
    c.q.upload(q3)
    for name, got in run_all_paths(fa, c, S, Hq, Hkv, d, S).items():
        exp = np.concatenate([as_f32(vc[123, (h // 4) * d:(h // 4 + 1) * d]) for h in range(Hq)])
        assert np.array_equal(got, exp), name
    # NaN in a K row: that score becomes -1e30 (excluded)
    kc4 = kc.copy()
    kc4[50, :] = np.float16(np.nan).view(np.uint16)
    c.k.upload(kc4)
    c.q.upload(q)
    ref = oracle.decode(q, kc4, vc, S, Hq, Hkv, d)
    for name, got in run_all_paths(fa, c, S, Hq, Hkv, d, S).items():
        assert_close(got, ref, f"nan row {name}")
    # all-NaN q: every score -1e30 -> uniform weights -> mean of V
    qn = np.full(Hq * d, np.float16(np.nan).view(np.uint16), np.uint16)
    c.k.upload(kc)
    c.q.upload(qn)
    ref = oracle.decode(qn, kc, vc, S, Hq, Hkv, d)
    for name, got in run_all_paths(fa, c, S, Hq, Hkv, d, S).items():
        assert_close(got, ref, f"nan q {name}")


def test_gqa_heads_share_kv(gpu):
    """Query heads of one group given the same q give identical outputs."""
    fa = gpu
    Hq, Hkv, d, S = 40, 8, 128, 3000
    rng = np.random.default_rng(11)
    kc = f16(rng, (S, Hkv * d))
    vc = f16(rng, (S, Hkv * d))
    q1 = f16(rng, (Hkv, 1, d))
    q = np.repeat(q1, Hq // Hkv, axis=1).reshape(-1)
    c = Cache(fa, q, kc, vc, Hq, S)
    fa.launchDecodeAttentionSplit(c.q, c.k, c.v, c.out, S, None, S, Hq, Hkv, d, c.ws)
    got = c.result().reshape(Hkv, Hq // Hkv, d)
    assert np.array_equal(got, np.repeat(got[:, :1], Hq // Hkv, axis=1))


@pytest.mark.parametrize("Hq,Hkv,d,S", [(40, 8, 128, 1000),
                                         (14, 2, 64, 513),
                                         (10, 2, 128, 60000)])  # 118 splits: general merge
def test_int8_decode(gpu, oracle, Hq, Hkv, d, S):
    """int8 KV with fp16 scales per 32 values (k_scale/v_scale path); the fused merge gives
    the merge kernel's bits."""
    fa = gpu
    rng = np.random.default_rng(5 + S)
    k8 = rng.integers(-127, 128, (S, Hkv * d), dtype=np.int8)
    v8 = rng.integers(-127, 128, (S, Hkv * d), dtype=np.int8)
    ks = rng.uniform(0.005, 0.03, (S, Hkv * d // 32)).astype(np.float16).view(np.uint16)
    vs = rng.uniform(0.005, 0.03, (S, Hkv * d // 32)).astype(np.float16).view(np.uint16)
    q = f16(rng, Hq * d)
    ref = oracle.decode_q8(q, k8, ks, v8, vs, S, Hq, Hkv, d)
    dq = fa.DeviceBuffer.from_array(q)
    dk, dv = fa.DeviceBuffer.from_array(k8), fa.DeviceBuffer.from_array(v8)
    dks, dvs = fa.DeviceBuffer.from_array(ks), fa.DeviceBuffer.from_array(vs)
    out = fa.DeviceBuffer(q.nbytes)
    ws = fa.DeviceBuffer(fa.splitAttentionWorkspaceBytes(Hq, S))
    fa.launchDecodeAttentionSplit(dq, dk, dv, out, S, None, S, Hq, Hkv, d, ws, k_scale=dks, v_scale=dvs)
    fa.Hip.sync()
    split = out.download(Hq * d, np.uint16)
    assert_close(as_f32(split), ref, "int8 decode")
    wsf = fa.DeviceBuffer(fa.splitAttentionWorkspaceBytes(Hq, S))
    fa.decodeWorkspaceInit(wsf)
    out.fill_bytes(0xFF)
    fa.launchDecodeAttentionFused(dq, dk, dv, out, S, None, S, Hq, Hkv, d, wsf, k_scale=dks, v_scale=dvs)
    fa.Hip.sync()
    assert np.array_equal(out.download(Hq * d, np.uint16), split), "int8 fused merge differs from the merge kernel"
