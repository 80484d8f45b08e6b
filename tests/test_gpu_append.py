"""GPU parity of the KV append (ropeStoreKvKernel / ropeKernel / storeKvQ8Kernel semantics).

Bar: bit-exact. Rotated q and k (in place), the cache rows written, and every
other cache row untouched (canary fill).
"""
import numpy as np
import pytest

from fa_helpers import f16

pytestmark = pytest.mark.gpu

CANARY = 0x7BCD


def run_append(fa, oracle, Hq, Hkv, d, T, pos0, max_ctx, base, neox, ff=None, devpos=True, seed=0):
    rng = np.random.default_rng(seed)
    q = f16(rng, (T, Hq * d), 3.0)
    k = f16(rng, (T, Hkv * d), 3.0)
    v = f16(rng, (T, Hkv * d))
    k_orig = k.copy()
    kc = np.full((max_ctx, Hkv * d), CANARY, np.uint16)
    vc = kc.copy()
    table = fa.rope_table_host(max_ctx, d, base, ff)
    assert np.array_equal(table.view(np.uint32), oracle.rope_table(max_ctx, d, base, ff).view(np.uint32))
    dt = fa.DeviceBuffer(fa.rope_table_bytes(max_ctx, d))
    fa.rope_table_upload(dt, max_ctx, d, base, ff)
    dq, dk, dv = (fa.DeviceBuffer.from_array(a) for a in (q, k, v))
    dkc, dvc = fa.DeviceBuffer.from_array(kc), fa.DeviceBuffer.from_array(vc)
    dpos = fa.DeviceBuffer.from_array(np.array([pos0], np.int32))
    fa.ropeStoreKv(dq, dk, dv, dkc, dvc, dpos if devpos else None, 0 if devpos else pos0, T, d, Hq, Hkv, max_ctx,
                   dt, neox)
    fa.Hip.sync()
    gq, gk = dq.download(q.shape, np.uint16), dk.download(k.shape, np.uint16)
    gkc, gvc = dkc.download(kc.shape, np.uint16), dvc.download(vc.shape, np.uint16)
    oracle.rope_append(q, k, v, kc, vc, table, pos0, Hq, Hkv, d, neox)
    assert np.array_equal(gq, q), "rotated q"
    assert np.array_equal(gk, k), "rotated k"
    assert np.array_equal(gkc, kc), "k cache"
    assert np.array_equal(gvc, vc), "v cache"
    return q, k, kc, k_orig


@pytest.mark.parametrize("Hq,Hkv,d,T,pos0,base,neox", [
    (14, 2, 64, 1, 512, 1e6, 1),       # config 1: Qwen2.5-0.5B, append at 512
    (32, 8, 128, 1, 4095, 5e5, 0),     # config 2 shapes, llama (interleaved) pairs
    (40, 8, 128, 1, 32767, 1e6, 1),    # config 3 shapes, last position of a 32k cache
    (40, 8, 128, 512, 7680, 1e6, 1),   # config 4: prefill chunk append
    (16, 16, 128, 9, 31, 1e4, 0),
    (40, 8, 128, 3, 0, 1e6, 1),
    (8, 2, 64, 4, 100, 1e4, 0),        # d = 64 with interleaved pairs
])
def test_rope_store_kv(gpu, oracle, Hq, Hkv, d, T, pos0, base, neox):
    run_append(gpu, oracle, Hq, Hkv, d, T, pos0, pos0 + T + 5, base, neox, seed=pos0 + T)


def test_host_position_and_freq_factors(gpu, oracle):
    rng = np.random.default_rng(9)
    ff = rng.uniform(1.0, 8.0, 64).astype(np.float32)  # Llama-3 rope_freqs
    run_append(gpu, oracle, 32, 8, 128, 4, 100, 200, 5e5, 0, ff=ff, devpos=False, seed=4)


def test_position_zero_is_identity(gpu, oracle):
    """theta = 0 at pos 0: cos 1, sin 0 -> K stored unchanged."""
    _, _, kc, k_orig = run_append(gpu, oracle, 40, 8, 128, 1, 0, 4, 1e6, 1, seed=2)
    assert np.array_equal(kc[0], k_orig[0])


def test_rotation_only(gpu, oracle):
    """k_layer = v_layer = NULL: ropeKernel semantics (q and k rotated, no cache write)."""
    fa = gpu
    Hq, Hkv, d, max_ctx = 40, 8, 128, 64
    rng = np.random.default_rng(8)
    q, k = f16(rng, (1, Hq * d)), f16(rng, (1, Hkv * d))
    table = fa.rope_table_host(max_ctx, d, 1e6)
    dt = fa.DeviceBuffer.from_array(table)
    dq, dk = fa.DeviceBuffer.from_array(q), fa.DeviceBuffer.from_array(k)
    fa.ropeStoreKv(dq, dk, None, None, None, None, 33, 1, d, Hq, Hkv, max_ctx, dt, 1)
    fa.Hip.sync()
    oracle.rope_append(q, k, k, None, None, table, 33, Hq, Hkv, d, 1)
    assert np.array_equal(dq.download(q.shape, np.uint16), q)
    assert np.array_equal(dk.download(k.shape, np.uint16), k)


def test_nan_and_overflow_rules(gpu, oracle):
    """NaN -> 0 and clamp to +-65504 after the rotation (cuda_math_kernels.cu:393-394)."""
    fa = gpu
    Hq, Hkv, d, max_ctx = 4, 2, 64, 16
    q = np.full((1, Hq * d), np.float16(60000.0).view(np.uint16), np.uint16)
    k = np.full((1, Hkv * d), np.float16(np.nan).view(np.uint16), np.uint16)
    v = np.full((1, Hkv * d), np.float16(1.5).view(np.uint16), np.uint16)
    table = fa.rope_table_host(max_ctx, d, 1e4)
    dt = fa.DeviceBuffer.from_array(table)
    dq, dk, dv = (fa.DeviceBuffer.from_array(a) for a in (q, k, v))
    kc = np.zeros((max_ctx, Hkv * d), np.uint16)
    dkc, dvc = fa.DeviceBuffer.from_array(kc), fa.DeviceBuffer.from_array(kc)
    fa.ropeStoreKv(dq, dk, dv, dkc, dvc, None, 7, 1, d, Hq, Hkv, max_ctx, dt, 1)
    fa.Hip.sync()
    vc = kc.copy()
    oracle.rope_append(q, k, v, kc, vc, table, 7, Hq, Hkv, d, 1)
    assert np.array_equal(dq.download(q.shape, np.uint16), q)
    assert np.array_equal(dkc.download(kc.shape, np.uint16), kc)
    assert (kc[7] == 0).all()  # NaN -> 0
    assert np.abs(q.view(np.float16).astype(np.float32)).max() <= 65504.0


@pytest.mark.parametrize("T,pos0,kv_dim", [(1, 0, 1024), (1, 777, 1024), (37, 5, 1024), (5, 3, 256)])
def test_store_kv_q8(gpu, oracle, T, pos0, kv_dim):
    fa = gpu
    max_ctx = pos0 + T + 3
    rng = np.random.default_rng(T * 31 + pos0)
    k = f16(rng, (T, kv_dim), 2.0)
    v = f16(rng, (T, kv_dim), 0.5)
    k[0, :32] = 0  # all-zero block: dh = 0 -> q = 0
    v[0, 40] = np.float16(np.nan).view(np.uint16)
    k8 = np.full((max_ctx, kv_dim), 99, np.int8)
    v8 = k8.copy()
    ks = np.full((max_ctx, kv_dim // 32), CANARY, np.uint16)
    vs = ks.copy()
    bufs = [fa.DeviceBuffer.from_array(a) for a in (k, v, k8, ks, v8, vs)]
    dpos = fa.DeviceBuffer.from_array(np.array([pos0], np.int32))
    fa.storeKvQ8(bufs[0], bufs[1], bufs[2], bufs[3], bufs[4], bufs[5], dpos, 0, T, kv_dim, max_ctx)
    fa.Hip.sync()
    got = [bufs[i].download(a.shape, a.dtype) for i, a in ((2, k8), (3, ks), (4, v8), (5, vs))]
    oracle.store_kv_q8(k, v, k8, ks, v8, vs, pos0, kv_dim)
    for g, e, name in zip(got, (k8, ks, v8, vs), ("k8", "k_scale", "v8", "v_scale")):
        assert np.array_equal(g, e), name


def test_store_kv_q8_past_cache(gpu, oracle):
    """A device position near the end of the cache: tokens at or beyond max_ctx are skipped,
    the ones before are written, and rows after the cache (a guard region) stay untouched."""
    fa = gpu
    T, pos0, kv_dim, max_ctx, guard = 6, 60, 1024, 63, 5
    rng = np.random.default_rng(63)
    k, v = f16(rng, (T, kv_dim), 2.0), f16(rng, (T, kv_dim))
    k8 = np.full((max_ctx + guard, kv_dim), 99, np.int8)
    v8 = k8.copy()
    ks = np.full((max_ctx + guard, kv_dim // 32), CANARY, np.uint16)
    vs = ks.copy()
    bufs = [fa.DeviceBuffer.from_array(a) for a in (k, v, k8, ks, v8, vs)]
    dpos = fa.DeviceBuffer.from_array(np.array([pos0], np.int32))
    fa.storeKvQ8(bufs[0], bufs[1], bufs[2], bufs[3], bufs[4], bufs[5], dpos, 0, T, kv_dim, max_ctx)
    fa.Hip.sync()
    got = [bufs[i].download(a.shape, a.dtype) for i, a in ((2, k8), (3, ks), (4, v8), (5, vs))]
    n = max_ctx - pos0  # tokens inside the cache
    oracle.store_kv_q8(k[:n], v[:n], k8, ks, v8, vs, pos0, kv_dim)
    for g, e, name in zip(got, (k8, ks, v8, vs), ("k8", "k_scale", "v8", "v_scale")):
        assert np.array_equal(g, e), name
