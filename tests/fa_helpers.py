"""Shared helpers of the test suite: seeded inputs and the parity metrics."""
import numpy as np

# Attention tolerance of the KV-cache path (fp16 KV, fp32 accumulation):
# |got - ref| <= ATOL + RTOL * |ref| elementwise, plus the reference kernel
# tests' own rel-L2 < 1e-3 (test_decode_attention.cu:70-77).
ATOL = 2e-3
RTOL = 1e-2
REL_L2 = 1e-3


def f16(rng, shape, scale=1.0):
    """N(0, scale^2) rounded to fp16, returned as uint16 bits."""
    return (rng.standard_normal(shape, dtype=np.float32) * np.float32(scale)).astype(np.float16).view(np.uint16)


def bf16(rng, shape, scale=1.0):
    """N(0, scale^2) rounded to nearest even bf16, returned as uint16 bits."""
    x = (rng.standard_normal(shape, dtype=np.float32) * np.float32(scale)).view(np.uint32)
    return ((x + np.uint32(0x7FFF) + ((x >> 16) & np.uint32(1))) >> 16).astype(np.uint16)


def bf16_as_f32(bits):
    return (np.asarray(bits, np.uint16).astype(np.uint32) << 16).view(np.float32)


def as_f32(bits):
    return np.asarray(bits).view(np.float16).astype(np.float32)


def metrics(got, ref):
    got = np.asarray(got, np.float64).ravel()
    ref = np.asarray(ref, np.float64).ravel()
    d = got - ref
    den = np.sqrt(np.sum(ref * ref))
    rel = np.sqrt(np.sum(d * d)) / (den if den > 0 else 1e-300)
    return float(np.max(np.abs(d))) if d.size else 0.0, float(rel)


def assert_close(got, ref, what="", atol=ATOL, rtol=RTOL, rel_l2=REL_L2):
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    assert np.all(np.isfinite(got)), f"{what}: non-finite output"
    mx, rel = metrics(got, ref)
    bad = np.abs(got - ref) > atol + rtol * np.abs(ref)
    assert not bad.any(), (f"{what}: {bad.sum()} elements outside atol={atol} rtol={rtol}; max_abs={mx:.3e} "
                           f"rel_l2={rel:.3e}")
    assert rel < rel_l2, f"{what}: rel_l2 {rel:.3e} >= {rel_l2}"
    return mx, rel


# ---- prefill projection GEMM (K-quant weights x int8 activations) ----
# kind codes of friday_hpc::Q8Kind (hpc_k_quants.h:39); block bytes, values per block
# and the byte offsets of the fp16 scale fields of each GGML block layout
KQ_KINDS = {1: ("Q2_K", 84, 256, (80, 82)), 2: ("Q3_K", 110, 256, (108,)), 3: ("Q4_K", 144, 256, (0, 2)),
            4: ("Q5_K", 176, 256, (0, 2)), 5: ("Q6_K", 210, 256, (208,)), 6: ("Q8_0", 34, 32, (0,))}


def kq_random_weights(rng, kind, N, K):
    """Random K-quant rows as the reference GEMM test builds them (test_prefill_gemm.cu:25-36):
    uniform random bytes, then fp16 scales in [1e-3, 1e-2] written over the scale fields."""
    _, bb, vals, offs = KQ_KINDS[kind]
    w = rng.integers(0, 256, size=(N, K // vals, bb), dtype=np.uint8)
    for off in offs:
        s = rng.uniform(1e-3, 1e-2, size=(N, K // vals)).astype(np.float16)
        w[:, :, off:off + 2] = s.view(np.uint8).reshape(N, K // vals, 2)
    return w.reshape(N, -1)


# The reference GEMM test's bar (test_prefill_gemm.cu:111-129): rel-L2 < 1e-3 and the largest
# |difference| below 1e-2 of the reference's RMS, no non-finite outputs.
GEMM_REL_L2 = 1e-3
GEMM_MAX_REL = 1e-2


def assert_gemm_close(got, ref, what=""):
    got = np.asarray(got, np.float64).ravel()
    ref = np.asarray(ref, np.float64).ravel()
    assert np.all(np.isfinite(got)), f"{what}: non-finite output"
    d = got - ref
    den = np.sum(ref * ref)
    rel = np.sqrt(np.sum(d * d) / (den if den > 0 else 1e-300))
    max_rel = np.max(np.abs(d)) / np.sqrt(den / ref.size + 1e-30)
    assert rel < GEMM_REL_L2 and max_rel < GEMM_MAX_REL, f"{what}: rel_l2 {rel:.2e} max_rel {max_rel:.2e}"
    return rel, max_rel

