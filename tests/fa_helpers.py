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
