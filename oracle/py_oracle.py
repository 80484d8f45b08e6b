"""ctypes bindings of the CPU oracle (TEST INFRASTRUCTURE ONLY).

Loaded by tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg.
The product library never imports this module.

  Oracle   -> oracle/lib/libfa_oracle.so      (C restatement, fa_oracle.c)
  RefCpu   -> oracle/_ref/libfriday_cpu_ref.so (reference cpu_ops.cpp et al.,
              compiled from the reference sources; absent on machines without
              /root/reference at build time)
"""
from __future__ import annotations

import ctypes as C
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ORACLE_SO = os.path.join(HERE, "lib", "libfa_oracle.so")
REF_SO = os.path.join(HERE, "_ref", "libfriday_cpu_ref.so")

_u16p = np.ctypeslib.ndpointer(np.uint16, flags="C_CONTIGUOUS")
_i8p = np.ctypeslib.ndpointer(np.int8, flags="C_CONTIGUOUS")
_f32p = np.ctypeslib.ndpointer(np.float32, flags="C_CONTIGUOUS")
_f64p = np.ctypeslib.ndpointer(np.float64, flags="C_CONTIGUOUS")
_i32p = np.ctypeslib.ndpointer(np.int32, flags="C_CONTIGUOUS")
_u8p = np.ctypeslib.ndpointer(np.uint8, flags="C_CONTIGUOUS")
_i = C.c_int


def _f16bits(a) -> np.ndarray:
    a = np.ascontiguousarray(a)
    if a.dtype == np.float16:
        return a.view(np.uint16)
    assert a.dtype == np.uint16, a.dtype
    return a


class Oracle:
    def __init__(self, path: str = ORACLE_SO):
        if not os.path.exists(path):
            raise FileNotFoundError(f"{path} missing: run `make -C oracle`")
        L = self.lib = C.CDLL(path)
        L.or_half_to_float.restype = C.c_float
        L.or_half_to_float.argtypes = [C.c_uint16]
        L.or_float_to_half.restype = C.c_uint16
        L.or_float_to_half.argtypes = [C.c_float]
        L.or_round_to_half.restype = C.c_float
        L.or_round_to_half.argtypes = [C.c_float]
        L.or_halves_to_floats.argtypes = [_u16p, _f32p, C.c_size_t]
        L.or_floats_to_halves.argtypes = [_f32p, _u16p, C.c_size_t]
        L.or_rope_table.argtypes = [_f32p, _i, _i, C.c_float, C.c_void_p]
        L.or_rope_append.argtypes = [_u16p, _u16p, _u16p, C.c_void_p, C.c_void_p, _f32p, _i, _i, _i, _i, _i, _i]
        L.or_store_kv_q8.argtypes = [_u16p, _u16p, _i8p, _u16p, _i8p, _u16p, _i, _i, _i]
        L.or_decode_attention.argtypes = [_u16p, _u16p, _u16p, _f32p, _i, _i, _i, _i, _i]
        L.or_decode_attention_q8.argtypes = [_u16p, _i8p, _u16p, _i8p, _u16p, _f32p, _i, _i, _i, _i]
        L.or_decode_attention_f64.argtypes = [_u16p, _u16p, _u16p, _f64p, _i, _i, _i, _i, _i]
        L.or_decode_attention_split.argtypes = [_u16p, _u16p, _u16p, _f32p, _i, _i, _i, _i, _i]
        L.or_lse_merge.argtypes = [_f32p, _f32p, _f32p, _i, _i, _f32p]
        L.or_prefill_attention.argtypes = [_u16p, _u16p, _u16p, _f32p, _i, _i, _i, _i, _i]
        L.or_bf16_to_float.restype = C.c_float
        L.or_bf16_to_float.argtypes = [C.c_uint16]
        L.or_float_to_bf16.restype = C.c_uint16
        L.or_float_to_bf16.argtypes = [C.c_float]
        L.or_round_to_bf16.restype = C.c_float
        L.or_round_to_bf16.argtypes = [C.c_float]
        L.or_prefill_attention_bf16.argtypes = [_u16p, _u16p, _u16p, _f32p, _i, _i, _i, _i, _i]
        L.or_prefill_attention_q8.argtypes = [_u16p, _i8p, _u16p, _i8p, _u16p, _f32p, _i, _i, _i, _i, _i]
        L.or_paged_gather.argtypes = [_u16p, _i32p, _i, _i, _i, _u16p]
        L.or_prefill_widen.argtypes = [C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p, _i, _i, _i, _i, _f32p, _f32p]
        L.or_prefill_rows_f32.argtypes = [_u16p, _f32p, _f32p, _i, _f32p, _i, _i, _i, _i, _i, _i]
        L.or_q8_row_bytes.restype = C.c_size_t
        L.or_q8_row_bytes.argtypes = [_i, _i]
        L.or_quantize_q8_rows.argtypes = [_u16p, _i, _i, _i8p, _f32p]
        L.or_kq_block.restype = _i
        L.or_kq_block.argtypes = [_i, _u8p, _i, _i32p, _f32p, _f32p]
        L.or_dequant_row.argtypes = [_i, _u8p, _i, _f32p]
        L.or_gemm_q8.argtypes = [_i, _u8p, _i8p, _f32p, _i, _i, _i, C.c_void_p, C.c_void_p, _i, C.c_void_p,
                                 C.c_void_p]

    # fp16
    def h2f(self, h) -> np.ndarray:
        h = _f16bits(h)
        out = np.empty(h.shape, np.float32)
        self.lib.or_halves_to_floats(h.ravel(), out.ravel(), h.size)
        return out

    def f2h(self, f) -> np.ndarray:
        f = np.ascontiguousarray(f, np.float32)
        out = np.empty(f.shape, np.uint16)
        self.lib.or_floats_to_halves(f.ravel(), out.ravel(), f.size)
        return out

    def round_to_half(self, x: float) -> float:
        return self.lib.or_round_to_half(x)

    # rope
    def rope_table(self, max_pos, head_dim, base, freq_factors=None) -> np.ndarray:
        cs = np.empty((max_pos, head_dim // 2, 2), np.float32)
        ff = None
        if freq_factors is not None:
            ff = np.ascontiguousarray(freq_factors, np.float32)
        self.lib.or_rope_table(cs.ravel(), max_pos, head_dim, base, None if ff is None else ff.ctypes.data)
        return cs

    def rope_append(self, q, k, v, k_cache, v_cache, cs, pos0, Hq, Hkv, d, neox):
        """q [T][Hq*d], k/v [T][Hkv*d] uint16 (modified in place); caches [max_ctx][Hkv*d] or None."""
        T = q.shape[0]
        self.lib.or_rope_append(q, k, v, None if k_cache is None else k_cache.ctypes.data,
                                None if v_cache is None else v_cache.ctypes.data, cs.ravel(), pos0, T, Hq, Hkv, d,
                                int(neox))

    def store_kv_q8(self, k, v, k8, ks, v8, vs, pos0, kv_dim):
        T = k.shape[0]
        self.lib.or_store_kv_q8(_f16bits(k), _f16bits(v), k8, ks, v8, vs, pos0, T, kv_dim)

    # attention
    def decode(self, q, kc, vc, S, Hq, Hkv, d, kv_stride=None) -> np.ndarray:
        out = np.empty(Hq * d, np.float32)
        self.lib.or_decode_attention(_f16bits(q).ravel(), _f16bits(kc).ravel(), _f16bits(vc).ravel(), out, S, Hq,
                                     Hkv, d, kv_stride or Hkv * d)
        return out

    def decode_q8(self, q, k8, ks, v8, vs, S, Hq, Hkv, d) -> np.ndarray:
        out = np.empty(Hq * d, np.float32)
        self.lib.or_decode_attention_q8(_f16bits(q).ravel(), k8.ravel(), _f16bits(ks).ravel(), v8.ravel(),
                                        _f16bits(vs).ravel(), out, S, Hq, Hkv, d)
        return out

    def decode_f64(self, q, kc, vc, S, Hq, Hkv, d) -> np.ndarray:
        out = np.empty(Hq * d, np.float64)
        self.lib.or_decode_attention_f64(_f16bits(q).ravel(), _f16bits(kc).ravel(), _f16bits(vc).ravel(), out, S,
                                         Hq, Hkv, d, Hkv * d)
        return out

    def decode_split(self, q, kc, vc, S, Hq, Hkv, d, nsplit) -> np.ndarray:
        out = np.empty(Hq * d, np.float32)
        self.lib.or_decode_attention_split(_f16bits(q).ravel(), _f16bits(kc).ravel(), _f16bits(vc).ravel(), out, S,
                                           Hq, Hkv, d, nsplit)
        return out

    def lse_merge(self, part_o, part_m, part_l) -> np.ndarray:
        nsp, d = part_o.shape
        out = np.empty(d, np.float32)
        self.lib.or_lse_merge(np.ascontiguousarray(part_o, np.float32).ravel(),
                              np.ascontiguousarray(part_m, np.float32), np.ascontiguousarray(part_l, np.float32),
                              nsp, d, out)
        return out

    def prefill(self, q, kc, vc, T, p0, Hq, Hkv, d) -> np.ndarray:
        out = np.empty((T, Hq * d), np.float32)
        self.lib.or_prefill_attention(_f16bits(q).ravel(), _f16bits(kc).ravel(), _f16bits(vc).ravel(), out.ravel(),
                                      T, p0, Hq, Hkv, d)
        return out

    def prefill_bf16(self, q, kc, vc, T, p0, Hq, Hkv, d) -> np.ndarray:
        """q / kc / vc: bf16 bit patterns (uint16 arrays)."""
        out = np.empty((T, Hq * d), np.float32)
        u16 = lambda a: np.ascontiguousarray(a, np.uint16).ravel()
        self.lib.or_prefill_attention_bf16(u16(q), u16(kc), u16(vc), out.ravel(), T, p0, Hq, Hkv, d)
        return out

    def prefill_q8(self, q, k8, ks, v8, vs, T, p0, Hq, Hkv, d) -> np.ndarray:
        out = np.empty((T, Hq * d), np.float32)
        self.lib.or_prefill_attention_q8(_f16bits(q).ravel(), k8.ravel(), _f16bits(ks).ravel(), v8.ravel(),
                                         _f16bits(vs).ravel(), out.ravel(), T, p0, Hq, Hkv, d)
        return out

    def prefill_all(self, q, kc, vc, T, p0, Hq, Hkv, d, ks=None, vs=None, bf16=False, block=16,
                    workers=16) -> np.ndarray:
        """Every row of prefill / prefill_q8 (ks, vs given: int8 codes kc / vc) / prefill_bf16, bit
        for bit, by the blocked evaluator (or_prefill_rows_f32) on `workers` threads over row
        blocks (the C calls release the GIL)."""
        from concurrent.futures import ThreadPoolExecutor

        S = p0 + T
        kind = 1 if ks is not None else (2 if bf16 else 0)
        kt = np.empty(S * Hkv * d, np.float32)
        vf = np.empty(S * Hkv * d, np.float32)
        if kind == 1:
            kk, vv = np.ascontiguousarray(kc[:S], np.int8), np.ascontiguousarray(vc[:S], np.int8)
            kss, vss = _f16bits(ks[:S]).ravel(), _f16bits(vs[:S]).ravel()
            self.lib.or_prefill_widen(kk.ctypes.data, kss.ctypes.data, vv.ctypes.data, vss.ctypes.data, 1, S, Hkv, d,
                                      kt, vf)
        else:
            kk = np.ascontiguousarray(kc[:S], np.uint16).ravel()
            vv = np.ascontiguousarray(vc[:S], np.uint16).ravel()
            self.lib.or_prefill_widen(kk.ctypes.data, None, vv.ctypes.data, None, kind, S, Hkv, d, kt, vf)
        qq = np.ascontiguousarray(q, np.uint16).reshape(T, Hq * d)
        out = np.empty((T, Hq * d), np.float32)

        def rows(t0):
            n = min(block, T - t0)
            self.lib.or_prefill_rows_f32(qq[t0:t0 + n].ravel(), kt, vf, S, out[t0:t0 + n].ravel(), n, p0 + t0, Hq,
                                         Hkv, d, int(bf16))

        starts = list(range(0, T, block))
        with ThreadPoolExecutor(max_workers=max(1, min(workers, len(starts)))) as ex:
            list(ex.map(rows, starts))
        return out

    def paged_gather(self, pool, block_table, S, page, kv_dim) -> np.ndarray:
        dst = np.empty((S, kv_dim), np.uint16)
        self.lib.or_paged_gather(_f16bits(pool).ravel(), np.ascontiguousarray(block_table, np.int32), S, page,
                                 kv_dim, dst.ravel())
        return dst


    # prefill projection GEMM (kind = friday_hpc::Q8Kind code: 1 Q2_K .. 5 Q6_K, 6 Q8_0)
    def q8_row_bytes(self, kind, K) -> int:
        return int(self.lib.or_q8_row_bytes(kind, K))

    def quantize_q8_rows(self, x):
        x = _f16bits(x)
        rows, K = x.shape
        xq = np.empty((rows, K), np.int8)
        xd = np.empty((rows, K // 32), np.float32)
        self.lib.or_quantize_q8_rows(x.ravel(), rows, K, xq.ravel(), xd.ravel())
        return xq, xd

    def kq_block(self, kind, row, blk):
        q = np.empty(32, np.int32)
        ws = np.empty(2, np.float32)
        wm = np.empty(2, np.float32)
        assert self.lib.or_kq_block(kind, np.ascontiguousarray(row, np.uint8), blk, q, ws, wm) == 0
        return q, ws, wm

    def dequant_row(self, kind, row, K) -> np.ndarray:
        out = np.empty(K, np.float32)
        self.lib.or_dequant_row(kind, np.ascontiguousarray(row, np.uint8), K, out)
        return out

    def gemm_q8(self, kind, W, xq, xd, T, K, N, bias=None, res=None, ldy=None):
        """Returns (Y fp16 bits [T][ldy], fp32 sums before the epilogue [T][N])."""
        ldy = N if ldy is None else ldy
        W = np.ascontiguousarray(W, np.uint8)
        b = None if bias is None else np.ascontiguousarray(bias, np.float32)
        r = None if res is None else _f16bits(res).copy()
        Y = np.zeros((T, ldy), np.uint16)
        raw = np.empty((T, N), np.float32)
        self.lib.or_gemm_q8(kind, W.ravel(), np.ascontiguousarray(xq, np.int8).ravel(),
                            np.ascontiguousarray(xd, np.float32).ravel(), T, K, N,
                            None if b is None else b.ctypes.data, None if r is None else r.ctypes.data, ldy,
                            Y.ctypes.data, raw.ctypes.data)
        return Y, raw


class RefCpu:
    """The reference's own CPU functions (cpu_ops.cpp), compiled from source."""

    def __init__(self, path: str = REF_SO):
        if not os.path.exists(path):
            raise FileNotFoundError(path)
        L = self.lib = C.CDLL(path)
        L.ref_half_to_float.restype = C.c_float
        L.ref_half_to_float.argtypes = [C.c_uint16]
        L.ref_float_to_half.restype = C.c_uint16
        L.ref_float_to_half.argtypes = [C.c_float]
        L.ref_round_to_half.argtypes = [_f32p, _i]
        L.ref_rope.argtypes = [_f32p, _f32p, _i, _i, _i, _i, C.c_float, _i, C.c_void_p]
        L.ref_decode_attention.argtypes = [_f32p, _f32p, _f32p, _f32p, _i, _i, _i, _i, _i]
        L.ref_pool_size.restype = _i
        L.ref_pool_size.argtypes = [_i]
        L.ref_quantize_activation.argtypes = [_f32p, _i, _i8p, _f32p]
        L.ref_dequantize_row.restype = _i
        L.ref_dequantize_row.argtypes = [C.c_char_p, _u8p, _f32p, _i]
        L.ref_gemv_rows_scalar.argtypes = [C.c_char_p, _u8p, _f32p, _i, _f32p, _i, _i]
        L.ref_gemv_rows.argtypes = [C.c_char_p, _u8p, _f32p, _i, _f32p, _i, _i]

    def rope(self, q, k, head_dim, nq, nk, pos, base, neox, freq_factors=None):
        ff = None if freq_factors is None else np.ascontiguousarray(freq_factors, np.float32)
        self.lib.ref_rope(q, k, head_dim, nq, nk, pos, base, int(neox), None if ff is None else ff.ctypes.data)

    def decode(self, q, kc, vc, seq, Hq, Hkv, d, threads=1) -> np.ndarray:
        out = np.empty(Hq * d, np.float32)
        self.lib.ref_decode_attention(np.ascontiguousarray(q, np.float32).ravel(),
                                      np.ascontiguousarray(kc, np.float32).ravel(),
                                      np.ascontiguousarray(vc, np.float32).ravel(), out, seq, Hq, Hkv, d, threads)
        return out

    def quantize_activation(self, x):
        x = np.ascontiguousarray(x, np.float32)
        K = x.size
        q = np.empty(K, np.int8)
        d = np.empty(K // 32, np.float32)
        self.lib.ref_quantize_activation(x, K, q, d)
        return q, d

    def dequantize_row(self, dtype, row, K) -> np.ndarray:
        out = np.empty(K, np.float32)
        assert self.lib.ref_dequantize_row(dtype.encode(), np.ascontiguousarray(row, np.uint8), out, K) == 1
        return out

    def gemv_rows_scalar(self, dtype, W, x, K, N) -> np.ndarray:
        y = np.zeros(N, np.float32)
        self.lib.ref_gemv_rows_scalar(dtype.encode(), np.ascontiguousarray(W, np.uint8).ravel(),
                                      np.ascontiguousarray(x, np.float32), K, y, 0, N)
        return y

    def gemv_rows(self, dtype, W, x, K, r0, r1, y=None) -> np.ndarray:
        y = np.zeros(r1, np.float32) if y is None else y
        self.lib.ref_gemv_rows(dtype.encode(), np.ascontiguousarray(W, np.uint8).ravel(),
                               np.ascontiguousarray(x, np.float32), K, y, r0, r1)
        return y


def ref_available() -> bool:
    return os.path.exists(REF_SO)
