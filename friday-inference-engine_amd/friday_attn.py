"""Python host mirror of the friday_attn C ABI (include/friday_attn.h).

The reference exposes the path as C++ launchers in namespace friday_attn
(attention_kernels.h:18-50) that throw std::runtime_error on bad input; this
module binds the C ABI with ctypes and mirrors those launchers under the same
names (launchDecodeAttention, launchDecodeAttentionSplit, ...), raising
RuntimeError on a non-zero status. Device memory, copies, streams and events go
straight to the HIP runtime that libfriday_attn.so links (libamdhip64): this is
plumbing for tests and the benchmark, not part of the product.

Loading fails loudly when the library has not been built: there is no CPU
fallback.
"""
from __future__ import annotations

import ctypes as C
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.environ.get("FRIDAY_ATTN_LIB") or os.path.join(HERE, "lib", "libfriday_attn.so")

FA_OK = 0
FA_ERR_INVALID = -1
FA_ERR_UNSUPPORTED = -2
FA_ERR_LAUNCH = -3
FA_ERR_WORKSPACE = -4
FA_ERR_TIMEOUT = -5
PAGE_TOKENS = 16

# (name, restype, argtypes) of every C-ABI entry point in include/friday_attn.h
_P, _I, _F, _SZ = C.c_void_p, C.c_int, C.c_float, C.c_size_t
API = [
    ("friday_attn_last_error", C.c_char_p, []),
    ("friday_attn_version", _I, []),
    ("friday_attn_rope_table_bytes", _SZ, [_I, _I]),
    ("friday_attn_rope_table_fill_host", _I, [_P, _I, _I, _F, _P]),
    ("friday_attn_rope_table_upload", _I, [_P, _I, _I, _F, _P, _P]),
    ("friday_attn_rope_store_kv", _I, [_P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _I, _I, _P, _I, _P]),
    ("friday_attn_store_kv_q8", _I, [_P, _P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _P]),
    ("friday_attn_decode_attention", _I, [_P, _P, _P, _P, _I, _I, _I, _I, _P]),
    ("friday_attn_decode_attention_dev_pos", _I, [_P, _P, _P, _P, _P, _I, _I, _I, _I, _P]),
    ("friday_attn_decode_fits_shared_memory", _I, [_I]),
    ("friday_attn_split_workspace_bytes", _SZ, [_I, _I]),
    ("friday_attn_decode_attention_split", _I, [_P, _P, _P, _P, _I, _P, _I, _I, _I, _I, _P, _SZ, _P, _P, _P]),
    ("friday_attn_decode_workspace_init", _I, [_P, _SZ, _P]),
    ("friday_attn_decode_workspace_status", _I, [_P, _SZ, _P]),
    ("friday_attn_set_decode_form", _I, [_I, _I, _I]),
    ("friday_attn_decode_attention_fused", _I, [_P, _P, _P, _P, _I, _P, _I, _I, _I, _I, _P, _SZ, _P, _P, _P]),
    ("friday_attn_decode_step", _I, [_P, _P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _I, _P, _I, _P, _SZ, _P]),
    ("friday_attn_decode_step_noalloc", _I, [_P, _P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _I, _P, _I, _P]),
    ("friday_attn_decode_step_q8", _I,
     [_P, _P, _P, _P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _I, _P, _I, _P, _SZ, _P]),
    ("friday_attn_prefill_supported", _I, [_I, _I, _I]),
    ("friday_attn_prefill_attention", _I, [_P, _P, _P, _P, _I, _P, _I, _I, _I, _P, _P, _P]),
    ("friday_attn_prefill_attention_bf16", _I, [_P, _P, _P, _P, _I, _P, _I, _I, _I, _P]),
    ("friday_attn_paged_workspace_bytes", _SZ, [_I, _I, _I]),
    ("friday_attn_paged_rope_store_kv", _I, [_P, _P, _P, _P, _P, _P, _I, _P, _I, _I, _I, _I, _I, _P, _I, _P]),
    ("friday_attn_paged_decode_step", _I,
     [_P, _P, _P, _P, _P, _P, _P, _I, _P, _I, _I, _I, _I, _I, _P, _I, _P, _SZ, _P]),
    ("friday_attn_paged_decode_attention", _I,
     [_P, _P, _P, _P, _P, _I, _P, _I, _I, _I, _I, _I, _P, _SZ, _P]),
    ("friday_attn_decode_step_quant", _I,
     [_P, _P, _P, _P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _I, _P, _I, _P, _SZ, _P]),
    ("friday_q8_row_bytes", _SZ, [_I, _I]),
    ("friday_quantize_q8_rows", _I, [_P, _I, _I, _P, _P, _P]),
    ("friday_gemm_q8_supported", _I, [_I, _I]),
    ("friday_gemm_q8", _I, [_I, _P, _P, _P, _I, _I, _I, _P, _I, _P, _P, _P]),
    ("friday_gemm_q8_reserve", _I, [_I, _I, _I, _P]),
    ("friday_gemm_q8_workspace_bytes", _SZ, [_I, _I, _I]),
    ("friday_gemm_q8_ws", _I, [_I, _P, _P, _P, _I, _I, _I, _P, _I, _P, _P, _P, _P, _SZ]),
    ("friday_gemv_q8", _I, [_I, _P, _P, _P, _I, _I, _P, _P, _P, _P, _P, _P]),
]

_lib = None


def load(path: str = LIB_PATH) -> C.CDLL:
    """Load libfriday_attn.so (raises if it is not built)."""
    global _lib
    if _lib is None:
        if not os.path.exists(path):
            raise RuntimeError(f"{path} is not built: run __graft_entry__.build() "
                               f"or python friday-inference-engine_amd/build.py")
        lib = C.CDLL(path, mode=C.RTLD_GLOBAL)
        for name, res, args in API:
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = args
        _lib = lib
    return _lib


class FridayAttnError(RuntimeError):
    def __init__(self, status: int, msg: str):
        super().__init__(f"[{status}] {msg}")
        self.status = status


def _check(rc: int):
    if rc != FA_OK:
        raise FridayAttnError(rc, load().friday_attn_last_error().decode())


def _ptr(x):
    if x is None:
        return None
    if isinstance(x, DeviceBuffer):
        return x.ptr
    return int(x)


# ---------------------------------------------------------------- HIP plumbing
class Hip:
    """Minimal ctypes access to the HIP runtime (same libamdhip64 as the library)."""

    _h = None

    @classmethod
    def lib(cls):
        if cls._h is None:
            load()  # pulls in libamdhip64.so.7 with the product library
            h = C.CDLL("libamdhip64.so.7")
            h.hipMalloc.argtypes = [C.POINTER(C.c_void_p), _SZ]
            h.hipFree.argtypes = [_P]
            h.hipMemcpy.argtypes = [_P, _P, _SZ, _I]
            h.hipMemcpyAsync.argtypes = [_P, _P, _SZ, _I, _P]
            h.hipMemset.argtypes = [_P, _I, _SZ]
            h.hipDeviceSynchronize.argtypes = []
            h.hipStreamSynchronize.argtypes = [_P]
            h.hipGetDeviceCount.argtypes = [C.POINTER(C.c_int)]
            h.hipEventCreate.argtypes = [C.POINTER(C.c_void_p)]
            h.hipEventRecord.argtypes = [_P, _P]
            h.hipEventSynchronize.argtypes = [_P]
            h.hipEventElapsedTime.argtypes = [C.POINTER(C.c_float), _P, _P]
            h.hipEventDestroy.argtypes = [_P]
            h.hipStreamCreate.argtypes = [C.POINTER(C.c_void_p)]
            h.hipStreamDestroy.argtypes = [_P]
            h.hipGetErrorString.restype = C.c_char_p
            h.hipGetErrorString.argtypes = [_I]
            h.hipDeviceGetAttribute.argtypes = [C.POINTER(C.c_int), _I, _I]
            h.hipStreamBeginCapture.argtypes = [_P, _I]
            h.hipStreamEndCapture.argtypes = [_P, C.POINTER(C.c_void_p)]
            h.hipGraphInstantiate.argtypes = [C.POINTER(C.c_void_p), _P, _P, _P, _SZ]
            h.hipGraphLaunch.argtypes = [_P, _P]
            h.hipGraphExecDestroy.argtypes = [_P]
            h.hipGraphDestroy.argtypes = [_P]
            cls._h = h
        return cls._h

    @classmethod
    def check(cls, rc, what="hip"):
        if rc != 0:
            raise RuntimeError(f"{what} failed: {cls.lib().hipGetErrorString(rc).decode()}")

    @classmethod
    def device_count(cls) -> int:
        n = C.c_int(0)
        rc = cls.lib().hipGetDeviceCount(C.byref(n))
        return n.value if rc == 0 else 0

    @classmethod
    def sync(cls):
        cls.check(cls.lib().hipDeviceSynchronize(), "hipDeviceSynchronize")


class Stream:
    """A default-priority HIP stream, destroyed by destroy() or when collected."""

    def __init__(self):
        s = C.c_void_p()
        Hip.check(Hip.lib().hipStreamCreate(C.byref(s)), "hipStreamCreate")
        self.s = s.value

    def synchronize(self):
        Hip.check(Hip.lib().hipStreamSynchronize(self.s), "hipStreamSynchronize")

    def destroy(self):
        if self.s:
            s, self.s = self.s, None
            Hip.check(Hip.lib().hipStreamDestroy(s), "hipStreamDestroy")

    def __del__(self):
        try:
            self.destroy()
        except Exception:
            pass


# Graphs that are instantiated and not yet destroyed. A graph's kernel nodes hold the raw
# device pointers of every buffer that was alive while it was captured; freeing one of
# those buffers while the graph lives would leave the graph pointing at memory that the
# next allocation reuses, so DeviceBuffer.free() refuses it.
_live_graphs: dict = {}
_deferred_frees: list = []  # (ptr, serial) of collected buffers that a live graph captured


def _release_deferred():
    keep = []
    for ptr, serial in _deferred_frees:
        if any(serial in g.captured for g in _live_graphs.values()):
            keep.append((ptr, serial))
        else:
            DeviceBuffer._live.discard(serial)
            Hip.lib().hipFree(ptr)
    _deferred_frees[:] = keep


class Graph:
    """Capture of the launches issued on `stream` by fn(), replayed with launch().

    destroy() (or leaving a `with` block) releases the executable graph and the graph:
    do that before freeing any buffer the captured launches use."""

    def __init__(self, stream: Stream, fn):
        h = Hip.lib()
        self.exec = self.graph = None
        Hip.check(h.hipStreamBeginCapture(stream.s, 2), "hipStreamBeginCapture")  # relaxed mode
        try:
            fn()
        finally:
            g = C.c_void_p()
            rc = h.hipStreamEndCapture(stream.s, C.byref(g))
        Hip.check(rc, "hipStreamEndCapture")
        self.graph = g.value
        e = C.c_void_p()
        try:
            Hip.check(h.hipGraphInstantiate(C.byref(e), self.graph, None, None, 0), "hipGraphInstantiate")
        except Exception:
            h.hipGraphDestroy(self.graph)
            self.graph = None
            raise
        self.exec = e.value
        self.stream = stream
        self.captured = frozenset(DeviceBuffer._live)  # buffers the launches may reference
        _live_graphs[id(self)] = self

    def launch(self):
        if not self.exec:
            raise RuntimeError("Graph.launch after destroy()")
        Hip.check(Hip.lib().hipGraphLaunch(self.exec, self.stream.s), "hipGraphLaunch")

    def destroy(self):
        """Release the executable graph, then the graph (a launch in flight completes first:
        HIP defers the release of an executable graph until its launches are done)."""
        h = Hip.lib()
        _live_graphs.pop(id(self), None)
        if self.exec:
            e, self.exec = self.exec, None
            Hip.check(h.hipGraphExecDestroy(e), "hipGraphExecDestroy")
        if self.graph:
            g, self.graph = self.graph, None
            Hip.check(h.hipGraphDestroy(g), "hipGraphDestroy")
        _release_deferred()

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.destroy()
        return False

    def __del__(self):
        try:
            self.destroy()
        except Exception:
            pass


class DeviceBuffer:
    """Owned device allocation."""

    _live: set = set()  # serials of the buffers allocated and not yet freed
    _serial = 0

    def __init__(self, nbytes: int):
        self.nbytes = int(nbytes)
        self.ptr = None
        p = C.c_void_p()
        Hip.check(Hip.lib().hipMalloc(C.byref(p), max(self.nbytes, 1)), f"hipMalloc({self.nbytes})")
        self.ptr = p.value
        DeviceBuffer._serial += 1
        self.serial = DeviceBuffer._serial
        DeviceBuffer._live.add(self.serial)

    @classmethod
    def from_array(cls, a: np.ndarray) -> "DeviceBuffer":
        a = np.ascontiguousarray(a)
        b = cls(a.nbytes)
        b.upload(a)
        return b

    def upload(self, a: np.ndarray, offset: int = 0):
        a = np.ascontiguousarray(a)
        assert self.ptr and offset + a.nbytes <= self.nbytes
        Hip.check(Hip.lib().hipMemcpy(self.ptr + offset, a.ctypes.data, a.nbytes, 1), "hipMemcpy H2D")

    def download(self, shape, dtype, offset: int = 0) -> np.ndarray:
        out = np.empty(shape, dtype)
        assert self.ptr and offset + out.nbytes <= self.nbytes
        Hip.check(Hip.lib().hipMemcpy(out.ctypes.data, self.ptr + offset, out.nbytes, 2), "hipMemcpy D2H")
        return out

    def fill_bytes(self, value: int):
        Hip.check(Hip.lib().hipMemset(self.ptr, value, self.nbytes), "hipMemset")

    def captured_by_live_graph(self) -> bool:
        return any(self.serial in g.captured for g in _live_graphs.values())

    def free(self):
        """Free the allocation. Raises while a live Graph may reference it (destroy the
        graph first)."""
        if self.ptr:
            if self.captured_by_live_graph():
                raise RuntimeError(f"DeviceBuffer({self.nbytes} B) freed while a live Graph captured with it "
                                   f"exists: destroy the graph first")
            p, self.ptr = self.ptr, None
            DeviceBuffer._live.discard(self.serial)
            Hip.check(Hip.lib().hipFree(p), "hipFree")

    def __del__(self):
        # a buffer collected while a live graph may still use it is freed when the last such
        # graph is destroyed (never earlier: no dangling pointer)
        try:
            if self.ptr and self.captured_by_live_graph():
                _deferred_frees.append((self.ptr, self.serial))
                self.ptr = None
            else:
                self.free()
        except Exception:
            pass


class Event:
    def __init__(self):
        e = C.c_void_p()
        Hip.check(Hip.lib().hipEventCreate(C.byref(e)), "hipEventCreate")
        self.e = e.value

    def record(self, stream=None):
        Hip.check(Hip.lib().hipEventRecord(self.e, stream), "hipEventRecord")

    def synchronize(self):
        Hip.check(Hip.lib().hipEventSynchronize(self.e), "hipEventSynchronize")

    def elapsed_ms(self, end: "Event") -> float:
        ms = C.c_float()
        Hip.check(Hip.lib().hipEventElapsedTime(C.byref(ms), self.e, end.e), "hipEventElapsedTime")
        return ms.value

    def destroy(self):
        if self.e:
            e, self.e = self.e, None
            Hip.check(Hip.lib().hipEventDestroy(e), "hipEventDestroy")

    def __del__(self):
        try:
            self.destroy()
        except Exception:
            pass


# ------------------------------------------------- friday_attn launcher mirror
def rope_table_bytes(max_ctx, head_dim) -> int:
    return load().friday_attn_rope_table_bytes(max_ctx, head_dim)


def rope_table_host(max_ctx, head_dim, freq_base, freq_factors=None) -> np.ndarray:
    t = np.empty((max_ctx, head_dim // 2, 2), np.float32)
    ff = None if freq_factors is None else np.ascontiguousarray(freq_factors, np.float32)
    _check(load().friday_attn_rope_table_fill_host(t.ctypes.data, max_ctx, head_dim, freq_base,
                                                   None if ff is None else ff.ctypes.data))
    return t


def rope_table_upload(d_table, max_ctx, head_dim, freq_base, freq_factors=None, stream=None):
    ff = None if freq_factors is None else np.ascontiguousarray(freq_factors, np.float32)
    _check(load().friday_attn_rope_table_upload(_ptr(d_table), max_ctx, head_dim, freq_base,
                                                None if ff is None else ff.ctypes.data, stream))


def ropeStoreKv(q, k, v, k_layer, v_layer, d_pos, pos, T, head_dim, num_q_heads, num_kv_heads, max_ctx,
                rope_table, neox, stream=None):
    """ropeStoreKvKernel launch (cuda_math_kernels.cu:363-404); caches None -> ropeKernel."""
    _check(load().friday_attn_rope_store_kv(_ptr(q), _ptr(k), _ptr(v), _ptr(k_layer), _ptr(v_layer), _ptr(d_pos),
                                            pos, T, head_dim, num_q_heads, num_kv_heads, max_ctx, _ptr(rope_table),
                                            int(neox), stream))


def storeKvQ8(k, v, k_layer, k_scale, v_layer, v_scale, d_pos, pos, T, kv_dim, max_ctx, stream=None):
    """storeKvQ8Kernel launch (cuda_math_kernels.cu:409-432)."""
    _check(load().friday_attn_store_kv_q8(_ptr(k), _ptr(v), _ptr(k_layer), _ptr(k_scale), _ptr(v_layer),
                                          _ptr(v_scale), _ptr(d_pos), pos, T, kv_dim, max_ctx, stream))


def launchDecodeAttention(q, k_cache, v_cache, out, seq_len, num_heads, num_kv_heads, head_dim, stream=None):
    _check(load().friday_attn_decode_attention(_ptr(q), _ptr(k_cache), _ptr(v_cache), _ptr(out), seq_len, num_heads,
                                               num_kv_heads, head_dim, stream))


def launchDecodeAttentionDevPos(q, k_cache, v_cache, out, d_pos, max_seq_len, num_heads, num_kv_heads, head_dim,
                                stream=None):
    _check(load().friday_attn_decode_attention_dev_pos(_ptr(q), _ptr(k_cache), _ptr(v_cache), _ptr(out),
                                                       _ptr(d_pos), max_seq_len, num_heads, num_kv_heads,
                                                       head_dim, stream))


def decodeAttentionFitsSharedMemory(max_seq_len) -> bool:
    return bool(load().friday_attn_decode_fits_shared_memory(max_seq_len))


def splitAttentionWorkspaceBytes(num_heads, max_seq_len) -> int:
    return load().friday_attn_split_workspace_bytes(num_heads, max_seq_len)


def launchDecodeAttentionSplit(q, k_cache, v_cache, out, seq_len, d_pos, max_seq_len, num_heads, num_kv_heads,
                               head_dim, workspace, stream=None, k_scale=None, v_scale=None, workspace_bytes=None):
    if workspace_bytes is None:
        workspace_bytes = workspace.nbytes if isinstance(workspace, DeviceBuffer) else 0
    _check(load().friday_attn_decode_attention_split(_ptr(q), _ptr(k_cache), _ptr(v_cache), _ptr(out), seq_len,
                                                     _ptr(d_pos), max_seq_len, num_heads, num_kv_heads, head_dim,
                                                     _ptr(workspace), workspace_bytes, stream, _ptr(k_scale),
                                                     _ptr(v_scale)))


def decodeWorkspaceInit(workspace, workspace_bytes=None, stream=None):
    if workspace_bytes is None:
        workspace_bytes = workspace.nbytes
    _check(load().friday_attn_decode_workspace_init(_ptr(workspace), workspace_bytes, stream))


def setDecodeForm(local_merge: int = -1, split_major: int = -1, kv_pair: int = -1) -> None:
    """friday_attn_set_decode_form: process-wide decode placement / merge form (-1: the
    environment's choice). local_merge and split_major give bit-identical results; kv_pair
    changes the split bound (results within the decode tolerance)."""
    _check(load().friday_attn_set_decode_form(local_merge, split_major, kv_pair))


def decodeWorkspaceStatus(workspace, workspace_bytes=None, stream=None) -> int:
    """FA_OK, or FA_ERR_TIMEOUT once a fused merge on this workspace gave up waiting
    (synchronises `stream`)."""
    if workspace_bytes is None:
        workspace_bytes = workspace.nbytes
    rc = load().friday_attn_decode_workspace_status(_ptr(workspace), workspace_bytes, stream)
    if rc not in (FA_OK, FA_ERR_TIMEOUT):
        _check(rc)
    return rc


def launchDecodeAttentionFused(q, k_cache, v_cache, out, seq_len, d_pos, max_seq_len, num_heads, num_kv_heads,
                               head_dim, workspace, stream=None, k_scale=None, v_scale=None, workspace_bytes=None):
    """Split-K decode with the merge done inside the same kernel by the last-dispatched splits."""
    if workspace_bytes is None:
        workspace_bytes = workspace.nbytes if isinstance(workspace, DeviceBuffer) else 0
    _check(load().friday_attn_decode_attention_fused(_ptr(q), _ptr(k_cache), _ptr(v_cache), _ptr(out), seq_len,
                                                     _ptr(d_pos), max_seq_len, num_heads, num_kv_heads, head_dim,
                                                     _ptr(workspace), workspace_bytes, stream, _ptr(k_scale),
                                                     _ptr(v_scale)))


def decodeStep(q, k, v, k_layer, v_layer, out, d_pos, pos, max_ctx, num_heads, num_kv_heads, head_dim, rope_table,
               neox, workspace, stream=None, workspace_bytes=None):
    """RoPE + KV append + split-K decode attention + merge in one launch (fused workspace)."""
    if workspace_bytes is None:
        workspace_bytes = workspace.nbytes if isinstance(workspace, DeviceBuffer) else 0
    _check(load().friday_attn_decode_step(_ptr(q), _ptr(k), _ptr(v), _ptr(k_layer), _ptr(v_layer), _ptr(out),
                                          _ptr(d_pos), pos, max_ctx, num_heads, num_kv_heads, head_dim,
                                          _ptr(rope_table), int(neox), _ptr(workspace), workspace_bytes, stream))


def decodeStepNoAlloc(q, k, v, k_layer, v_layer, out, d_pos, pos, max_ctx, num_heads, num_kv_heads, head_dim,
                      rope_table, neox, stream=None):
    """decodeStep on the library's per-GPU device scratch: no workspace, no allocation."""
    _check(load().friday_attn_decode_step_noalloc(_ptr(q), _ptr(k), _ptr(v), _ptr(k_layer), _ptr(v_layer), _ptr(out),
                                                  _ptr(d_pos), pos, max_ctx, num_heads, num_kv_heads, head_dim,
                                                  _ptr(rope_table), int(neox), stream))


def decodeStepQ8(q, k, v, k_layer, k_scale, v_layer, v_scale, out, d_pos, pos, max_ctx, num_heads, num_kv_heads,
                 head_dim, rope_table, neox, workspace, stream=None, workspace_bytes=None):
    """decodeStep for an int8 KV cache (values [max_ctx][Hkv*d] int8, scales [max_ctx][Hkv*d/32] fp16)."""
    if workspace_bytes is None:
        workspace_bytes = workspace.nbytes if isinstance(workspace, DeviceBuffer) else 0
    _check(load().friday_attn_decode_step_q8(_ptr(q), _ptr(k), _ptr(v), _ptr(k_layer), _ptr(k_scale), _ptr(v_layer),
                                             _ptr(v_scale), _ptr(out), _ptr(d_pos), pos, max_ctx, num_heads,
                                             num_kv_heads, head_dim, _ptr(rope_table), int(neox), _ptr(workspace),
                                             workspace_bytes, stream))


def prefillAttentionSupported(num_heads, num_kv_heads, head_dim) -> bool:
    return bool(load().friday_attn_prefill_supported(num_heads, num_kv_heads, head_dim))


def launchPrefillAttention(q, k_cache, v_cache, out, T, d_pos0, num_heads, num_kv_heads, head_dim, stream=None,
                           k_scale=None, v_scale=None):
    _check(load().friday_attn_prefill_attention(_ptr(q), _ptr(k_cache), _ptr(v_cache), _ptr(out), T, _ptr(d_pos0),
                                                num_heads, num_kv_heads, head_dim, stream, _ptr(k_scale),
                                                _ptr(v_scale)))


def launchPrefillAttentionBf16(q, k_cache, v_cache, out, T, d_pos0, num_heads, num_kv_heads, head_dim, stream=None):
    """launchPrefillAttention with bf16 q / K / V / out (no counterpart in the reference)."""
    _check(load().friday_attn_prefill_attention_bf16(_ptr(q), _ptr(k_cache), _ptr(v_cache), _ptr(out), T,
                                                     _ptr(d_pos0), num_heads, num_kv_heads, head_dim, stream))


def pagedWorkspaceBytes(batch, num_heads, max_seq_len) -> int:
    return load().friday_attn_paged_workspace_bytes(batch, num_heads, max_seq_len)


def pagedRopeStoreKv(q, k, v, k_pool, v_pool, block_table, block_table_stride, seq_lens, batch, head_dim,
                     num_q_heads, num_kv_heads, max_ctx, rope_table, neox, stream=None):
    _check(load().friday_attn_paged_rope_store_kv(_ptr(q), _ptr(k), _ptr(v), _ptr(k_pool), _ptr(v_pool),
                                                  _ptr(block_table), block_table_stride, _ptr(seq_lens), batch,
                                                  head_dim, num_q_heads, num_kv_heads, max_ctx, _ptr(rope_table),
                                                  int(neox), stream))


def pagedDecodeStep(q, k, v, k_pool, v_pool, out, block_table, block_table_stride, seq_lens, batch, max_seq_len,
                    num_heads, num_kv_heads, head_dim, rope_table, neox, workspace, stream=None, workspace_bytes=None):
    if workspace_bytes is None:
        workspace_bytes = workspace.nbytes if isinstance(workspace, DeviceBuffer) else 0
    _check(load().friday_attn_paged_decode_step(_ptr(q), _ptr(k), _ptr(v), _ptr(k_pool), _ptr(v_pool), _ptr(out),
                                                _ptr(block_table), block_table_stride, _ptr(seq_lens), batch,
                                                max_seq_len, num_heads, num_kv_heads, head_dim, _ptr(rope_table),
                                                int(neox), _ptr(workspace), workspace_bytes, stream))


def launchPagedDecodeAttention(q, k_pool, v_pool, out, block_table, block_table_stride, seq_lens, batch,
                               max_seq_len, num_heads, num_kv_heads, head_dim, workspace, stream=None,
                               workspace_bytes=None):
    if workspace_bytes is None:
        workspace_bytes = workspace.nbytes if isinstance(workspace, DeviceBuffer) else 0
    _check(load().friday_attn_paged_decode_attention(_ptr(q), _ptr(k_pool), _ptr(v_pool), _ptr(out),
                                                     _ptr(block_table), block_table_stride, _ptr(seq_lens), batch,
                                                     max_seq_len, num_heads, num_kv_heads, head_dim,
                                                     _ptr(workspace), workspace_bytes, stream))


# ---- prefill projection GEMM (friday_prefill::gemmQ8, friday_hpc::quantizeQ8Rows) ----
# weight kinds: the codes of friday_hpc::Q8Kind
Q2_K, Q3_K, Q4_K, Q5_K, Q6_K, Q8_0 = 1, 2, 3, 4, 5, 6


def q8RowBytes(kind, K) -> int:
    return load().friday_q8_row_bytes(kind, K)


def quantizeQ8Rows(x, rows, K, xq, xd, stream=None):
    _check(load().friday_quantize_q8_rows(_ptr(x), rows, K, _ptr(xq), _ptr(xd), stream))


def gemmQ8Supported(kind, K) -> bool:
    return bool(load().friday_gemm_q8_supported(kind, K))


def gemmQ8(kind, W, xq, xd, T, K, N, Y, ldy, stream=None, bias=None, res=None):
    _check(load().friday_gemm_q8(kind, _ptr(W), _ptr(xq), _ptr(xd), T, K, N, _ptr(Y), ldy, stream, _ptr(bias),
                                 _ptr(res)))


def gemmQ8Reserve(T, K, N, stream=None):
    """Size the K-split workspace of gemmQ8 for (T, K, N) on `stream` before stream capture."""
    _check(load().friday_gemm_q8_reserve(T, K, N, stream))


def gemmQ8WorkspaceBytes(T, K, N) -> int:
    return load().friday_gemm_q8_workspace_bytes(T, K, N)


def gemmQ8Ws(kind, W, xq, xd, T, K, N, Y, ldy, workspace, stream=None, bias=None, res=None, workspace_bytes=None):
    """gemmQ8 with a caller-owned workspace (zeroed once with decodeWorkspaceInit)."""
    if workspace_bytes is None:
        workspace_bytes = workspace.nbytes if isinstance(workspace, DeviceBuffer) else 0
    _check(load().friday_gemm_q8_ws(kind, _ptr(W), _ptr(xq), _ptr(xd), T, K, N, _ptr(Y), ldy, stream, _ptr(bias),
                                    _ptr(res), _ptr(workspace), workspace_bytes))


def gemvQ8(kind, W, xq, xd, K, N, y, stream=None, W2=None, y2=None, bias=None, res=None):
    """friday_hpc::gemvQ8 with the activation scratch (xq, xd) passed explicitly."""
    _check(load().friday_gemv_q8(kind, _ptr(W), _ptr(xq), _ptr(xd), K, N, _ptr(y), stream, _ptr(W2), _ptr(y2),
                                 _ptr(bias), _ptr(res)))


def decodeStepQuant(q, k, v, k_layer, v_layer, out, out_q, out_d, d_pos, pos, max_ctx, num_heads, num_kv_heads,
                    head_dim, rope_table, neox, workspace, stream=None, workspace_bytes=None):
    """decodeStep plus the int8 form of `out` (quantizeQ8) in the same launch."""
    if workspace_bytes is None:
        workspace_bytes = workspace.nbytes if isinstance(workspace, DeviceBuffer) else 0
    _check(load().friday_attn_decode_step_quant(_ptr(q), _ptr(k), _ptr(v), _ptr(k_layer), _ptr(v_layer), _ptr(out),
                                                _ptr(out_q), _ptr(out_d), _ptr(d_pos), pos, max_ctx, num_heads,
                                                num_kv_heads, head_dim, _ptr(rope_table), int(neox), _ptr(workspace),
                                                workspace_bytes, stream))
