"""C-ABI checks that need no GPU: libfriday_attn.so loads, exports every entry point
declared in include/friday_attn.h, validates arguments before any HIP call (the
reference throws / aborts at the same points, attention_kernels.cu:416-454,
:657-661), and builds the RoPE table with the CPU formula bit for bit.
"""
import ctypes as C
import os
import re

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "friday_attn.h")
FAKE = 0x1000  # non-null pointer value: every call below must fail before touching it


def declared_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(friday_(?:attn|gemm|gemv|quantize|q8)_\w+)\s*\(", text)))


def test_header_and_binding_agree(fa):
    names = declared_functions()
    assert len(names) >= 20
    bound = {n for n, _, _ in fa.API}
    assert set(names) == bound, set(names) ^ bound


def test_every_symbol_exported(fa):
    lib = fa.load()
    for name in declared_functions():
        assert hasattr(lib, name), name


def err(fa):
    return fa.load().friday_attn_last_error().decode()


def test_decode_validation(fa):
    L = fa.load()
    # head_dim must be 64 or 128 (the reference accepts 128 only)
    assert L.friday_attn_decode_attention(FAKE, FAKE, FAKE, FAKE, 10, 40, 8, 96, None) == fa.FA_ERR_UNSUPPORTED
    assert "head_dim" in err(fa)
    # Hq % Hkv != 0, Hkv <= 0
    assert L.friday_attn_decode_attention(FAKE, FAKE, FAKE, FAKE, 10, 40, 7, 128, None) == fa.FA_ERR_INVALID
    assert L.friday_attn_decode_attention(FAKE, FAKE, FAKE, FAKE, 10, 40, 0, 128, None) == fa.FA_ERR_INVALID
    # seq_len <= 0 with a host length
    assert L.friday_attn_decode_attention(FAKE, FAKE, FAKE, FAKE, 0, 40, 8, 128, None) == fa.FA_ERR_INVALID
    # null tensors
    assert L.friday_attn_decode_attention(None, FAKE, FAKE, FAKE, 10, 40, 8, 128, None) == fa.FA_ERR_INVALID
    # dev-pos variant needs d_pos
    assert L.friday_attn_decode_attention_dev_pos(FAKE, FAKE, FAKE, FAKE, None, 10, 40, 8, 128,
                                                  None) == fa.FA_ERR_INVALID


def test_split_workspace_rules(fa):
    L = fa.load()
    need = L.friday_attn_split_workspace_bytes(40, 32768)
    assert need > 0 and L.friday_attn_split_workspace_bytes(0, 10) == 0
    # layout: a 256-byte counter slot per query head, then per (head, split) d = 128 partial
    # values, (max, sum) and one flag word; at most 128 splits of >= 128 positions
    assert need == 40 * 256 + 40 * 128 * (128 + 3) * 4
    assert L.friday_attn_split_workspace_bytes(40, 1000) == 40 * 256 + 40 * 8 * (128 + 3) * 4
    # too small a workspace is refused before any launch
    rc = L.friday_attn_decode_attention_split(FAKE, FAKE, FAKE, FAKE, 32768, None, 32768, 40, 8, 128, FAKE, need // 2,
                                              None, None, None)
    assert rc == fa.FA_ERR_WORKSPACE, err(fa)
    rc = L.friday_attn_decode_attention_fused(FAKE, FAKE, FAKE, FAKE, 100, None, 32768, 40, 8, 128, None, need,
                                              None, None, None)
    assert rc == fa.FA_ERR_WORKSPACE
    # seq_len beyond max_seq_len
    rc = L.friday_attn_decode_attention_split(FAKE, FAKE, FAKE, FAKE, 5000, None, 4096, 40, 8, 128, FAKE, need,
                                              None, None, None)
    assert rc == fa.FA_ERR_INVALID
    # only one of the int8 scales
    rc = L.friday_attn_decode_attention_split(FAKE, FAKE, FAKE, FAKE, 100, None, 4096, 40, 8, 128, FAKE, need,
                                              None, FAKE, None)
    assert rc == fa.FA_ERR_INVALID
    assert L.friday_attn_decode_fits_shared_memory(1 << 20) == 1
    assert L.friday_attn_decode_workspace_init(None, 16, None) == fa.FA_ERR_INVALID


def test_append_validation(fa):
    L = fa.load()
    # positions past max_ctx with a host position
    assert L.friday_attn_rope_store_kv(FAKE, FAKE, FAKE, FAKE, FAKE, None, 100, 5, 128, 40, 8, 102, FAKE, 1,
                                       None) == fa.FA_ERR_INVALID
    # cache pointers must come together
    assert L.friday_attn_rope_store_kv(FAKE, FAKE, FAKE, FAKE, None, None, 0, 1, 128, 40, 8, 10, FAKE, 1,
                                       None) == fa.FA_ERR_INVALID
    # no rope table
    assert L.friday_attn_rope_store_kv(FAKE, FAKE, FAKE, FAKE, FAKE, None, 0, 1, 128, 40, 8, 10, None, 1,
                                       None) == fa.FA_ERR_INVALID
    # the append moves 16-byte chunks: misaligned tensors are rejected
    assert L.friday_attn_rope_store_kv(FAKE + 2, FAKE, FAKE, FAKE, FAKE, None, 0, 1, 128, 40, 8, 10, FAKE, 1,
                                       None) == fa.FA_ERR_INVALID
    assert "aligned" in err(fa)
    # int8: kv_dim must be a multiple of 32
    assert L.friday_attn_store_kv_q8(FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, None, 0, 1, 100, 10,
                                     None) == fa.FA_ERR_INVALID
    assert L.friday_attn_decode_step(FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, None, 10, 10, 40, 8, 128, FAKE, 1, FAKE, 1 << 30,
                                     None) == fa.FA_ERR_INVALID  # pos == max_ctx


def test_prefill_and_paged_validation(fa):
    L = fa.load()
    assert L.friday_attn_prefill_supported(40, 8, 128) == 1
    assert L.friday_attn_prefill_supported(40, 8, 96) == 0
    assert L.friday_attn_prefill_supported(40, 7, 128) == 0
    # T <= 0 returns early like the reference launcher (attention_kernels.cu:656)
    assert L.friday_attn_prefill_attention(None, None, None, None, 0, None, 40, 8, 128, None, None, None) == fa.FA_OK
    assert L.friday_attn_prefill_attention(FAKE, FAKE, FAKE, FAKE, 5, None, 40, 8, 128, None, None,
                                           None) == fa.FA_ERR_INVALID
    # a block table row too short for max_seq_len
    need = L.friday_attn_paged_workspace_bytes(4, 40, 4096)
    assert L.friday_attn_paged_decode_attention(FAKE, FAKE, FAKE, FAKE, FAKE, 10, FAKE, 4, 4096, 40, 8, 128, FAKE,
                                                need, None) == fa.FA_ERR_INVALID
    assert L.friday_attn_paged_decode_attention(FAKE, FAKE, FAKE, FAKE, FAKE, 256, FAKE, 4, 4096, 40, 8, 128, FAKE,
                                                need - 1, None) == fa.FA_ERR_WORKSPACE


def test_rope_table_matches_oracle(fa, oracle):
    for d, base, ff in [(64, 1e6, None), (128, 5e5, np.linspace(1, 8, 64).astype(np.float32)), (128, 1e4, None)]:
        t = fa.rope_table_host(3000, d, base, ff)
        assert np.array_equal(t.view(np.uint32), oracle.rope_table(3000, d, base, ff).view(np.uint32))
    assert fa.rope_table_bytes(32768, 128) == 32768 * 64 * 8
    with pytest.raises(fa.FridayAttnError):
        fa.rope_table_host(10, 96, 1e4)


def test_error_message_is_thread_local(fa):
    import threading
    L = fa.load()
    L.friday_attn_decode_attention(FAKE, FAKE, FAKE, FAKE, 10, 40, 7, 128, None)
    seen = []
    t = threading.Thread(target=lambda: seen.append(L.friday_attn_last_error().decode()))
    t.start()
    t.join()
    assert seen == [""] and "num_kv_heads" in err(fa)


def test_cpp_shim_compiles():
    """include/friday_attn.hpp (the friday_attn:: / friday_hpc:: / friday_prefill:: drop-in)
    compiles as C++17 host code."""
    import subprocess
    import tempfile
    src = ('#include "friday_attn.hpp"\nint main() { return friday_attn::decodeAttentionFitsSharedMemory(10) && '
           'friday_prefill::gemmQ8Supported(friday_hpc::Q8Kind::Q4_K, 256) && '
           'friday_hpc::gemvQ8Supported(friday_hpc::Q8Kind::Q8_0) ? 0 : 1; }\n')
    with tempfile.TemporaryDirectory() as d:
        f = os.path.join(d, "t.cpp")
        open(f, "w").write(src)
        r = subprocess.run(["g++", "-std=c++17", "-fsyntax-only", "-I", os.path.join(ROOT, "include"),
                            "-I", "/opt/rocm/include", "-D__HIP_PLATFORM_AMD__", f], capture_output=True, text=True)
        assert r.returncode == 0, r.stderr


def test_gemm_q8_validation(fa):
    """gemmQ8Supported rules (prefill_kernels.cu:340: a known kind and K % 256 == 0) and the
    argument checks that run before any HIP call."""
    L = fa.load()
    assert L.friday_gemm_q8_supported(fa.Q4_K, 4096) == 1 and L.friday_gemm_q8_supported(fa.Q8_0, 256) == 1
    assert L.friday_gemm_q8_supported(fa.Q4_K, 4000) == 0 and L.friday_gemm_q8_supported(0, 4096) == 0
    assert L.friday_gemm_q8_supported(7, 4096) == 0
    # unsupported kind / K (the reference aborts there, prefill_kernels.cu:344-347)
    assert L.friday_gemm_q8(fa.Q4_K, FAKE, FAKE, FAKE, 4, 1000, 64, FAKE, 64, None, None, None) == fa.FA_ERR_UNSUPPORTED
    assert "K" in err(fa)
    # T <= 0: nothing to do
    assert L.friday_gemm_q8(fa.Q4_K, FAKE, FAKE, FAKE, 0, 256, 64, FAKE, 64, None, None, None) == fa.FA_OK
    # ldy < N, null Y, misaligned xq
    assert L.friday_gemm_q8(fa.Q4_K, FAKE, FAKE, FAKE, 4, 256, 64, FAKE, 32, None, None, None) == fa.FA_ERR_INVALID
    assert L.friday_gemm_q8(fa.Q4_K, FAKE, FAKE, FAKE, 4, 256, 64, None, 64, None, None, None) == fa.FA_ERR_INVALID
    assert L.friday_gemm_q8(fa.Q4_K, FAKE, FAKE + 4, FAKE, 4, 256, 64, FAKE, 64, None, None, None) == fa.FA_ERR_INVALID
    # row bytes of the GGML layouts
    assert [L.friday_q8_row_bytes(k, 512) for k in range(1, 7)] == [168, 220, 288, 352, 420, 544]
    assert L.friday_q8_row_bytes(fa.Q2_K, 300) == 0
    # workspace reservation: positive T, N and K a multiple of 256 (checked before any HIP call)
    assert L.friday_gemm_q8_reserve(0, 4096, 64, None) == fa.FA_ERR_INVALID
    assert L.friday_gemm_q8_reserve(4, 4000, 64, None) == fa.FA_ERR_INVALID
    assert L.friday_gemm_q8_reserve(4, 4096, -1, None) == fa.FA_ERR_INVALID
    # caller-owned workspace: sized by friday_gemm_q8_workspace_bytes, missing / small / misaligned rejected
    assert L.friday_gemm_q8_workspace_bytes(0, 4096, 64) == 0
    assert L.friday_gemm_q8_workspace_bytes(4, 4000, 64) == 0
    need = L.friday_gemm_q8_workspace_bytes(512, 14336, 4096)
    assert need > L.friday_gemm_q8_workspace_bytes(512, 4096, 4096) > 0
    args = (fa.Q4_K, FAKE, FAKE, FAKE, 512, 14336, 4096, FAKE, 4096, None, None, None)
    assert L.friday_gemm_q8_ws(*args, None, need) == fa.FA_ERR_WORKSPACE
    assert L.friday_gemm_q8_ws(*args, FAKE, need - 1) == fa.FA_ERR_WORKSPACE
    assert L.friday_gemm_q8_ws(*args, FAKE + 16, need) == fa.FA_ERR_WORKSPACE
    assert "workspace" in err(fa)
    assert L.friday_gemm_q8_ws(fa.Q4_K, FAKE, FAKE, FAKE, 0, 256, 64, FAKE, 64, None, None, None, None, 0) == fa.FA_OK
    # activation quantiser: K multiple of 32
    assert L.friday_quantize_q8_rows(FAKE, 2, 48, FAKE, FAKE, None) == fa.FA_ERR_INVALID
    assert L.friday_quantize_q8_rows(FAKE, 0, 64, FAKE, FAKE, None) == fa.FA_OK


def test_gemv_q8_validation(fa):
    L = fa.load()
    # K: a multiple of 256 (of 32 for Q8_0); unknown kind
    assert L.friday_gemv_q8(fa.Q4_K, FAKE, FAKE, FAKE, 1000, 64, FAKE, None, None, None, None, None) == \
        fa.FA_ERR_UNSUPPORTED
    assert L.friday_gemv_q8(0, FAKE, FAKE, FAKE, 1024, 64, FAKE, None, None, None, None, None) == fa.FA_ERR_UNSUPPORTED
    # W2 without y2, N <= 0, misaligned W
    assert L.friday_gemv_q8(fa.Q8_0, FAKE, FAKE, FAKE, 96, 64, FAKE, None, FAKE, None, None, None) == fa.FA_ERR_INVALID
    assert L.friday_gemv_q8(fa.Q8_0, FAKE, FAKE, FAKE, 96, 0, FAKE, None, None, None, None, None) == fa.FA_ERR_INVALID
    assert L.friday_gemv_q8(fa.Q8_0, FAKE + 2, FAKE, FAKE, 96, 8, FAKE, None, None, None, None, None) == \
        fa.FA_ERR_INVALID


def test_decode_alignment_and_status_checks(fa):
    """The decode paths move q, the caches and the new rows as 16-byte chunks and the
    output as 8-byte ones: misaligned pointers are refused before any launch."""
    L = fa.load()
    ws = 1 << 30
    assert L.friday_attn_decode_step(FAKE + 2, FAKE, FAKE, FAKE, FAKE, FAKE, None, 5, 10, 40, 8, 128, FAKE, 1, FAKE,
                                     ws, None) == fa.FA_ERR_INVALID
    assert "aligned" in err(fa)
    assert L.friday_attn_decode_step(FAKE, FAKE + 8, FAKE, FAKE, FAKE, FAKE, None, 5, 10, 40, 8, 128, FAKE, 1, FAKE,
                                     ws, None) == fa.FA_ERR_INVALID
    assert L.friday_attn_decode_step(FAKE, FAKE, FAKE, FAKE, FAKE, FAKE + 4, None, 5, 10, 40, 8, 128, FAKE, 1, FAKE,
                                     ws, None) == fa.FA_ERR_INVALID
    assert L.friday_attn_decode_step_q8(FAKE, FAKE, FAKE, FAKE + 1, FAKE, FAKE, FAKE, FAKE, None, 5, 10, 40, 8, 128,
                                        FAKE, 1, FAKE, ws, None) == fa.FA_ERR_INVALID
    assert L.friday_attn_decode_step_noalloc(FAKE, FAKE, FAKE, FAKE, FAKE + 2, FAKE, None, 5, 10, 40, 8, 128, FAKE, 1,
                                             None) == fa.FA_ERR_INVALID
    assert L.friday_attn_decode_attention_fused(FAKE + 2, FAKE, FAKE, FAKE, 5, None, 10, 40, 8, 128, FAKE, ws, None,
                                                None, None) == fa.FA_ERR_INVALID
    assert L.friday_attn_decode_attention(FAKE, FAKE, FAKE + 8, FAKE, 5, 40, 8, 128, None) == fa.FA_ERR_INVALID
    assert L.friday_attn_paged_decode_step(FAKE, FAKE + 2, FAKE, FAKE, FAKE, FAKE, FAKE, 256, FAKE, 4, 4096, 40, 8,
                                           128, FAKE, 1, FAKE, ws, None) == fa.FA_ERR_INVALID
    assert L.friday_attn_paged_decode_attention(FAKE, FAKE + 4, FAKE, FAKE, FAKE, 256, FAKE, 4, 4096, 40, 8, 128,
                                                FAKE, ws, None) == fa.FA_ERR_INVALID
    # the status query needs a workspace that holds counter slot 0
    assert L.friday_attn_decode_workspace_status(None, 4096, None) == fa.FA_ERR_INVALID
    assert L.friday_attn_decode_workspace_status(FAKE, 16, None) == fa.FA_ERR_INVALID


def test_set_decode_form_rejects_bad_values(fa):
    L = fa.load()
    assert L.friday_attn_set_decode_form(2, 0, 0) == fa.FA_ERR_INVALID
    assert L.friday_attn_set_decode_form(0, -2, 0) == fa.FA_ERR_INVALID
    assert L.friday_attn_set_decode_form(0, 0, 3) == fa.FA_ERR_INVALID
    assert L.friday_attn_set_decode_form(-1, -1, -1) == fa.FA_OK
