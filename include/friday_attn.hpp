// Header-only C++17 drop-in for the reference's friday_attn:: launchers
// (attention_kernels.h:7-52), the direct ropeStoreKvKernel / storeKvQ8Kernel launches of
// transformer.cpp, and the int8-activation matmuls on either side of attention
// (friday_hpc::quantizeQ8 / quantizeQ8Rows / gemvQ8, hpc_k_quants.h:39-68;
// friday_prefill::gemmQ8, prefill_kernels.h:15-25), implemented on the friday_attn C ABI.
//
// Same names, argument order and meaning; tensors are taken as void pointers so
// that half* / __half* / uint16_t* arguments all convert. Errors throw
// std::runtime_error with the library's message, as the reference launchers do
// (attention_kernels.cu:416-427, 431-441, 450-454, 483-485); an unsupported
// prefill layout prints and aborts like launchPrefillAttention (:657-661).
#ifndef FRIDAY_ATTN_HPP
#define FRIDAY_ATTN_HPP

#include <hip/hip_runtime_api.h>

#include <cstddef>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <stdexcept>
#include <vector>
#include <string>

#include "friday_attn.h"

namespace friday_attn {

namespace detail {
inline void check(int rc) {
    if (rc != FA_OK) throw std::runtime_error(std::string("friday_attn: ") + friday_attn_last_error());
}
inline const uint16_t* h(const void* p) { return static_cast<const uint16_t*>(p); }
inline uint16_t* h(void* p) { return static_cast<uint16_t*>(p); }
}  // namespace detail

// ---- attention_kernels.h:18-20
inline void launchDecodeAttention(const void* q, const void* k_cache, const void* v_cache, void* out, int seq_len,
                                  int num_heads, int num_kv_heads, int head_dim, hipStream_t stream) {
    detail::check(friday_attn_decode_attention(detail::h(q), detail::h(k_cache), detail::h(v_cache), detail::h(out),
                                               seq_len, num_heads, num_kv_heads, head_dim, stream));
}

// ---- attention_kernels.h:24-26
inline void launchDecodeAttentionDevPos(const void* q, const void* k_cache, const void* v_cache, void* out,
                                        const int* d_pos, int max_seq_len, int num_heads, int num_kv_heads,
                                        int head_dim, hipStream_t stream) {
    detail::check(friday_attn_decode_attention_dev_pos(detail::h(q), detail::h(k_cache), detail::h(v_cache),
                                                       detail::h(out), d_pos, max_seq_len, num_heads, num_kv_heads,
                                                       head_dim, stream));
}
inline bool decodeAttentionFitsSharedMemory(int max_seq_len) {
    return friday_attn_decode_fits_shared_memory(max_seq_len) != 0;
}

// ---- attention_kernels.h:32-38 (the workspace holds splitAttentionWorkspaceBytes bytes, as there)
inline size_t splitAttentionWorkspaceBytes(int num_heads, int max_seq_len) {
    return friday_attn_split_workspace_bytes(num_heads, max_seq_len);
}
// No counterpart in the reference: health of a fused-merge workspace (throws on a launch
// error; returns false once a fused merge gave up waiting, true otherwise). Synchronises
// `stream`; not for use under capture.
inline bool decodeWorkspaceHealthy(const void* workspace, size_t workspace_bytes, hipStream_t stream) {
    const int rc = friday_attn_decode_workspace_status(workspace, workspace_bytes, stream);
    if (rc == FA_ERR_TIMEOUT) return false;
    detail::check(rc);
    return true;
}
inline void launchDecodeAttentionSplit(const void* q, const void* k_cache, const void* v_cache, void* out,
                                       int seq_len, const int* d_pos, int max_seq_len, int num_heads,
                                       int num_kv_heads, int head_dim, void* workspace, hipStream_t stream,
                                       const void* k_scale = nullptr, const void* v_scale = nullptr) {
    detail::check(friday_attn_decode_attention_split(
        detail::h(q), k_cache, v_cache, detail::h(out), seq_len, d_pos, max_seq_len, num_heads, num_kv_heads,
        head_dim, workspace, splitAttentionWorkspaceBytes(num_heads, max_seq_len), stream, detail::h(k_scale),
        detail::h(v_scale)));
}

// ---- attention_kernels.h:46-50
inline bool prefillAttentionSupported(int num_heads, int num_kv_heads, int head_dim) {
    return friday_attn_prefill_supported(num_heads, num_kv_heads, head_dim) != 0;
}
inline void launchPrefillAttention(const void* q, const void* k_cache, const void* v_cache, void* out, int T,
                                   const int* d_pos0, int num_heads, int num_kv_heads, int head_dim,
                                   hipStream_t stream, const void* k_scale = nullptr,
                                   const void* v_scale = nullptr) {
    if (T <= 0) return;
    if (!prefillAttentionSupported(num_heads, num_kv_heads, head_dim)) {
        std::fprintf(stderr, "launchPrefillAttention: unsupported head layout\n");
        std::abort();
    }
    detail::check(friday_attn_prefill_attention(detail::h(q), k_cache, v_cache, detail::h(out), T, d_pos0,
                                                num_heads, num_kv_heads, head_dim, stream, detail::h(k_scale),
                                                detail::h(v_scale)));
}
// bf16 q / caches / out (friday_attn_prefill_attention_bf16; no reference counterpart)
inline void launchPrefillAttentionBf16(const void* q, const void* k_cache, const void* v_cache, void* out, int T,
                                       const int* d_pos0, int num_heads, int num_kv_heads, int head_dim,
                                       hipStream_t stream) {
    if (T <= 0) return;
    if (!prefillAttentionSupported(num_heads, num_kv_heads, head_dim)) {
        std::fprintf(stderr, "launchPrefillAttentionBf16: unsupported head layout\n");
        std::abort();
    }
    detail::check(friday_attn_prefill_attention_bf16(detail::h(q), detail::h(k_cache), detail::h(v_cache),
                                                     detail::h(out), T, d_pos0, num_heads, num_kv_heads, head_dim,
                                                     stream));
}

// ---- the kernels transformer.cpp launches directly
// ropeStoreKvKernel (cuda_math_kernels.cu:363-404; T tokens = grid.y there); the rope
// table replaces the (freq_base, freq_factors) kernel arguments: build it once with
// friday_attn_rope_table_upload. k_layer == v_layer == nullptr: ropeKernel semantics.
inline void ropeStoreKv(void* q, void* k, const void* v, void* k_layer, void* v_layer, const int* d_pos, int T,
                        int head_dim, int num_q_heads, int num_kv_heads, int max_ctx, const float* rope_table,
                        bool neox, hipStream_t stream) {
    detail::check(friday_attn_rope_store_kv(detail::h(q), detail::h(k), detail::h(v), detail::h(k_layer),
                                            detail::h(v_layer), d_pos, 0, T, head_dim, num_q_heads, num_kv_heads,
                                            max_ctx, rope_table, neox ? 1 : 0, stream));
}
// storeKvQ8Kernel (cuda_math_kernels.cu:409-432)
inline void storeKvQ8(const void* k, const void* v, int8_t* k_layer, void* k_scale, int8_t* v_layer, void* v_scale,
                      const int* d_pos, int T, int kv_dim, int max_ctx, hipStream_t stream) {
    detail::check(friday_attn_store_kv_q8(detail::h(k), detail::h(v), k_layer, detail::h(k_scale), v_layer,
                                          detail::h(v_scale), d_pos, 0, T, kv_dim, max_ctx, stream));
}

}  // namespace friday_attn

// ---- int8-activation matmuls: hpc_k_quants.h:39-68 and prefill_kernels.h:15-25
namespace friday_hpc {

enum class Q8Kind { None, Q2_K, Q3_K, Q4_K, Q5_K, Q6_K, Q8_0 };  // codes = FA_KQ_*

namespace detail {
struct Q8Scratch {
    int8_t* xq = nullptr;
    float* xd = nullptr;
    int cap = 0;
    std::vector<void*> retired;  // outgrown buffers: a captured graph may still use them
};
inline Q8Scratch& scratch() {
    static Q8Scratch s;
    return s;
}
}  // namespace detail

// The activation scratch shared by quantizeQ8 and gemvQ8 (hpc_k_quants.h:51-57, the
// reference's ensureQ8Scratch at hpc_k_quants.cu:869-878): allocate it for vectors of up to
// K values before any HIP graph capture. Growing it during a capture throws. The buffers it
// outgrows are not freed (graphs captured earlier keep using them) until the process ends.
inline void ensureQ8Scratch(int K, hipStream_t stream) {
    auto& s = detail::scratch();
    if (K <= s.cap) return;
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    if (hipStreamIsCapturing(stream, &cs) == hipSuccess && cs != hipStreamCaptureStatusNone)
        throw std::runtime_error("ensureQ8Scratch: cannot grow the scratch during stream capture");
    if (s.xq) s.retired.push_back(s.xq);
    if (s.xd) s.retired.push_back(s.xd);
    s.xq = nullptr;
    s.xd = nullptr;
    s.cap = 0;
    const int cap = (K + 255) / 256 * 256;
    if (hipMalloc(reinterpret_cast<void**>(&s.xq), (size_t)cap) != hipSuccess ||
        hipMalloc(reinterpret_cast<void**>(&s.xd), (size_t)cap / 32 * sizeof(float)) != hipSuccess)
        throw std::runtime_error("ensureQ8Scratch: hipMalloc failed");
    s.cap = cap;
}
inline void quantizeQ8(const void* x, int K, hipStream_t stream) {
    ensureQ8Scratch(K, stream);
    friday_attn::detail::check(
        friday_quantize_q8_rows(friday_attn::detail::h(x), 1, K, detail::scratch().xq, detail::scratch().xd, stream));
}
inline void quantizeQ8Rows(const void* x, int rows, int K, int8_t* xq, float* xd, hipStream_t stream) {
    friday_attn::detail::check(friday_quantize_q8_rows(friday_attn::detail::h(x), rows, K, xq, xd, stream));
}
inline bool gemvQ8Supported(Q8Kind k) { return k != Q8Kind::None; }
inline void gemvQ8(Q8Kind kind, const void* W, void* y, int K, int N, hipStream_t stream, const void* W2 = nullptr,
                   void* y2 = nullptr, const float* bias = nullptr, const void* res = nullptr) {
    if (!gemvQ8Supported(kind)) {
        std::fprintf(stderr, "gemvQ8: unsupported type\n");
        std::abort();
    }
    friday_attn::detail::check(friday_gemv_q8((int)kind, W, detail::scratch().xq, detail::scratch().xd, K, N,
                                              friday_attn::detail::h(y), stream, W2, friday_attn::detail::h(y2),
                                              bias, friday_attn::detail::h(res)));
}

}  // namespace friday_hpc

namespace friday_prefill {

inline bool gemmQ8Supported(friday_hpc::Q8Kind kind, int K) { return friday_gemm_q8_supported((int)kind, K) != 0; }
inline void gemmQ8(friday_hpc::Q8Kind kind, const void* W, const int8_t* xq, const float* xd, int T, int K, int N,
                   void* Y, int ldy, hipStream_t stream, const float* bias = nullptr, const void* res = nullptr) {
    if (!gemmQ8Supported(kind, K)) {  // prefill_kernels.cu:344-347
        std::fprintf(stderr, "gemmQ8: unsupported type, K=%d or device\n", K);
        std::abort();
    }
    friday_attn::detail::check(friday_gemm_q8((int)kind, W, xq, xd, T, K, N, friday_attn::detail::h(Y), ldy, stream,
                                              bias, friday_attn::detail::h(res)));
}

}  // namespace friday_prefill


#endif  // FRIDAY_ATTN_HPP
