/*
 * friday_attn — MI355X (gfx950) KV-cache path of the FRIDAY inference engine:
 * RoPE + KV append, GQA decode attention (split-K + log-sum-exp merge), causal
 * prefill attention on MFMA, and paged multi-sequence decode.
 *
 * C ABI. Plain pointers and sizes; fp16 tensors are passed as uint16_t bit
 * patterns (IEEE binary16), int8 caches as int8_t, `stream` is a hipStream_t
 * (NULL = the null stream). Every entry point:
 *   - returns FA_OK (0) or a negative status; friday_attn_last_error() gives the
 *     message of the calling thread's last failure (the reference throws
 *     std::runtime_error or aborts at the same points);
 *   - validates its arguments on the host before any HIP call;
 *   - never allocates and never synchronises: launches are asynchronous on
 *     `stream` and may be captured into a HIP graph;
 *   - reads sequence lengths from device memory when given `d_pos`, so a
 *     captured launch replays correctly for a new position.
 *
 * Layouts (same as the reference Transformer, transformer.cpp:483-503,852-853):
 *   q, out            [T][num_heads * head_dim]            fp16
 *   k/v layer cache   [max_ctx][num_kv_heads * head_dim]   fp16, or int8 with
 *                     fp16 scales [max_ctx][num_kv_heads * head_dim / 32]
 *   paged pool        [num_pages][16][num_kv_heads * head_dim] fp16, addressed
 *                     through block_table[seq][pos / 16]
 * head_dim is 64 or 128 (the reference GPU kernels accept 128 only,
 * attention_kernels.cu:416); num_heads % num_kv_heads == 0.
 */
#ifndef FRIDAY_ATTN_H
#define FRIDAY_ATTN_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define FA_OK 0
#define FA_ERR_INVALID (-1)     /* bad shape / null pointer / out of range */
#define FA_ERR_UNSUPPORTED (-2) /* valid but not implemented for these shapes */
#define FA_ERR_LAUNCH (-3)      /* a HIP launch or copy failed */
#define FA_ERR_WORKSPACE (-4)   /* workspace too small or missing */
#define FA_ERR_TIMEOUT (-5)     /* a fused merge gave up waiting (friday_attn_decode_workspace_status) */

#define FA_PAGE_TOKENS 16 /* paged_kv_cache.h:16 KV_BLOCK_SIZE */

/* Message of the calling thread's last failed call ("" if none). */
const char* friday_attn_last_error(void);
/* Library version, major * 10000 + minor * 100 + patch. */
int friday_attn_version(void);

/* ---------------- RoPE table (setup) ----------------
 * The reference evaluates theta_i = pos / base^(2i/d) (/ freq_factors[i]) and
 * its cos/sin inside ropeStoreKvKernel (cuda_math_kernels.cu:376-381) and
 * friday_cpu::rope (cpu_ops.cpp:29-32). Here they are evaluated once on the host
 * with the CPU formula into a table [max_ctx][head_dim/2][2] of float (cos, sin),
 * which makes the GPU rotation bit-identical to the reference CPU path. */
size_t friday_attn_rope_table_bytes(int max_ctx, int head_dim);
int friday_attn_rope_table_fill_host(float* table, int max_ctx, int head_dim, float freq_base,
                                     const float* freq_factors_host);
/* Fills on the host and copies into device memory d_table (synchronous; setup only). */
int friday_attn_rope_table_upload(float* d_table, int max_ctx, int head_dim, float freq_base,
                                  const float* freq_factors_host, void* stream);

/* ---------------- KV append ----------------
 * Replaces the launches of ropeStoreKvKernel (cuda_math_kernels.cu:363-404, launched at
 * transformer.cpp:1046-1048 and :1247-1248) and, with k_layer == v_layer == NULL,
 * ropeKernel (cuda_math_kernels.cu:331-359). Token t of T sits at position
 * P + t with P = *d_pos when d_pos != NULL, else P = pos. q [T][Hq*d] and
 * k [T][Hkv*d] are rotated in place (fp32 math, NaN -> 0, clamp, RNE fp16);
 * rotated k and raw v are written to row P + t of k_layer / v_layer.
 * Positions >= max_ctx are skipped (the reference would write out of bounds). The kernel
 * moves 16-byte chunks: q, k, v and the caches must be 16-byte aligned (FA_ERR_INVALID
 * otherwise; device allocations and row offsets of the reference's layout always are). */
int friday_attn_rope_store_kv(uint16_t* q, uint16_t* k, const uint16_t* v, uint16_t* k_layer, uint16_t* v_layer,
                              const int* d_pos, int pos, int T, int head_dim, int num_q_heads, int num_kv_heads,
                              int max_ctx, const float* rope_table, int neox, void* stream);

/* int8 KV append: replaces storeKvQ8Kernel (cuda_math_kernels.cu:409-432, launched at
 * transformer.cpp:1038-1040, 1233-1234). Per 32 values: dh = fp16(amax / 127),
 * q = clamp(rne(x / dh), +-127). */
int friday_attn_store_kv_q8(const uint16_t* k, const uint16_t* v, int8_t* k_layer, uint16_t* k_scale,
                            int8_t* v_layer, uint16_t* v_scale, const int* d_pos, int pos, int T, int kv_dim,
                            int max_ctx, void* stream);

/* ---------------- decode attention ----------------
 * friday_attn::launchDecodeAttention (attention_kernels.h:18-20, .cu:415-428):
 * single-query GQA attention over positions [0, seq_len). Needs no workspace. */
int friday_attn_decode_attention(const uint16_t* q, const uint16_t* k_cache, const uint16_t* v_cache, uint16_t* out,
                                 int seq_len, int num_heads, int num_kv_heads, int head_dim, void* stream);
/* friday_attn::launchDecodeAttentionDevPos (attention_kernels.h:24-25, .cu:430-442):
 * sequence length *d_pos + 1, read on the device; max_seq_len bounds it. */
int friday_attn_decode_attention_dev_pos(const uint16_t* q, const uint16_t* k_cache, const uint16_t* v_cache,
                                         uint16_t* out, const int* d_pos, int max_seq_len, int num_heads,
                                         int num_kv_heads, int head_dim, void* stream);
/* friday_attn::decodeAttentionFitsSharedMemory (attention_kernels.h:26, .cu:488-490).
 * The LDS use here does not grow with the context: 1 for every max_seq_len > 0. */
int friday_attn_decode_fits_shared_memory(int max_seq_len);
/* friday_attn::splitAttentionWorkspaceBytes (attention_kernels.h:32, .cu:444-447):
 * bytes of workspace for friday_attn_decode_attention_split, any head_dim <= 128. */
size_t friday_attn_split_workspace_bytes(int num_heads, int max_seq_len);
/* friday_attn::launchDecodeAttentionSplit (attention_kernels.h:35-38, .cu:449-486):
 * split-K (flash-decoding) attention + LSE merge. Length = d_pos ? *d_pos + 1 : seq_len.
 * k_scale/v_scale non-NULL: int8 caches with fp16 scales per 32 values. */
int friday_attn_decode_attention_split(const uint16_t* q, const void* k_cache, const void* v_cache, uint16_t* out,
                                       int seq_len, const int* d_pos, int max_seq_len, int num_heads,
                                       int num_kv_heads, int head_dim, void* workspace, size_t workspace_bytes,
                                       void* stream, const uint16_t* k_scale, const uint16_t* v_scale);

/* Zeroes a decode workspace (a small fill kernel, no hipMemset node). Required once,
 * after allocation, before the workspace is used by friday_attn_decode_attention_fused
 * or friday_attn_paged_decode_attention; those calls leave it ready for the next call
 * (each group's arrival counter and its base advance together, nothing is reset).
 * A workspace is laid out for one batch size (batch * num_heads counter slots first, the
 * split partials after them; a contiguous call counts as batch 1): calls with another
 * batch size or head count may share it only after it is initialised again. */
int friday_attn_decode_workspace_init(void* workspace, size_t workspace_bytes, void* stream);
/* No counterpart in the reference (its merge is a second kernel and cannot wait). The
 * fused merge waits, bounded (1 s), for every split of its group to arrive; a merger that
 * gives up sets a sticky error word in the workspace and merges nothing, so that call's
 * output and rotated q are not written, and the workspace's counters are no longer in step.
 * This query (a 4-byte copy and a synchronisation of `stream`: not for use under capture)
 * returns FA_ERR_TIMEOUT once that has happened on `workspace`, FA_OK otherwise;
 * friday_attn_decode_workspace_init clears it. Covers every call that takes a workspace
 * (fused, step, int8 step, quant step, paged). */
int friday_attn_decode_workspace_status(const void* workspace, size_t workspace_bytes, void* stream);
/* No counterpart in the reference (a tuning switch of this implementation). Chooses, for
 * the whole process, how later contiguous decode launches place their workgroups and merge
 * their splits. local_merge = 1 (fp16 caches): when the fixed mergers serve the launch and
 * every (kv head, head block) group maps to one XCD (the group count a multiple of 8), the
 * splits hand their partials to the mergers through that XCD's L2 (flag words in the
 * workspace) instead of through device-coherent memory; results are bit-identical.
 * split_major = 1 (fp16 caches): the workgroups of one split (all groups) are dealt to one
 * XCD, as the int8 kernel always does (this excludes local_merge); bit-identical.
 * kv_pair = 1 (fp16 and int8 caches, G <= 16, an even kv head count): a workgroup serves two
 * adjacent kv heads (four waves each), so it reads two adjacent kv-head slices of every
 * cache row; the split bound follows the halved group count, so results agree with the
 * other forms within the decode tolerance, not bit for bit. -1 restores the environment's
 * choice (FRIDAY_ATTN_LOCAL_MERGE, FRIDAY_ATTN_SPLIT_MAJOR, FRIDAY_ATTN_KV_PAIR; default 0).
 * Paged launches keep one kv head per workgroup and the counter merge. A captured launch
 * keeps the form it was recorded with. The local form needs a one-time placement check per
 * device (a few small launches and a synchronisation; no allocation): local_merge = 1 runs
 * it here on the null stream; otherwise the first launch that wants the form and is not
 * being captured runs it on its own stream, and until then launches use the counter form. */
int friday_attn_set_decode_form(int local_merge, int split_major, int kv_pair);
/* launchDecodeAttentionSplit in one kernel: the split partials are merged by the last
 * few workgroups of each kv head (the ones dispatched last), each over a slice of the
 * columns, once an arrival counter in the workspace shows every split stored, instead
 * of by a second kernel. Same arguments, same results bit for bit as
 * friday_attn_decode_attention_split; the workspace must have been initialised with
 * friday_attn_decode_workspace_init. Calls that share a workspace must not overlap. */
int friday_attn_decode_attention_fused(const uint16_t* q, const void* k_cache, const void* v_cache, uint16_t* out,
                                       int seq_len, const int* d_pos, int max_seq_len, int num_heads,
                                       int num_kv_heads, int head_dim, void* workspace, size_t workspace_bytes,
                                       void* stream, const uint16_t* k_scale, const uint16_t* v_scale);

/* One decode layer-step in a single launch: friday_attn_rope_store_kv (T = 1) followed
 * by friday_attn_decode_attention_fused over S = P + 1 positions, P = *d_pos (or pos),
 * i.e. the sequence transformer.cpp:1044-1052 issues as two launches (ropeStoreKvKernel,
 * then launchDecodeAttentionSplit). Every workgroup rotates q itself; the one whose
 * split holds position P writes rotated k and raw v into row P of k_layer / v_layer;
 * the rotated q is written back to q. Unlike ropeStoreKvKernel, k is not rotated in
 * place (the rotated row lives in the cache). Outputs are bit-identical to the
 * two-call sequence. Workspace as for friday_attn_decode_attention_fused
 * (friday_attn_split_workspace_bytes(num_heads, max_ctx), initialised once). */
int friday_attn_decode_step(uint16_t* q, const uint16_t* k, const uint16_t* v, uint16_t* k_layer, uint16_t* v_layer,
                            uint16_t* out, const int* d_pos, int pos, int max_ctx, int num_heads, int num_kv_heads,
                            int head_dim, const float* rope_table, int neox, void* workspace, size_t workspace_bytes,
                            void* stream);

/* No counterpart in the reference. For callers that cannot allocate device memory (code
 * under HIP graph capture, tight serving loops, harnesses that forbid hipMalloc):
 * friday_attn_decode_step with the workspace replaced by a scratch the library holds in
 * device memory, 4 MiB per GPU: 1 MiB of counter slots (up to 4096 query heads) and 3 MiB
 * of split partials. Allocates nothing and launches nothing but the step: the scratch is zero
 * when the library's code object loads, and the first call on a device only looks up its
 * address, so that call may be made under stream capture. Results are bit-identical to
 * friday_attn_decode_step. All calls on one GPU share its scratch, whatever their head
 * counts: calls that overlap (other streams, concurrent graph replays) race and must be
 * serialised by the caller. FA_ERR_WORKSPACE when the call would need more than that. */
int friday_attn_decode_step_noalloc(uint16_t* q, const uint16_t* k, const uint16_t* v, uint16_t* k_layer,
                                    uint16_t* v_layer, uint16_t* out, const int* d_pos, int pos, int max_ctx,
                                    int num_heads, int num_kv_heads, int head_dim, const float* rope_table, int neox,
                                    void* stream);

/* int8 KV cache (FRIDAY --kv q8): the same single launch as friday_attn_decode_step
 * for the sequence transformer.cpp:1035-1040, 1049-1051 issues as three launches:
 * ropeStoreKvKernel with null caches (q and k rotated), storeKvQ8Kernel (rotated k and
 * v quantized into row P: int8 values plus one fp16 scale per 32 values,
 * cuda_math_kernels.cu:409-432), then launchDecodeAttentionSplit with k_scale/v_scale.
 * Cache layout [max_ctx][Hkv*d] int8, scales [max_ctx][Hkv*d/32] fp16. Outputs, cache
 * row and scales are bit-identical to that sequence; k is not rotated in place. */
int friday_attn_decode_step_q8(uint16_t* q, const uint16_t* k, const uint16_t* v, int8_t* k_layer,
                               uint16_t* k_scale, int8_t* v_layer, uint16_t* v_scale, uint16_t* out,
                               const int* d_pos, int pos, int max_ctx, int num_heads, int num_kv_heads,
                               int head_dim, const float* rope_table, int neox, void* workspace,
                               size_t workspace_bytes, void* stream);

/* friday_attn_decode_step that also writes the attention output in the int8 activation
 * format of the next matmul: out_q [Hq*d] int8 and out_d [Hq*d/32] fp32, bit for bit what
 * friday_quantize_q8_rows(out, 1, Hq*d, ...) (quantizeQ8, hpc_k_quants.cu:386-400) gives.
 * Replaces ropeStoreKvKernel + launchDecodeAttentionSplit + quantizeQ8 of gpuLayerFused
 * (transformer.cpp:1046-1051, 1057) with one launch; the O-projection gemvQ8 then reads
 * out_q / out_d (friday_gemv_q8). No reference counterpart as a single entry point. */
int friday_attn_decode_step_quant(uint16_t* q, const uint16_t* k, const uint16_t* v, uint16_t* k_layer,
                                  uint16_t* v_layer, uint16_t* out, int8_t* out_q, float* out_d, const int* d_pos,
                                  int pos, int max_ctx, int num_heads, int num_kv_heads, int head_dim,
                                  const float* rope_table, int neox, void* workspace, size_t workspace_bytes,
                                  void* stream);

/* ---------------- prefill attention ----------------
 * friday_attn::prefillAttentionSupported / launchPrefillAttention
 * (attention_kernels.h:46-50, .cu:649-684): causal attention of T queries at
 * positions *d_pos0 + t over cache positions [0, *d_pos0 + t] (the T new rows are
 * already appended). q/out [T][num_heads*head_dim]. Runs on gfx950 MFMA.
 * Returns 1 / 0 for supported / unsupported. */
int friday_attn_prefill_supported(int num_heads, int num_kv_heads, int head_dim);
int friday_attn_prefill_attention(const uint16_t* q, const void* k_cache, const void* v_cache, uint16_t* out, int T,
                                  const int* d_pos0, int num_heads, int num_kv_heads, int head_dim, void* stream,
                                  const uint16_t* k_scale, const uint16_t* v_scale);
/* The same causal prefill with bf16 q, K/V cache and out (bf16 MFMA operands, fp32
 * scores and softmax, weights rounded to bf16 for the PV product, output NaN -> 0 and
 * round to nearest even bf16). No counterpart in the reference, whose caches are fp16
 * (attention_kernels.cu:513-645); it serves callers that keep bf16 activations and
 * caches, the input type the prefill benchmark allows besides fp16. */
int friday_attn_prefill_attention_bf16(const uint16_t* q, const uint16_t* k_cache, const uint16_t* v_cache,
                                       uint16_t* out, int T, const int* d_pos0, int num_heads, int num_kv_heads,
                                       int head_dim, void* stream);

/* ---------------- paged multi-sequence decode ----------------
 * Semantics of the (unbuilt) experimental paged cache: 16-token pages, physical
 * page = block_table[seq * block_table_stride + pos / 16], row pos % 16
 * (experimental/runtime/src/kernels/paged_attention.cu:18-45, paged_kv_cache.h:16).
 * seq_lens[b] = context length of sequence b AFTER its append (device int32).
 * Every sequence gives the same result, bit for bit, as the contiguous-cache
 * friday_attn_decode_attention_split over the same logical rows. The decode uses the
 * fused merge: its workspace must be initialised once with friday_attn_decode_workspace_init. */
size_t friday_attn_paged_workspace_bytes(int batch, int num_heads, int max_seq_len);
/* Append one token per sequence at position seq_lens[b] - 1 (RoPE as above, same
 * 16-byte alignment rule). q [B][Hq*d], k/v [B][Hkv*d] rotated in place. */
int friday_attn_paged_rope_store_kv(uint16_t* q, uint16_t* k, const uint16_t* v, uint16_t* k_pool, uint16_t* v_pool,
                                    const int32_t* block_table, int block_table_stride, const int32_t* seq_lens,
                                    int batch, int head_dim, int num_q_heads, int num_kv_heads, int max_ctx,
                                    const float* rope_table, int neox, void* stream);
/* Append (position seq_lens[b] - 1) plus decode attention for all sequences in one
 * launch: friday_attn_paged_rope_store_kv followed by friday_attn_paged_decode_attention,
 * with the same single-launch rules as friday_attn_decode_step (k not rotated in place). */
int friday_attn_paged_decode_step(uint16_t* q, const uint16_t* k, const uint16_t* v, uint16_t* k_pool,
                                  uint16_t* v_pool, uint16_t* out, const int32_t* block_table,
                                  int block_table_stride, const int32_t* seq_lens, int batch, int max_seq_len,
                                  int num_heads, int num_kv_heads, int head_dim, const float* rope_table, int neox,
                                  void* workspace, size_t workspace_bytes, void* stream);
int friday_attn_paged_decode_attention(const uint16_t* q, const uint16_t* k_pool, const uint16_t* v_pool,
                                       uint16_t* out, const int32_t* block_table, int block_table_stride,
                                       const int32_t* seq_lens, int batch, int max_seq_len, int num_heads,
                                       int num_kv_heads, int head_dim, void* workspace, size_t workspace_bytes,
                                       void* stream);

/* ---------------- prefill projection GEMM (int8 activations x K-quant weights) ----------------
 * The batched matmul on either side of prefill attention in prefillLayerFused
 * (transformer.cpp:1194-1207, 1266-1280). Weight kinds are the codes of
 * friday_hpc::Q8Kind (hpc_k_quants.h:39); W holds N rows in the GGML block layout of the
 * kind (row bytes = friday_q8_row_bytes(kind, K)). */
#define FA_KQ_Q2_K 1
#define FA_KQ_Q3_K 2
#define FA_KQ_Q4_K 3
#define FA_KQ_Q5_K 4
#define FA_KQ_Q6_K 5
#define FA_KQ_Q8_0 6
size_t friday_q8_row_bytes(int kind, int K);
/* Replaces friday_hpc::quantizeQ8Rows (hpc_k_quants.h:58-61, hpc_k_quants.cu:898-901):
 * x [rows][K] fp16 -> xq [rows][K] int8, xd [rows][K/32] fp32; per 32 values
 * d = amax / 127, q = clamp(rne(x / d), +-127), exactly as quantize_x_q8_kernel
 * (hpc_k_quants.cu:386-400). K must be a multiple of 32. */
int friday_quantize_q8_rows(const uint16_t* x, int rows, int K, int8_t* xq, float* xd, void* stream);
/* Replaces friday_prefill::gemmQ8Supported (prefill_kernels.h:17-18, prefill_kernels.cu:340):
 * 1 / 0. K must be a multiple of 256. */
int friday_gemm_q8_supported(int kind, int K);
/* Replaces friday_prefill::gemmQ8 (prefill_kernels.h:20-25, prefill_kernels.cu:342-362):
 * Y[t*ldy + n] = sum_k W[n][k] x_t[k] for t < T, n < N, x_t = xq row t scaled by xd per
 * 32 values; epilogue per element as storeY (prefill_kernels.cu:155-171): fp16 rounding,
 * then + bias[n] (fp32) if bias, then res[t*ldy + n] + y (fp16) if res; NaN inputs of
 * each sum count as 0 and sums clamp to +-65504. Y may alias res. T <= 0 is a no-op.
 * W must be 4-byte aligned, xq 16-byte aligned, ldy >= N. Runs on gfx950 fp16 MFMA over
 * operands decoded in LDS; agrees with the reference's integer form within its own GEMM
 * test bar (test_prefill_gemm.cu:111-129: rel-L2 < 1e-3, max |diff| < 1e-2 RMS).
 * A library-held workspace, one per (device, stream), allocated on first use (as the
 * reference's module scratch, hpc_k_quants.cu:869-880), holds the activations dequantised
 * to fp16 once per call and, for shapes whose output tiles do not fill the GPU (e.g.
 * T = 512 with N = 4096, K = 14336), the fp32 partials of a K split, summed in a fixed
 * order so that results do not depend on timing. Under stream capture the workspace is not
 * allocated: a call then dequantises per workgroup and runs unsplit (same values, slower)
 * unless friday_gemm_q8_reserve sized it beforehand. Calls on one stream share its
 * workspace in stream order: a graph that contains friday_gemm_q8 must be replayed on the
 * stream it was captured on, and never concurrently with another replay or call that uses
 * that stream's workspace (friday_gemm_q8_ws with a workspace per graph has no such rule). */
int friday_gemm_q8(int kind, const void* W, const int8_t* xq, const float* xd, int T, int K, int N, uint16_t* Y,
                   int ldy, void* stream, const float* bias, const uint16_t* res);
/* No counterpart in the reference (its GEMM needs no workspace; cf. ensureQ8Scratch,
 * hpc_k_quants.h:52): sizes the workspace of friday_gemm_q8 for (T, K, N) on
 * `stream` ahead of stream capture. FA_ERR_WORKSPACE when called during capture and an
 * allocation would be needed. */
int friday_gemm_q8_reserve(int T, int K, int N, void* stream);
/* No counterpart in the reference: friday_gemm_q8 with a caller-owned workspace, so that
 * each captured graph (or each concurrent stream) can have its own. Size it with
 * friday_gemm_q8_workspace_bytes (0 for invalid shapes), align it to 256 bytes and zero it
 * once with friday_attn_decode_workspace_init before first use; every call leaves its
 * split counters at zero again. Calls that share one workspace must not overlap.
 * FA_ERR_WORKSPACE if it is missing, misaligned or too small. */
size_t friday_gemm_q8_workspace_bytes(int T, int K, int N);
int friday_gemm_q8_ws(int kind, const void* W, const int8_t* xq, const float* xd, int T, int K, int N, uint16_t* Y,
                      int ldy, void* stream, const float* bias, const uint16_t* res, void* workspace,
                      size_t workspace_bytes);
/* Replaces friday_hpc::gemvQ8 (hpc_k_quants.h:64-68, hpc_k_quants.cu:904-931), the decode
 * GEMV with int8 activations (the O-projection after attention, transformer.cpp:1057-1059):
 * y[n] = sum_k W[n][k] x[k] for one vector x given as xq [K] int8 and xd [K/32] fp32 (the
 * output of friday_quantize_q8_rows with rows = 1; the reference keeps them in a hidden
 * scratch filled by quantizeQ8). If W2, rows of W2 go to y2 in the same launch. Epilogue
 * as friday_gemm_q8 with bias[n] and res[n] (res may alias y), applied to y and y2 alike
 * (storeQ8, hpc_k_quants.cu:422-437). Per 32 values the integer dot products are exact
 * (v_dot4_i32_i8) and scaled in fp32. K a multiple of 256 (of 32 for Q8_0); W, W2 4-byte
 * aligned, xq 16-byte aligned. */
int friday_gemv_q8(int kind, const void* W, const int8_t* xq, const float* xd, int K, int N, uint16_t* y,
                   void* stream, const void* W2, uint16_t* y2, const float* bias, const uint16_t* res);

#ifdef __cplusplus
}
#endif
#endif /* FRIDAY_ATTN_H */
