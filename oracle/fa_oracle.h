/*
 * CPU oracle for the FRIDAY per-layer KV-cache path (TEST INFRASTRUCTURE ONLY).
 *
 * This library is the checker, never the product: only tests/, the smoke()
 * entry of __graft_entry__.py and the cpu_baseline leg of bench.py may load it.
 * It restates, in plain C, the reference's CPU arithmetic for the path:
 *   - fp16 conversion/rounding     cpu_kquants.cpp:17-58, 141-163
 *   - RoPE                         cpu_ops.cpp:26-43
 *   - KV append (rotated K, raw V)  cpu_backend.cpp:111-116, cuda_math_kernels.cu:363-404
 *   - int8 KV append               cuda_math_kernels.cu:409-432
 *   - GQA decode attention         cpu_ops.cpp:45-83
 *   - split-K partials + LSE merge attention_kernels.cu:131-235, 267-411
 *   - causal prefill attention     attention_kernels.h:36-45 (row t == decode at p0+t+1)
 *   - paged addressing             experimental/runtime/src/kernels/paged_attention.cu:18-45
 *   - bf16 prefill (no counterpart: the reference caches are fp16): the causal prefill
 *     above with bf16 inputs widened exactly and the output rounded to bf16
 *
 * fp16 values travel as uint16_t bit patterns. Every accumulation is fp32 in
 * the reference's order unless a function name says f64.
 */
#ifndef FA_ORACLE_H
#define FA_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* fp16 helpers */
float or_half_to_float(uint16_t h);
uint16_t or_float_to_half(float f);
/* NaN -> 0, clamp to +-65504, then RNE to fp16 precision (returned as float). */
float or_round_to_half(float x);
/* bf16 <-> fp32 (round to nearest even); or_round_to_bf16: NaN -> 0, then rounded */
float or_bf16_to_float(uint16_t b);
uint16_t or_float_to_bf16(float f);
float or_round_to_bf16(float x);
void or_halves_to_floats(const uint16_t* h, float* f, size_t n);
void or_floats_to_halves(const float* f, uint16_t* h, size_t n);

/* (cos, sin) table: cs[(p * (head_dim/2) + i) * 2 + {0,1}] for p < max_pos. */
void or_rope_table(float* cs, int max_pos, int head_dim, float freq_base, const float* freq_factors);

/* RoPE + KV append for T tokens at positions pos0 .. pos0+T-1.
 * q [T][Hq*d], k, v [T][Hkv*d] fp16; q and k are rotated in place;
 * k_cache/v_cache [max_ctx][Hkv*d] fp16 (row pos0+t receives rotated k and raw v);
 * either cache pointer may be NULL (rotation only). */
void or_rope_append(uint16_t* q, uint16_t* k, const uint16_t* v, uint16_t* k_cache, uint16_t* v_cache,
                    const float* cs, int pos0, int T, int Hq, int Hkv, int head_dim, int neox);

/* int8 append (storeKvQ8Kernel): per 32 values amax (NaN->0), dh = fp16(amax/127),
 * q = clamp(rne(x / dh)) using 1/float(dh). Row layout [pos][kv_dim], scales [pos][kv_dim/32]. */
void or_store_kv_q8(const uint16_t* k, const uint16_t* v, int8_t* k_cache, uint16_t* k_scale, int8_t* v_cache,
                    uint16_t* v_scale, int pos0, int T, int kv_dim);

/* Decode attention over positions [0, S) of a contiguous cache with row stride
 * kv_stride elements. fp16 cache (kq8 == NULL) or int8 cache with scales. out is
 * fp32 holding fp16-rounded values ([Hq*d]). Sequential fp32 order of cpu_ops.cpp:45-83. */
void or_decode_attention(const uint16_t* q, const uint16_t* k_cache, const uint16_t* v_cache, float* out, int S,
                         int Hq, int Hkv, int head_dim, int kv_stride);
void or_decode_attention_q8(const uint16_t* q, const int8_t* k_cache, const uint16_t* k_scale, const int8_t* v_cache,
                            const uint16_t* v_scale, float* out, int S, int Hq, int Hkv, int head_dim);
/* Same softmax rules in double precision, no fp16 rounding of the output. */
void or_decode_attention_f64(const uint16_t* q, const uint16_t* k_cache, const uint16_t* v_cache, double* out, int S,
                             int Hq, int Hkv, int head_dim, int kv_stride);

/* Split-K restatement: nsplit chunks of ceil(S/nsplit) positions, per-split
 * local max/sum/unnormalised PV, then the LSE merge. out as above. */
void or_decode_attention_split(const uint16_t* q, const uint16_t* k_cache, const uint16_t* v_cache, float* out, int S,
                               int Hq, int Hkv, int head_dim, int nsplit);
/* LSE merge of nsp partials for one head: part_o [nsp][d], part_m/part_l [nsp]. */
void or_lse_merge(const float* part_o, const float* part_m, const float* part_l, int nsp, int head_dim, float* out);

/* Causal prefill: query t at position p0+t attends to [0, p0+t]. q/out [T][Hq*d]. */
void or_prefill_attention(const uint16_t* q, const uint16_t* k_cache, const uint16_t* v_cache, float* out, int T,
                          int p0, int Hq, int Hkv, int head_dim);
void or_prefill_attention_q8(const uint16_t* q, const int8_t* k_cache, const uint16_t* k_scale, const int8_t* v_cache,
                             const uint16_t* v_scale, float* out, int T, int p0, int Hq, int Hkv, int head_dim);
/* Blocked evaluation of the prefill rows above with the same fp32 operations per value
 * (test infrastructure for checking whole chunks): widen a cache once (kind 0 fp16, 1 int8
 * with scales, 2 bf16) into kt [Hkv][hd][S] and vf [S][Hkv*hd], then compute rows. */
void or_prefill_widen(const void* kc, const uint16_t* ks, const void* vc, const uint16_t* vs, int kind, int S,
                      int Hkv, int hd, float* kt, float* vf);
void or_prefill_rows_f32(const uint16_t* q, const float* kt, const float* vf, int Smax, float* out, int T, int p0,
                         int Hq, int Hkv, int hd, int bf16);
/* or_prefill_attention with bf16 q / caches and the bf16 output rule (no reference counterpart) */
void or_prefill_attention_bf16(const uint16_t* q, const uint16_t* k_cache, const uint16_t* v_cache, float* out, int T,
                               int p0, int Hq, int Hkv, int hd);

/* Paged layout: pool [num_pages][page][kv_dim]; block_table row of one sequence.
 * Gathers positions [0, S) into a contiguous [S][kv_dim] buffer. */
void or_paged_gather(const uint16_t* pool, const int32_t* block_table, int S, int page, int kv_dim, uint16_t* dst);

/* ---- prefill projection GEMM (gemm_oracle.c); kind = friday_hpc::Q8Kind code 1..6 ---- */
size_t or_q8_row_bytes(int kind, int K);
/* x [rows][K] fp16 -> xq [rows][K] int8, xd [rows][K/32] fp32 */
void or_quantize_q8_rows(const uint16_t* x, int rows, int K, int8_t* xq, float* xd);
/* 32-value block blk of a weight row: value l = ws[l/16] * q[l] - wm[l/16] */
int or_kq_block(int kind, const uint8_t* row, int blk, int32_t* q, float* ws, float* wm);
void or_dequant_row(int kind, const uint8_t* row, int K, float* out);
/* Y[t*ldy + n] (fp16, epilogue with optional bias[N] and res (same layout as Y));
 * yraw [T][N] (optional) gets the fp32 sums before the epilogue */
void or_gemm_q8(int kind, const uint8_t* W, const int8_t* xq, const float* xd, int T, int K, int N,
                const float* bias, const uint16_t* res, int ldy, uint16_t* Y, float* yraw);

#ifdef __cplusplus
}
#endif
#endif
