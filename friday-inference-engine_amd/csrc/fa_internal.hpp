// Internal launch interface between the C-ABI layer (fa_api.cpp) and the
// kernel translation units. Arguments are validated by the caller.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

namespace fa {

// ---- split-K partition, a function of the context length only ----
// Each workgroup (4 waves x 32-position tiles) covers `chunk` positions, a
// multiple of 128: about S / min_chunk splits, at most max_splits per (sequence,
// kv head head block). Because the partition depends on S (and the two library
// constants) alone, a paged sequence and a contiguous cache with the same rows
// reduce in the same order, so their outputs are bit-identical.
constexpr int kSpan = 128;
constexpr int kPageTokens = 16;  // paged_kv_cache.h:16 KV_BLOCK_SIZE
constexpr int kMaxSplitsLimit = 128;
// arrival counters of the fused merge sit 256 bytes apart, so that the atomics of
// different head groups do not queue on one cache line
constexpr int kCounterStride = 64;
// Sticky error word of a decode workspace: int index kStatusWord of counter slot 0 (byte 192,
// away from slot 0's counter at 0 and base at 128). A fused merge that gives up waiting for
// its arrival count sets bit kStatusMergeTimeout there; friday_attn_decode_workspace_status
// reports it and friday_attn_decode_workspace_init clears it.
constexpr int kStatusWord = 48;
constexpr unsigned kStatusMergeTimeout = 1u;

__host__ __device__ inline int split_bound(int S, int min_chunk, int max_splits) {
    int ns = S > 0 ? (S + min_chunk - 1) / min_chunk : 1;
    return ns < max_splits ? ns : max_splits;
}
__host__ __device__ inline int split_chunk(int S, int min_chunk, int max_splits) {
    const int ns = split_bound(S, min_chunk, max_splits);
    const int c = S > 0 ? (S + ns - 1) / ns : 1;
    return ((c + kSpan - 1) / kSpan) * kSpan;
}
__host__ __device__ inline int split_count(int S, int min_chunk, int max_splits) {
    if (S <= 0) return 1;
    const int c = split_chunk(S, min_chunk, max_splits);
    return (S + c - 1) / c;
}

// Library-wide partition constants (environment FRIDAY_ATTN_MIN_CHUNK /
// FRIDAY_ATTN_MAX_SPLITS, read once); see fa_api.cpp.
int min_chunk();
int max_splits();
int splits_for(int Hkv, int ngb);
int device_cus();  // compute units of the current device
int split_major_default();  // FRIDAY_ATTN_SPLIT_MAJOR (0 or 1), read once
int local_merge_default();  // FRIDAY_ATTN_LOCAL_MERGE (0 or 1), read once
int kv_pair_for(bool paged, int Hkv, int ngb);
int q8_deep_default();  // FRIDAY_ATTN_Q8_DEEP (0 or 1), read once
// XCD-local merge placement check of the current device (once; not while `stream` captures)
bool local_placement_ok(hipStream_t stream);  // kv heads per decode workgroup (FRIDAY_ATTN_KV_PAIR)

struct DecodeParams {
    const uint16_t* q;         // [B][Hq*D]
    const void* k;             // contiguous layer [max_ctx][kv_dim] or paged pool
    const void* v;
    const uint16_t* k_scale;   // int8 mode: [rows][kv_dim/32]
    const uint16_t* v_scale;
    const int32_t* block_table;  // paged only
    int bt_stride;
    const int32_t* seq_lens;   // paged only: context length per sequence
    const int* d_pos;          // contiguous: S = *d_pos + 1 when non-null
    int seq_len;               // contiguous: S when d_pos is null
    int max_seq;               // S is clamped to this (grid was sized for it)
    float* part_o;             // [B*Hq][nsplit_grid][D]
    float* part_ml;            // [B*Hq][nsplit_grid][2]  (max in log2 units, sum)
    int* counters;             // fused merge: [B][Hkv*ngb] arrival counters (zero between launches); null: merge kernel
    uint16_t* out;             // [B][Hq*D]
    int8_t* out_q;             // optional: out quantised per 32 values (quantizeQ8 rule), [B][Hq*D]
    float* out_d;              // with out_q: the fp32 scales, [B][Hq*D/32]
    int Hq, Hkv, G, ngb, nsplit_grid, kv_dim;
    int single;                // 1: one split covers the whole context, no merge
    int min_chunk, max_splits; // split partition constants
    int merge_slices;          // fused merge: column slices over the last splits, 0 = the last arriver merges (set by the launcher)
    float scale2;              // softmax scale * log2(e)
    // fused RoPE + KV append (decode step): the kernel rotates q itself, the
    // workgroup owning position S-1 rotates k and writes the new K/V row, and the
    // rotated q is written back to `q`. Null rope_table: plain decode.
    const float* rope_table;   // [max_ctx][D/2][2]
    const uint16_t* k_new;     // [B][kv_dim] raw k of the new token
    const uint16_t* v_new;     // [B][kv_dim] v of the new token
    int neox;
    // contiguous fp16 caches: 1 deals the workgroups of one split (every group) to one XCD,
    // as the int8 kernel always does; 0 (default) deals the splits of one group to one XCD
    int split_major;
    // fused merge, XCD-local form: per-split flag words [B][Hkv*ngb][nsplit_grid] (in the
    // workspace after the partials) and the launcher's choice of that form
    unsigned* flags;
    int local_merge;
    // kv heads per workgroup (1, or 2 for contiguous caches with G <= 16): set by the host
    // together with the split bound it implies (splits_for over Hkv / kpw groups)
    int kpw;
};

int launch_zero_fill(void* ptr, size_t bytes, hipStream_t stream);
int launch_decode(const DecodeParams& p, int head_dim, int batch, bool paged, bool q8, hipStream_t stream);

struct RopeParams {
    uint16_t* q;
    uint16_t* k;
    const uint16_t* v;
    uint16_t* k_dst;           // contiguous layer or paged pool (null: rotation only)
    uint16_t* v_dst;
    const float* table;        // [max_ctx][D/2][2]
    const int* d_pos;          // contiguous: base position from device
    int pos;                   // contiguous: base position when d_pos is null
    const int32_t* block_table;  // paged
    int bt_stride;
    const int32_t* seq_lens;   // paged: token b at seq_lens[b] - 1
    int T, D, Hq, Hkv, max_ctx, neox;
};

int launch_rope_store(const RopeParams& p, bool paged, hipStream_t stream);

struct Q8StoreParams {
    const uint16_t* k;
    const uint16_t* v;
    int8_t* k_dst;
    uint16_t* ks_dst;
    int8_t* v_dst;
    uint16_t* vs_dst;
    const int* d_pos;
    int pos, T, kv_dim, max_ctx;
};

int launch_store_kv_q8(const Q8StoreParams& p, hipStream_t stream);

struct PrefillParams {
    const uint16_t* q;     // [T][Hq*D]
    const void* k;
    const void* v;
    const uint16_t* k_scale;
    const uint16_t* v_scale;
    uint16_t* out;         // [T][Hq*D]
    const int* d_pos0;
    int T, Hq, Hkv, G;
    float scale2;
    int prefetch2;         // fp16 caches: copy the first two stages at the start (set by the launcher)
};

int launch_prefill(const PrefillParams& p, int head_dim, bool q8, hipStream_t stream);
// bf16 q / K / V / out (fp16 caches only; no counterpart in the reference)
int launch_prefill_bf16(const PrefillParams& p, int head_dim, hipStream_t stream);

// Prefill projection GEMM (kq_gemm.hip). Weight kinds: the codes of friday_hpc::Q8Kind.
enum KqKind { kKqQ2K = 1, kKqQ3K = 2, kKqQ4K = 3, kKqQ5K = 4, kKqQ6K = 5, kKqQ80 = 6 };
struct KqGemmParams {
    const uint8_t* W;      // [N][row_bytes] GGML blocks
    const int8_t* xq;      // [T][K]
    const float* xd;       // [T][K / 32]
    uint16_t* Y;           // row t at Y + t * ldy (fp16)
    const float* bias;     // [N] or null
    const uint16_t* res;   // same layout as Y, or null (may alias Y)
    size_t row_bytes;
    int T, K, N, ldy;
    // K split (ksplit > 1): split z takes the 64-value stages [z sps, (z + 1) sps); the
    // workspace holds per-tile arrival counters (zero between launches) and fp32 partials
    int ksplit = 1, sps = 0;
    int* counters = nullptr;
    float* part = nullptr;
    // optional [T][K] fp16 buffer: the launch first dequantises xq / xd into it once, and
    // the GEMM stages fp16 activations from it (null: each workgroup dequantises its tile)
    const uint16_t* xh = nullptr;
};
// GEMM workspace: a fixed region of kKqMaxCounters split counters (kCounterStride ints
// apart; each launch leaves the counters it used at zero, so launches of any shape can
// share one workspace), the fp16 activations [T][K], then the split partials.
constexpr int kKqMaxCounters = 4096;
struct KqPlan {
    int ksplit, sps;
    bool xh;               // stage fp16 activations from the workspace (T K 2 < 4 GiB: 32-bit offsets)
    size_t xh_off;         // byte offset of the fp16 activations
    size_t part_off;       // byte offset of the partials (ksplit > 1)
    size_t bytes;          // whole workspace
};
KqPlan kq_gemm_plan(int T, int K, int N);
int launch_kq_gemm(int kind, const KqGemmParams& p, hipStream_t stream);
struct KqGemvParams {
    const uint8_t* W;      // [N][row_bytes]
    const uint8_t* W2;     // optional second matrix (rows N .. 2N - 1 of the launch), or null
    const int8_t* xq;      // [K]
    const float* xd;       // [K / 32]
    uint16_t* y;           // [N]
    uint16_t* y2;          // [N] for W2
    const float* bias;     // [N] or null (indexed by the row within its matrix)
    const uint16_t* res;   // [N] or null (may alias y)
    size_t row_bytes;
    int K, N;
};
int launch_kq_gemv(int kind, const KqGemvParams& p, hipStream_t stream);
int launch_quantize_q8_rows(const uint16_t* x, int rows, int K, int8_t* xq, float* xd, hipStream_t stream);

}  // namespace fa
