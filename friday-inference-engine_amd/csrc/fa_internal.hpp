// Internal launch interface between the C-ABI layer (fa_api.cpp) and the
// kernel translation units. Arguments are validated by the caller.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

namespace fa {

// ---- split-K partition, a function of the context length only ----
// Each workgroup (4 waves x 32-position tiles) covers `chunk` positions, a
// multiple of 128. Up to kNsplitCap splits per (sequence, kv head). Because the
// partition depends on S alone, a paged sequence and a contiguous cache with
// the same rows reduce in the same order (bit-identical outputs).
constexpr int kSpan = 128;
constexpr int kPageTokens = 16;  // paged_kv_cache.h:16 KV_BLOCK_SIZE
constexpr int kNsplitCap = 128;

__host__ __device__ inline int split_chunk(int S) {
    const int t = (S + kSpan - 1) / kSpan;
    const int ns = t < kNsplitCap ? t : kNsplitCap;
    return ns > 0 ? kSpan * ((t + ns - 1) / ns) : kSpan;
}
__host__ __device__ inline int split_count(int S) {
    if (S <= 0) return 1;
    const int c = split_chunk(S);
    return (S + c - 1) / c;
}

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
    uint16_t* out;             // [B][Hq*D]
    int Hq, Hkv, G, ngb, nsplit_grid, kv_dim;
    int single;                // 1: one split covers the whole context, no merge
    float scale2;              // softmax scale * log2(e)
};

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
};

int launch_prefill(const PrefillParams& p, int head_dim, bool q8, hipStream_t stream);

}  // namespace fa
