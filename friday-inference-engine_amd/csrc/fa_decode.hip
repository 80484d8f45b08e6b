// GQA decode attention for gfx950: split-K (flash-decoding) over the context,
// one workgroup per (split, kv head, head block of 16, sequence) serving the
// whole GQA query group, so each K/V byte is read from HBM once.
//
// Semantics follow decodeAttentionGqaKernel + decodeAttentionCombineKernel
// (attention_kernels.cu:207-235, 267-411) and friday_cpu::decodeAttention
// (cpu_ops.cpp:45-83): score = (q.k) / sqrt(d), NaN score -> -1e30, weights
// exp(s - max) cut to 0 below -50, fp32 accumulation, output NaN -> 0, clamped
// to +-65504, rounded to fp16. Only the order of the fp32 additions differs.
//
// Data flow of one wave per 16-position tile:
//   HBM --(coalesced 16 B loads through a per-tile buffer descriptor, the next tile in
//          flight in registers)--> the wave's LDS tile (padded rows; int8 rows are
//          dequantised to fp16 on the way)
//   S^T[16 x 16] = K[16 x D] . Q^T[D x 16]     v_mfma_f32_16x16x32_f16, K from LDS
//   online softmax on S^T in registers: every lane owns one query head (l % 16)
//   O^T[D x 16] += V^T[D x 16] . P^T[16 x 16]   P stays in the registers the S^T MFMA
//                                               produced it in; V^T by transposing
//                                               LDS reads (ds_read_b64_tr_b16)
// The waves of a workgroup take interleaved tiles of the split and combine through LDS;
// the splits are merged (log-sum-exp) by the last workgroups of each group in the same
// launch (fused merge) or by fa_merge_kernel (the reference's two-launch form).
#include "fa_common.hpp"
#include "fa_internal.hpp"

#include <mutex>
#include <type_traits>
#include <vector>

namespace fa {

#if FA_STAMPS
// Phase timestamps of the bench-only stamps build (compiled with FA_STAMPS=1 into a library
// of its own; the product build has none of this): thread 0 of every decode workgroup writes
// the 100 MHz real-time counter at each phase edge, with ordinary vector stores, into a
// host-set buffer of kStampWords 64-bit words per workgroup (workgroup = linear block id).
__device__ unsigned long long* g_stamps;
#endif

namespace {

// Stamp slots: 0 entry, 1 context length known, 2 q ready (rotation done), 3 wave 0's
// stream end, 4 wave combine done, 5 partial stores completed, 6 arrival counted / count
// observed by a merger, 7 merge stores completed; 8 + i: wave 0's tile i in LDS (i < 16);
// 24 XCC id, 25 HW_ID, 26 split | nsp << 12 | merger slice + 1 << 24, 27 tiles of the split.
constexpr int kStampWords = 32;
__device__ __forceinline__ void stamp_val(int k, unsigned long long v) {
#if FA_STAMPS
    if (g_stamps && threadIdx.x == 0) {
        const size_t wg = blockIdx.x + (size_t)gridDim.x * (blockIdx.y + (size_t)gridDim.y * blockIdx.z);
        g_stamps[wg * kStampWords + k] = v;
    }
#else
    (void)k;
    (void)v;
#endif
}
__device__ __forceinline__ void stamp(int k) {
#if FA_STAMPS
    stamp_val(k, __builtin_amdgcn_s_memrealtime());
#else
    (void)k;
#endif
}

constexpr int kWaves = 4;  // waves per workgroup (the merge kernel, fp16 and paged decode)
constexpr int kThreads = kWaves * 64;
constexpr int kTile = 16;  // positions per wave tile
constexpr int kStages = 1;    // register stages (tiles in flight) per wave
// Contiguous int8 caches: the loop issues about 2.4x the instructions of the fp16 one per
// tile (the dequantisation), and with one wave per SIMD issue time and memory waits add up.
// Eight waves of one tile in flight each (the fp16 bytes in flight per CU, two waves per
// SIMD, one workgroup per CU) let one wave's issue overlap the other's wait.
constexpr int kWavesQ8 = 8;
constexpr int kStagesQ8 = 1;
// waves per workgroup of a decode kernel; KPW = 2: two kv heads per workgroup, four waves each
constexpr int waves_for(bool paged, bool q8, int kpw = 1) { return kpw == 2 ? 2 * kWaves : (q8 && !paged ? kWavesQ8 : kWaves); }
constexpr int kShortStages = 4;  // stages when a wave has at most this many tiles
// Paged grids hold several workgroups per CU: three per CU (at most 168 registers), and at
// most two tiles in flight per wave in the short-split form, where four made the waves of a
// CU issue their loads in one burst and then wait together.
constexpr int kPagedWgsPerCu = 3;
constexpr int kShortStagesPaged = 2;
constexpr int kMergeSlices = 8;  // column slices of the distributed fused merge
constexpr float kLazy2 = 8.0f;   // lazy softmax reference: rescale when a max rises by > 2^8

// ALIAS: the wave combine reuses the tile region (after a barrier), so that two workgroups
// fit in a CU's LDS with room to spare; used by the paged kernel, whose grids hold many
// workgroups per CU. Otherwise the combine has a region of its own and needs no barrier.
template <int D, bool Q8, bool ALIAS, int W>
struct Geo {
    static constexpr int LROW = D * 2 + 16;           // LDS row stride in bytes (fp16 row + 16 B pad)
    static constexpr int KSTEPS = D / 32;             // MFMA k-steps over the head dimension
    static constexpr int DTILES = D / 16;             // 16-wide output tiles of O^T
    // global load geometry: one lane moves 16 bytes
    static constexpr int ROWB = Q8 ? D : D * 2;       // bytes of one kv-head row in the cache
    static constexpr int CPR = ROWB / 16;             // 16-byte chunks per row
    static constexpr int RPI = 64 / CPR;              // rows per wave load
    static constexpr int NLD = kTile / RPI;           // loads per tile per tensor
    static constexpr int WAVE_LDS = 2 * kTile * LROW;  // K and V tile of one wave
    static constexpr int CROW = D + 4;                 // combine row stride in floats (bank spread)
    static constexpr int COMB_LDS = (2 * W * 16 + W * 16 * CROW) * 4;
    static constexpr int TILES = W * WAVE_LDS;
    static constexpr int COMB_OFF = ALIAS ? 0 : TILES;
    static constexpr int QX_OFF = ALIAS ? (TILES > COMB_LDS ? TILES : COMB_LDS) : TILES + COMB_LDS;  // rotated q rows
    // tiles, the wave combine, and (paged: the q rotation goes through LDS) the q rows,
    // 16 heads x D fp16
    static constexpr int LDS = QX_OFF + (ALIAS ? 16 * D * 2 : 0);
    // LDS slot of the 16-byte chunk k (values 8k .. 8k+7) of a tile row. int8 rows: lane c
    // dequantises chunks 2c and 2c+1 and writes them with two instructions; placing even
    // chunks in slots 0 .. D/16-1 and odd ones after them makes each instruction's lanes of
    // one row write 128 contiguous bytes (consecutive slots), free of bank conflicts.
    static __device__ __forceinline__ int slot(int k) { return Q8 ? (k >> 1) + (k & 1) * (D / 16) : k; }
};

__device__ __forceinline__ int context_len(const DecodeParams& p, int b, bool paged) {
    int S = paged ? p.seq_lens[b] : (p.d_pos ? *p.d_pos + 1 : p.seq_len);
    return S < p.max_seq ? S : p.max_seq;
}

template <bool PAGED>
__device__ __forceinline__ size_t row_index(const DecodeParams& p, int b, int pos) {
    if (PAGED) {
        const int phys = p.block_table[(size_t)b * p.bt_stride + (pos >> 4)];
        return (size_t)phys * kPageTokens + (pos & 15);
    }
    return (size_t)pos;
}

// int8 append of one 16-value chunk (two fp16 vectors) of a new K or V row, the lanes
// l and l ^ 1 holding the two halves of a 32-value block (storeKvQ8Kernel,
// cuda_math_kernels.cu:409-432): NaN -> 0, scale = fp16(amax / 127), q = clamp(rne(x /
// scale), +-127) with the division as x * (1 / scale). Returns the 16 codes, the
// scale as a float and its fp16 bits. All 64 lanes of the wave must call it.
__device__ __forceinline__ void quant_chunk16(const h8* x, u4& q, float& scale, uint16_t& bits) {
    float v[16];
    float amax = 0.0f;
#pragma unroll
    for (int e = 0; e < 16; ++e) {
        float t = (float)x[e / 8][e % 8];
        if (__builtin_isnan(t)) t = 0.0f;
        v[e] = t;
        amax = fmaxf(amax, fabsf(t));
    }
    amax = fmaxf(amax, __shfl_xor(amax, 1, 64));
    const _Float16 dh = (_Float16)(amax / 127.0f);
    const float d = (float)dh;
    const float inv = d > 0.0f ? 1.0f / d : 0.0f;
    int8_t c[16];
#pragma unroll
    for (int e = 0; e < 16; ++e) {
        const int qi = (int)rintf(v[e] * inv);
        c[e] = (int8_t)max(-127, min(127, qi));
    }
    q = *reinterpret_cast<const u4*>(c);
    scale = d;
    bits = __builtin_bit_cast(uint16_t, dh);
}

// Writes 4 consecutive output values of one head row (columns 4c..4c+3) and, when the
// caller asked for it, their int8 form: per 32 values d = amax / 127, q = clamp(rne(x / d)),
// exactly as quantize_x_q8_kernel (hpc_k_quants.cu:386-400) applied to the fp16 output.
// The 8 lanes holding one 32-value block (consecutive c, same row) must call it together.
__device__ __forceinline__ void store_out4(const DecodeParams& p, size_t row, int D, int c, h4 o, bool st = true,
                                           int lstride = 1) {
    if (st) reinterpret_cast<h4*>(p.out + row * D)[c] = o;
    if (p.out_q) {
        float v[4], amax = 0.0f;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            v[i] = (float)o[i];
            amax = fmaxf(amax, fabsf(v[i]));
        }
#pragma unroll
        for (int off = 4; off > 0; off >>= 1) amax = fmaxf(amax, __shfl_xor(amax, off * lstride, 64));
        const float d = amax / 127.0f;
        const float inv = d > 0.0f ? 1.0f / d : 0.0f;
        uint32_t packed = 0;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            int q = (int)__builtin_rintf(v[i] * inv);
            q = q < -127 ? -127 : (q > 127 ? 127 : q);
            packed |= (uint32_t)(q & 0xFF) << (8 * i);
        }
        if (st) {
            *reinterpret_cast<uint32_t*>(p.out_q + row * D + 4 * c) = packed;
            if ((c & 7) == 0) p.out_d[(row * D + 4 * c) / 32] = d;
        }
    }
}

// Cross-lane steps within groups of 8 lanes by DPP (no LDS round trip): lane ^ 1, lane ^ 2
// (quad permutations) and lane 7 - i of its group (half-row mirror).
template <int CTRL>
__device__ __forceinline__ float dpp(float v) {
    return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), CTRL, 0xF, 0xF, true));
}
constexpr int kDppXor1 = 0xB1, kDppXor2 = 0x4E, kDppMirror8 = 0x141;
// Sum over the 8 lanes of a group by the tree ((0+1)+(2+3))+((4+5)+(6+7)) in every lane
// (float addition is commutative, so all 8 lanes hold the same bits).
__device__ __forceinline__ float sum8(float v) {
    v += dpp<kDppXor1>(v);
    v += dpp<kDppXor2>(v);
    return v + dpp<kDppMirror8>(v);
}
__device__ __forceinline__ float max8(float v) {
    v = fmaxf(v, dpp<kDppXor1>(v));
    v = fmaxf(v, dpp<kDppXor2>(v));
    return fmaxf(v, dpp<kDppMirror8>(v));
}

// Log-sum-exp merge of the split partials (attention_kernels.cu:207-235) over the output
// columns [4 c0, 4 (c0 + cw)) of nh consecutive head rows row0 ..: per (head, column)
//   M = max_s m_s; w_s = exp(m_s - M) (0 below -50); lane r of the unit's 8 lanes sums
//   L_r = sum w_s l_s and acc_r = sum w_s o_s over s = r, r + 8, ... in increasing order;
//   L and acc are the sums of the 8 lane values by the fixed tree of sum8;
//   out = L > 1e-12 ? acc * (1 / L) : 0, NaN -> 0, clamp, fp16.
// Eight lanes serve one (head, float4 column) unit straight from memory (sc1 loads,
// coherent with the sc1 stores of the other workgroups): up to 32 splits cost each lane
// 4 + 4 loads per unit, and the units of up to four passes of the workgroup are loaded in
// one round trip, with no LDS and no barrier. The order of the arithmetic
// does not depend on the column range or on which workgroup runs it, so the separate
// merge kernel and the column slices of the fused merge give the same bits. cw must be a
// power of two; with out_q, cw and c0 must be multiples of 8.
template <int D, int NT, bool LOCAL = false>  // NT: threads of the workgroup; LOCAL: partials in this XCD's L2
__device__ void merge_cols(const DecodeParams& p, size_t row0, int nh, int nsp, int c0, int cw) {
    constexpr int CP = LOCAL ? kCpolSc0 : kCpolSc1;
    constexpr int kUnitsPerPass = NT / 8;
    constexpr int kBatch = 4;  // passes whose partials are loaded in one round trip
    const int tid = threadIdx.x, r = tid & 7;
    const int wunit = __builtin_amdgcn_readfirstlane(tid >> 6) * 8;  // first unit of this wave in a pass
    const uint32_t ng = (uint32_t)p.nsplit_grid;
    const __amdgpu_buffer_rsrc_t ro = coherent_rsrc(p.part_o, 0x7fffffff);
    const __amdgpu_buffer_rsrc_t rml = coherent_rsrc(p.part_ml, 0x7fffffff);
    const int lc = __builtin_ctz(cw);
    const int units = nh * cw;
    for (int b0 = 0; b0 < units; b0 += kBatch * kUnitsPerPass) {
        if (b0 + wunit >= units) break;  // uniform: no unit left for this wave
        // splits r, r + 8, r + 16, r + 24 (all of them up to 32 splits) of up to kBatch units
        float2 ml[kBatch][4];
        f4 ov[kBatch][4];
#pragma unroll
        for (int k = 0; k < kBatch; ++k) {
            if (k > 0 && b0 + k * kUnitsPerPass + wunit >= units) break;  // uniform: no unit left for this wave
            const int u = min(b0 + k * kUnitsPerPass + (tid >> 3), units - 1);  // lanes past the last unit repeat it
            const uint32_t row = (uint32_t)(row0 + (u >> lc)) * ng;
            const int c = c0 + (u & (cw - 1));
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const uint32_t j = (uint32_t)min(r + 8 * i, nsp - 1);
                ml[k][i] = ld_pol2<CP>(rml, (row + j) * 8);
                ov[k][i] = ld_pol4<CP>(ro, ((row + j) * D + 4 * (uint32_t)c) * 4);
            }
        }
#pragma unroll
        for (int k = 0; k < kBatch; ++k) {
            if (b0 + k * kUnitsPerPass + wunit >= units) break;  // uniform
            const int uu = b0 + k * kUnitsPerPass + (tid >> 3);
            const int u = min(uu, units - 1);
            const int hh = u >> lc, c = c0 + (u & (cw - 1));
            const uint32_t row = (uint32_t)(row0 + hh) * ng;
            float M = -__builtin_inff();
#pragma unroll
            for (int i = 0; i < 4; ++i) M = fmaxf(M, r + 8 * i < nsp ? ml[k][i].x : -__builtin_inff());
            for (int j0 = r + 32; j0 < nsp; j0 += 8)  // beyond 32 splits
                M = fmaxf(M, ld_pol2<CP>(rml, (row + (uint32_t)j0) * 8).x);
            M = max8(M);
            float L = 0.0f;
            f4 acc = f4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const float df = (r + 8 * i < nsp ? ml[k][i].x : -__builtin_inff()) - M;
                const float w = df < kCut2 ? 0.0f : exp2_fast(df);
                L += w * (r + 8 * i < nsp ? ml[k][i].y : 0.0f);
                acc += w * ov[k][i];
            }
            for (int j0 = r + 32; j0 < nsp; j0 += 8) {
                const float2 m2 = ld_pol2<CP>(rml, (row + (uint32_t)j0) * 8);
                const f4 o2 = ld_pol4<CP>(ro, ((row + (uint32_t)j0) * D + 4 * (uint32_t)c) * 4);
                const float df = m2.x - M;
                const float w = df < kCut2 ? 0.0f : exp2_fast(df);
                L += w * m2.y;
                acc += w * o2;
            }
            L = sum8(L);
#pragma unroll
            for (int i = 0; i < 4; ++i) acc[i] = sum8(acc[i]);
            const float inv = L > 1e-12f ? 1.0f / L : 0.0f;
            h4 o;
#pragma unroll
            for (int i = 0; i < 4; ++i) o[i] = out_half(acc[i] * inv);
            store_out4(p, row0 + hh, D, c, o, uu < units && r == 0, 8);
        }
    }
}

// Whole-row merge of nh head rows.
template <int D, int NT>
__device__ __forceinline__ void merge_any(const DecodeParams& p, size_t row0, int nh, int nsp) {
    merge_cols<D, NT>(p, row0, nh, nsp, 0, D / 4);
}

// Column slice k of nslice of the fused merge.
template <int D, int NT, bool LOCAL = false>
__device__ __forceinline__ void merge_slice(const DecodeParams& p, size_t row0, int nh, int nsp, int k, int nslice) {
    const int cw = (D / 4) / nslice;
    merge_cols<D, NT, LOCAL>(p, row0, nh, nsp, k * cw, cw);
}

// Number of column slices the fused merge of a group is spread over: the launcher's
// choice (kMergeSlices), at most nsp, a divisor
// of the D/4 float4 columns, and with out_q at least 8 columns (whole 32-value
// blocks) per slice.
template <int D>
__device__ __forceinline__ int merge_slices(const DecodeParams& p, int nsp) {
    int n = p.merge_slices;
    while (n > 1 && (n > nsp || (p.out_q && (D / 4) / n < 8))) n >>= 1;
    return n;
}

// Wait of one thread until the arrival counter reaches `target` (unsigned, wrapping). The
// workgroups it waits for were dispatched before the waiting one, so the wait ends; it is
// still bounded (kSpinTicks of the 100 MHz real-time clock) so that a broken dispatch
// assumption cannot hang the GPU. Returns false when it gave up: the caller then records
// the failure in the workspace's sticky error word and does not merge.
constexpr uint64_t kSpinTicks = 100000000;  // 1 s
__device__ __forceinline__ bool wait_count(const unsigned* cnt, unsigned target) {
    const uint64_t t0 = __builtin_amdgcn_s_memrealtime();
    while ((int)(__hip_atomic_load(cnt, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) - target) < 0) {
        if (__builtin_amdgcn_s_memrealtime() - t0 > kSpinTicks) return false;
    }
    return true;
}

// Workgroups per CU the register budget is set for: fp16 two (two waves per SIMD, up to 256
// registers), paged three (up to 168), contiguous int8 one of eight waves (two per SIMD).
// Two kv heads per workgroup (eight waves): one.
constexpr int wgs_per_cu(bool paged, bool q8, int kpw = 1) { return kpw == 2 ? 1 : (paged ? kPagedWgsPerCu : (q8 ? 1 : 2)); }

// KPW: kv heads per workgroup. 1: the grid's x walks (kv head, head block) groups and all W
// waves take interleaved tiles of one kv head's split. 2 (contiguous caches, G <= 16): x
// walks kv-head pairs, waves [0, 4) take kv head 2x and waves [4, 8) kv head 2x + 1 over the
// same positions, so a workgroup reads twice the bytes of each cache row (two adjacent
// kv-head slices); the pair is the merge group.
// WOV > 0 overrides the wave count (contiguous int8, one kv head: 4 waves with NST = 2, a
// second tile in flight while a wave dequantises; one workgroup per CU).
template <int D, bool PAGED, bool Q8, int NST, bool ROPE, int KPW, int WOV = 0>
__global__ __launch_bounds__((WOV ? WOV : waves_for(PAGED, Q8, KPW)) * 64, WOV ? 1 : wgs_per_cu(PAGED, Q8, KPW)) void fa_decode_kernel(DecodeParams p) {
    static_assert(KPW == 1 || (KPW == 2 && !PAGED), "kv-head pairs: contiguous caches");
    static_assert(WOV == 0 || (Q8 && !PAGED && KPW == 1), "wave override: contiguous int8");
    constexpr int W = WOV ? WOV : waves_for(PAGED, Q8, KPW);  // waves of this workgroup
    constexpr int WT = W / KPW;                    // waves per kv head (tile interleave)
    constexpr int NT = W * 64;
    using Gm = Geo<D, Q8, PAGED, W>;
    __shared__ __align__(16) unsigned char smem[Gm::LDS];
    stamp(0);

    // grid x = (kv head, head block) group, y = split: consecutive workgroup ids walk the
    // groups first, so the dispatch order interleaves groups and, with round-robin
    // placement over the 8 XCDs, the splits of one group share an XCD when there are 8 groups
    // Kernel arguments are loaded lazily, and loads used only after the early return below
    // would each cost the prologue a scalar memory round trip: touch every field the
    // prologue and the first tile need here, so they arrive in one batch.
    pin_sgpr(p.q); pin_sgpr(p.k); pin_sgpr(p.v); pin_sgpr(p.d_pos); pin_sgpr(p.seq_len); pin_sgpr(p.max_seq);
    pin_sgpr(p.Hq); pin_sgpr(p.G); pin_sgpr(p.ngb); pin_sgpr(p.kv_dim); pin_sgpr(p.single);
    pin_sgpr(p.min_chunk); pin_sgpr(p.max_splits); pin_sgpr(p.counters); pin_sgpr(p.merge_slices);
    pin_sgpr(p.Hkv); pin_sgpr(p.out_q); pin_sgpr(p.scale2); pin_sgpr(p.nsplit_grid); pin_sgpr(p.local_merge);
    if (!PAGED) { pin_sgpr(p.split_major); pin_sgpr(p.flags); }
    if (Q8) { pin_sgpr(p.k_scale); pin_sgpr(p.v_scale); }
    if (PAGED) { pin_sgpr(p.seq_lens); pin_sgpr(p.block_table); pin_sgpr(p.bt_stride); }
    if (ROPE) { pin_sgpr(p.rope_table); pin_sgpr(p.neox); pin_sgpr(p.k_new); pin_sgpr(p.v_new); }
    // int8 caches: the block scales of one position, for all kv heads, share a cache line, so
    // the workgroups of one split (every kv head group) are placed on one XCD (ids are dealt
    // to the 8 XCDs in turn) to read those lines through one L2; fp16 caches with
    // split_major set are placed the same way, so that one XCD reads whole cache rows at a
    // time. Within a group the splits keep increasing with the id, as the fused merge requires.
    int group = blockIdx.x, split = blockIdx.y;
    if constexpr (!PAGED) {
        if ((Q8 || p.split_major) && (gridDim.y & 7) == 0) {
            const int lin = blockIdx.x + gridDim.x * blockIdx.y;
            const int r = lin >> 3;
            group = r % gridDim.x;
            split = (lin & 7) + 8 * (r / gridDim.x);
        }
    }
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // uniform: branches on it are scalar
    const int half = KPW == 2 ? wave / WT : 0;                  // this wave's kv head of the pair
    const int wt = KPW == 2 ? wave % WT : wave;                 // its place in the head's tile interleave
    const int kvh = (group / p.ngb) * KPW + half, gb = group % p.ngb;
    const int ngroups = p.Hkv / KPW * p.ngb;                    // grid x
    const int b = blockIdx.z;
    // context length: read once (the device position or sequence length), clamped to the cache
    const int S_raw = PAGED ? p.seq_lens[b] : (p.d_pos ? *p.d_pos + 1 : p.seq_len);
    const int S = min(S_raw, p.max_seq);
#if FA_STAMPS
    asm volatile("" ::"s"(S));
    stamp(1);
#endif
    const int chunk = p.single ? (S > 0 ? ((S + kSpan - 1) / kSpan) * kSpan : kSpan)
                               : split_chunk(S, p.min_chunk, p.max_splits);
    const int nsp = p.single ? 1 : split_count(S, p.min_chunk, p.max_splits);
    if (split >= nsp) return;  // inactive split; the merge ignores it
    // fused merge (see the end of the kernel): in the fixed-merger form, this workgroup's
    // merge slice (mk >= 0 for the last nslice splits)
    const bool last_arriver = p.merge_slices == 0;
    const int nslice = (nsp > 1 && p.counters && !last_arriver) ? merge_slices<D>(p, nsp) : 1;
    const int mk = split - (nsp - nslice);
    // (grid x = Hkv * ngb groups)
    unsigned* cnt = reinterpret_cast<unsigned*>(p.counters) + ((size_t)b * ngroups + group) * kCounterStride;
    // The group's counter base is loaded by the workgroups that need it (mergers; every one
    // in the last-arriver and XCD-local forms) right after their first tile loads (in
    // stream, below). Loaded here, before them, its round trip to the memory side came
    // before the first tile: the compiler placed a full wait for it ahead of the first loads
    // (it reused the load's destination register as the unused high half of an address
    // computation). After the stream, the compiler waited for it before the combine.
    const bool needs_base = nsp > 1 && p.counters && (mk >= 0 || last_arriver || p.local_merge);
    unsigned base = 0;
    const int start = split * chunk;
    const int end = min(S, start + chunk);  // positions [start, end)
#if FA_STAMPS
    {
        const unsigned xcc = __builtin_amdgcn_s_getreg((3 << 11) | 20);  // HW_REG_XCC_ID[3:0]
        const unsigned hwid = __builtin_amdgcn_s_getreg((31 << 11) | 4);  // HW_REG_HW_ID
        stamp_val(24, xcc);
        stamp_val(25, hwid);
        stamp_val(26, (unsigned)split | (unsigned)nsp << 12 | (unsigned)(mk + 1) << 24);
        stamp_val(27, (unsigned)((end - start + kTile - 1) / kTile));
    }
#endif

    const int col = lane & 15, kb = lane >> 4;
    const int g = gb * 16 + col;
    const bool gvalid = g < p.G;
    const int head = kvh * p.G + g;

    // Q^T as the B operand of S^T = K Q^T: lane (col = head, kb) holds q[d = s*32 + kb*8 .. +8].
    // Loads are unconditional (lanes past the group read the group's first head and are
    // zeroed later), so no branch drains the load counter.
    h8 qf[Gm::KSTEPS];

    // Step variant: the RoPE table entries of this lane's q fragment, and the new K/V row
    // chunk (plus its rotation partner chunk) of lane chunk `lane % CPR`, all at position
    // S-1. They are issued before the first K/V tile and used after it is in flight. A
    // chunk is the 16 bytes one lane moves per cache row: 8 fp16 values, or 16 int8 ones.
    constexpr int HD2 = D / 2;
    constexpr int TPH = NT / 16;                  // threads per head column in the q rotation
    constexpr int PPT = ROPE ? HD2 / TPH : 1;     // q rotation pairs per thread (16 head columns x D/2 pairs)
    constexpr int CW = Q8 ? 16 : 8;                       // values of one row chunk
    constexpr int NH = ROPE ? CW / 8 : 1;                 // fp16 vectors of one row chunk
    // q rotation. Contiguous caches: every lane rotates its own fragment in registers (no LDS,
    // no barrier). Lane i holds RoPE table entry i of the position (crow, one 8-byte load), and
    // a lane takes the entries of its own pairs from the lanes holding them (ds_bpermute:
    // NeoX pair i = 32 s + 8 kb + j, s < KSTEPS/2, partner in k-step s + KSTEPS/2 of the same
    // lane; interleaved: i = 16 s + 4 kb + j, pair (2j, 2j + 1) of k-step s). Paged (a smaller
    // register budget): the rotation is spread over the workgroup (rq0, rq1, rcs) and read
    // back through LDS.
    constexpr bool QREG = ROPE && !PAGED;
    float2 crow = float2{0.f, 0.f};
    _Float16 rq0[PPT], rq1[PPT];
    float2 rcs[PPT];
    h8 nk[NH], nkp[NH], nv[NH];
    float2 ncs[ROPE ? CW : 1];
    int append_wt = -1, append_tile = -1, append_row = -1;  // per kv head: its wave wt == append_wt
    // q is rotated only when position S-1 is the new token's own position inside the cache,
    // as the separate append does (it skips positions < 0 and >= max_ctx)
    bool rot_q = false;
    const int nchunk = (lane % Gm::CPR) * CW;  // first element of this lane's row chunk
    if constexpr (ROPE) {
        // the wave that loads the tile holding position S-1 (in the split holding it)
        // takes the new row from registers instead of the cache; past max_seq: no append
        rot_q = S > 0 && S_raw == S;
        if (rot_q && split == nsp - 1) {
            const int last_tile = (end - start - 1) / kTile;
            append_wt = last_tile % WT;
            append_tile = last_tile;
            append_row = (S - 1) - (start + last_tile * kTile);
        }
    }
    // The inputs other than the cache (q, the RoPE table entries, the new row). Decode only:
    // issued after the first K/V tiles, so that those, the longest wait, start first. Step:
    // issued before them, because vector loads complete in order: the q rotation waits for
    // these loads only, and runs while the first tiles are in flight.
    auto load_inputs = [&]() __attribute__((always_inline)) {
        const uint16_t* qrow = p.q + ((size_t)b * p.Hq + (gvalid ? head : kvh * p.G)) * D;
#pragma unroll
        for (int s = 0; s < Gm::KSTEPS; ++s) {
            const u4 raw = *reinterpret_cast<const u4*>(qrow + s * 32 + kb * 8);
            qf[s] = *reinterpret_cast<const h8*>(&raw);
        }
        if constexpr (!ROPE) return;
        // The table entries of the q rotation are loaded by every wave whatever rot_q and the
        // pair layout, and prepare() uses them unconditionally: the compiler counts
        // outstanding loads along each path and keeps the smallest count where paths join,
        // and it moves a load whose value is used in one branch only into that branch, behind
        // the first K/V tiles; either made the rotation's waits drain those tiles too.
        const int pos = S > 0 ? S - 1 : 0;
        const float2* cs = reinterpret_cast<const float2*>(p.rope_table) + (size_t)pos * HD2;
        if constexpr (QREG) crow = cs[lane < HD2 ? lane : HD2 - 1];
        if constexpr (!QREG) {  // this thread's share of the q rotation: PPT pairs of head column tid / TPH
            const int hg = gb * 16 + tid / TPH, i0 = (tid % TPH) * PPT;
            const uint16_t* qr = p.q + ((size_t)b * p.Hq + kvh * p.G + (hg < p.G ? hg : 0)) * D;
#pragma unroll
            for (int e = 0; e < PPT; ++e) {
                const int i = i0 + e;  // pair (i, i + D/2) (neox) or (2i, 2i + 1)
                rq0[e] = *reinterpret_cast<const _Float16*>(qr + (p.neox ? i : 2 * i));
                rq1[e] = *reinterpret_cast<const _Float16*>(qr + (p.neox ? i + HD2 : 2 * i + 1));
                rcs[e] = cs[i];
            }
        }
        // only the append wave needs the new row chunk (and its rotation partner) of its
        // lane (its loads may sink behind the first tiles: that only makes this one wave's
        // waits cover its own tiles)
        if (wt == append_wt) {
            const size_t src = (size_t)b * p.kv_dim + (size_t)kvh * D;
            const int partner = nchunk < HD2 ? nchunk + HD2 : nchunk - HD2;
#pragma unroll
            for (int i = 0; i < NH; ++i) {
                nk[i] = *reinterpret_cast<const h8*>(p.k_new + src + nchunk + 8 * i);
                nkp[i] = *reinterpret_cast<const h8*>(p.k_new + src + partner + 8 * i);
                nv[i] = *reinterpret_cast<const h8*>(p.v_new + src + nchunk + 8 * i);
            }
#pragma unroll
            for (int j = 0; j < CW; ++j) ncs[j] = cs[p.neox ? (nchunk % HD2) + j : (nchunk + j) / 2];
        }
    };

    // Rotate this lane's q fragment at position S-1 (neox pairs: k-steps s and
    // s + KSTEPS/2; interleaved pairs: neighbouring elements), then zero lanes past the
    // group. The new K row is rotated the same way and written to the cache by the
    // append wave; that wave substitutes the rotated row in its own tile, so it never
    // re-reads the cache row it wrote.
    // the new row as the append wave substitutes it into its tile: fp16 chunks (rk, nv[0]),
    // or int8 chunks with their block scales (kq, ksc, vq, vsc)
    u4 rk = u4{0, 0, 0, 0}, kq = u4{0, 0, 0, 0}, vq = u4{0, 0, 0, 0};
    float ksc = 0.0f, vsc = 0.0f;
    auto prepare = [&]() __attribute__((always_inline)) {
        // Every value load_inputs fetched is used here whatever rot_q and the wave's role
        // (results are then chosen by selects, and only the stores are conditional): a load
        // whose value is used in one conditional block only is moved into that block by the
        // compiler, behind the first K/V tiles, and its wait then drains those tiles too.
        if constexpr (ROPE) {
            if constexpr (QREG) {
                // in place; each pair keeps its inputs when rot_q is false. The table entries
                // of a k-step's 8 pairs are fetched from their lanes first (16 ds_bpermutes in
                // flight), then the 8 pairs are rotated.
                if (p.neox) {
                    constexpr int KH = Gm::KSTEPS / 2;
#pragma unroll
                    for (int s = 0; s < KH; ++s) {
                        float c[8], sn[8];
#pragma unroll
                        for (int j = 0; j < 8; ++j) {
                            const int i = 32 * s + 8 * kb + j;
                            c[j] = __shfl(crow.x, i, 64);
                            sn[j] = __shfl(crow.y, i, 64);
                        }
                        __builtin_amdgcn_sched_barrier(0);  // keep the 16 fetches together
#pragma unroll
                        for (int j = 0; j < 8; ++j) {
                            _Float16 r0, r1;
                            const _Float16 x0 = qf[s][j], x1 = qf[s + KH][j];
                            rope_rotate((float)x0, (float)x1, c[j], sn[j], r0, r1);
                            qf[s][j] = rot_q ? r0 : x0;
                            qf[s + KH][j] = rot_q ? r1 : x1;
                        }
                    }
                } else {
#pragma unroll
                    for (int s = 0; s < Gm::KSTEPS; s += 2) {
                        float c[8], sn[8];
#pragma unroll
                        for (int t = 0; t < 8; ++t) {
                            const int i = 16 * (s + t / 4) + 4 * kb + (t % 4);
                            c[t] = __shfl(crow.x, i, 64);
                            sn[t] = __shfl(crow.y, i, 64);
                        }
                        __builtin_amdgcn_sched_barrier(0);  // keep the 16 fetches together
#pragma unroll
                        for (int t = 0; t < 8; ++t) {
                            const int ss = s + t / 4, j = t % 4;
                            _Float16 r0, r1;
                            const _Float16 x0 = qf[ss][2 * j], x1 = qf[ss][2 * j + 1];
                            rope_rotate((float)x0, (float)x1, c[t], sn[t], r0, r1);
                            qf[ss][2 * j] = rot_q ? r0 : x0;
                            qf[ss][2 * j + 1] = rot_q ? r1 : x1;
                        }
                    }
                }
            }
            if constexpr (!QREG) {
                // The rotation of the group's q rows is spread over the workgroup (thread t:
                // rotation pairs i0 .. i0 + PPT - 1 of head column t / TPH, from the values
                // load_inputs fetched; unrotated when rot_q is false), and every lane reads
                // its fragment back from LDS.
                _Float16* qx = reinterpret_cast<_Float16*>(smem + Gm::QX_OFF);  // [16 heads][D]
                const int hc = tid / TPH, i0 = (tid % TPH) * PPT;
#pragma unroll
                for (int e = 0; e < PPT; ++e) {
                    _Float16 r0, r1;
                    rope_rotate((float)rq0[e], (float)rq1[e], rcs[e].x, rcs[e].y, r0, r1);
                    r0 = rot_q ? r0 : rq0[e];
                    r1 = rot_q ? r1 : rq1[e];
                    if (p.neox) {
                        qx[hc * D + i0 + e] = r0;
                        qx[hc * D + HD2 + i0 + e] = r1;
                    } else {
                        qx[hc * D + 2 * (i0 + e)] = r0;
                        qx[hc * D + 2 * (i0 + e) + 1] = r1;
                    }
                }
                __syncthreads();
#pragma unroll
                for (int s = 0; s < Gm::KSTEPS; ++s) qf[s] = *reinterpret_cast<const h8*>(qx + col * D + s * 32 + kb * 8);
            }
            if (wt == append_wt) {
            h8 r[NH];
#pragma unroll
            for (int i = 0; i < NH; ++i) {
                const h8 x = nk[i], y = nkp[i];
                if (p.neox) {
                    const bool lo = nchunk < HD2;
#pragma unroll
                    for (int j = 0; j < 8; ++j) {
                        _Float16 r0, r1;
                        const float2 c = ncs[8 * i + j];
                        // pair (i, i + D/2): x0 is the low-half element
                        rope_rotate((float)(lo ? x[j] : y[j]), (float)(lo ? y[j] : x[j]), c.x, c.y, r0, r1);
                        r[i][j] = lo ? r0 : r1;
                    }
                } else {
#pragma unroll
                    for (int j = 0; j < 8; j += 2) {
                        _Float16 r0, r1;
                        const float2 c = ncs[8 * i + j];
                        rope_rotate((float)x[j], (float)x[j + 1], c.x, c.y, r0, r1);
                        r[i][j] = r0;
                        r[i][j + 1] = r1;
                    }
                }
            }
            uint16_t kbits = 0, vbits = 0;
            if constexpr (!Q8) {
                rk = *reinterpret_cast<const u4*>(&r[0]);
            } else {
                // int8 cache: the rotated k (rounded to fp16 as the rope step leaves it) and
                // v are quantized per 32-value block (this lane's 16 values and those of
                // lane ^ 1) exactly as the int8 append does (storeKvQ8Kernel rules)
                quant_chunk16(r, kq, ksc, kbits);
                quant_chunk16(nv, vq, vsc, vbits);
            }
            {
                const size_t dst = row_index<PAGED>(p, b, S - 1) * p.kv_dim + (size_t)kvh * D + nchunk;
                if constexpr (!Q8) {
                    if (lane < Gm::CPR) {
                        *reinterpret_cast<u4*>(const_cast<uint16_t*>(reinterpret_cast<const uint16_t*>(p.k)) + dst) = rk;
                        *reinterpret_cast<h8*>(const_cast<uint16_t*>(reinterpret_cast<const uint16_t*>(p.v)) + dst) = nv[0];
                    }
                } else {
                    if (lane < Gm::CPR) {
                        *reinterpret_cast<u4*>(const_cast<char*>(static_cast<const char*>(p.k)) + dst) = kq;
                        *reinterpret_cast<u4*>(const_cast<char*>(static_cast<const char*>(p.v)) + dst) = vq;
                        if ((lane & 1) == 0) {
                            const_cast<uint16_t*>(p.k_scale)[dst / 32] = kbits;
                            const_cast<uint16_t*>(p.v_scale)[dst / 32] = vbits;
                        }
                    }
                }
            }
            }
        }
        if (!gvalid) {
#pragma unroll
            for (int s = 0; s < Gm::KSTEPS; ++s) qf[s] = h8{0, 0, 0, 0, 0, 0, 0, 0};
        }
    };

    unsigned char* kl = smem + wave * Gm::WAVE_LDS;
    unsigned char* vl = kl + kTile * Gm::LROW;
    const char* kbase = static_cast<const char*>(p.k) + (size_t)kvh * (Q8 ? D : D * 2);
    const char* vbase = static_cast<const char*>(p.v) + (size_t)kvh * (Q8 ? D : D * 2);
    const size_t rowb = (size_t)p.kv_dim * (Q8 ? 1 : 2);

    float m_run = kNegBig, l_run = 0.0f;
    f4 o[Gm::DTILES];
#pragma unroll
    for (int i = 0; i < Gm::DTILES; ++i) o[i] = f4{0.f, 0.f, 0.f, 0.f};

    // NST register stages per wave: while one 16-row tile is consumed, the next
    // NST-1 tiles of this wave are already in flight. Loads are unconditional (rows past
    // the end re-read the last valid row and are zeroed) so the wait counts stay
    // static and never collapse to a full drain.
    const int ntiles = (end - start + kTile - 1) / kTile;
    const int lrow = lane / Gm::CPR, lchunk = lane % Gm::CPR;
    struct Stage {
        u4 k[Gm::NLD], v[Gm::NLD];
        short ks[Gm::NLD], vs[Gm::NLD];  // int8 block scales (fp16 bits)
    };

    // Each tile is read through buffer descriptors that cover exactly its rows inside
    // [start, end), so rows past the end, and whole tiles past the last one (the refill after
    // a wave's last tile), read as zeros without touching memory; the lane's byte offsets are
    // the same for every tile. Paged pools: a tile is one page (splits start at multiples of
    // 128 positions), found through the block table. The pages of this wave's first 64 tiles
    // (tiles wave + 4 i) are loaded once, one per lane, and taken with a lane read per tile.
    static_assert(kTile == kPageTokens, "one page per tile");
    int wpages = 0;
    if constexpr (PAGED) {
        const int pt = start + (wt + WT * lane) * kTile;
        wpages = pt < end ? p.block_table[(size_t)b * p.bt_stride + (pt >> 4)] : 0;
    }
    const uint32_t lane_off = (uint32_t)(lrow * rowb + lchunk * 16);
    const uint32_t srow = (uint32_t)(p.kv_dim / 32) * 2;  // bytes of one position's int8 scales
    const uint32_t lane_soff = (uint32_t)lrow * srow + (uint32_t)(lchunk * 16 / 32) * 2;
    auto load_tile = [&](Stage& st, int t) {
        const int base = start + t * kTile;
        const uint32_t nrows = (uint32_t)min(max(end - base, 0), kTile);
        size_t row0 = (size_t)base;  // cache row of the tile's first position
        if constexpr (PAGED) {
            const int li = (t - wt) / WT;  // this wave's tile number (uniform)
            int phys;
            if (li < 64)
                phys = __builtin_amdgcn_readlane(wpages, li);
            else
                phys = nrows ? __builtin_amdgcn_readfirstlane(p.block_table[(size_t)b * p.bt_stride + (base >> 4)]) : 0;
            row0 = (size_t)phys * kPageTokens;
        }
        // issue order: the int8 scales, then every K row, then every V row (the same order as
        // the prefill's stage copies, where it measured fastest)
        if constexpr (Q8) {
            static_assert(!PAGED, "int8 pages are not supported");
            const size_t sb = (size_t)base * (p.kv_dim / 32) + (size_t)kvh * (D / 32);
            const __amdgpu_buffer_rsrc_t rks = uniform_rsrc(p.k_scale + sb, nrows * srow);
            const __amdgpu_buffer_rsrc_t rvs = uniform_rsrc(p.v_scale + sb, nrows * srow);
#pragma unroll
            for (int r = 0; r < Gm::NLD; ++r) {
                st.ks[r] = ld_buf_f16(rks, lane_soff + (uint32_t)(r * Gm::RPI) * srow);
                st.vs[r] = ld_buf_f16(rvs, lane_soff + (uint32_t)(r * Gm::RPI) * srow);
            }
        }
        const __amdgpu_buffer_rsrc_t rk = uniform_rsrc(kbase + row0 * rowb, nrows * (uint32_t)rowb);
        const __amdgpu_buffer_rsrc_t rv = uniform_rsrc(vbase + row0 * rowb, nrows * (uint32_t)rowb);
#pragma unroll
        for (int r = 0; r < Gm::NLD; ++r) st.k[r] = ld_buf_nt(rk, lane_off + (uint32_t)(r * Gm::RPI) * (uint32_t)rowb);
#pragma unroll
        for (int r = 0; r < Gm::NLD; ++r) st.v[r] = ld_buf_nt(rv, lane_off + (uint32_t)(r * Gm::RPI) * (uint32_t)rowb);
    };

    // phase (fp16): 0 = the whole tile; 1 = only its way into LDS and the refill of its
    // stage; 2 = only the attention over it (after phase 1 and the q rotation)
    auto consume = [&](Stage& st, int t, int t_next, auto phase_tag) {
        constexpr int PH = decltype(phase_tag)::value;
        const int tbase = start + t * kTile;
        if constexpr (Q8) {
            // int8 rows: dequantise the stage's codes into the wave's LDS tile, then refill the
            // stage. (Refilling first needs a register copy of every code and scale, about 30
            // moves per tile, and measured 1.5 % slower at 32k.)
            u4 ck[Gm::NLD], cv[Gm::NLD];
            _Float16 sk[Gm::NLD], sv[Gm::NLD];
#pragma unroll
            for (int r = 0; r < Gm::NLD; ++r) {
                const int row = r * Gm::RPI + lrow;
                ck[r] = st.k[r];  // zeros past the end
                cv[r] = st.v[r];
                sk[r] = __builtin_bit_cast(_Float16, st.ks[r]);
                sv[r] = __builtin_bit_cast(_Float16, st.vs[r]);
                // the new row, as quantized and written to the cache by this wave (selects on
                // the raw codes: cheaper here than rewriting the dequantised row afterwards)
                if (ROPE && t == append_tile && wt == append_wt && row == append_row) {
                    ck[r] = kq;
                    cv[r] = vq;
                    sk[r] = (_Float16)ksc;  // fp16 values: exact
                    sv[r] = (_Float16)vsc;
                }
            }
#pragma unroll
            for (int r = 0; r < Gm::NLD; ++r) {
                const int row = r * Gm::RPI + lrow;
                u4 lo, hi;
                dequant16(ck[r], sk[r], lo, hi);
                *reinterpret_cast<u4*>(kl + row * Gm::LROW + Gm::slot(2 * lchunk) * 16) = lo;
                *reinterpret_cast<u4*>(kl + row * Gm::LROW + Gm::slot(2 * lchunk + 1) * 16) = hi;
                dequant16(cv[r], sv[r], lo, hi);
                *reinterpret_cast<u4*>(vl + row * Gm::LROW + Gm::slot(2 * lchunk) * 16) = lo;
                *reinterpret_cast<u4*>(vl + row * Gm::LROW + Gm::slot(2 * lchunk + 1) * 16) = hi;
            }
            load_tile(st, t_next);
            // LDS operations of one wave complete in order: the reads below see these writes.
            __builtin_amdgcn_wave_barrier();
            if (wave == 0 && t < ntiles && t < 16 * WT) stamp(8 + t / WT);
        } else {
            if constexpr (PH != 2) {
                // registers -> wave-private LDS tile (rows past the end are zeros)
#pragma unroll
                for (int r = 0; r < Gm::NLD; ++r) {
                    const int row = r * Gm::RPI + lrow;
                    *reinterpret_cast<u4*>(kl + row * Gm::LROW + lchunk * 16) = st.k[r];
                    *reinterpret_cast<u4*>(vl + row * Gm::LROW + lchunk * 16) = st.v[r];
                }
            }
            if constexpr (PH != 1) {
                // the new row, as written to the cache by this wave, over the one loaded (a
                // wave's LDS writes complete in order); one tile of one wave
                if (ROPE && t == append_tile && wt == append_wt) {
                    if (lrow == append_row % Gm::RPI) {
                        *reinterpret_cast<u4*>(kl + append_row * Gm::LROW + lchunk * 16) = rk;
                        *reinterpret_cast<u4*>(vl + append_row * Gm::LROW + lchunk * 16) = *reinterpret_cast<const u4*>(&nv[0]);
                    }
                }
            }
            // LDS operations of one wave complete in order: the reads below see these writes.
            __builtin_amdgcn_wave_barrier();
            if constexpr (PH != 2) if (wave == 0 && t < ntiles && t < 16 * WT) stamp(8 + t / WT);
            // Refill this stage while computing. Unconditional, so no branch hides loads from
            // the wait counter (a tile past the end reads nothing and gives zeros).
            if constexpr (PH != 2) load_tile(st, t_next);
            if constexpr (PH == 1) return;
        }
        if (t >= ntiles) return;  // uniform: this stage held no tile

        // S^T[16 positions x 16 heads] = K Q^T
        f4 sacc = f4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int s = 0; s < Gm::KSTEPS; ++s) {
            const h8 a = *reinterpret_cast<const h8*>(kl + col * Gm::LROW + Gm::slot(4 * s + kb) * 16);
            sacc = mfma16x16x32(a, qf[s], sacc);
        }

        // online softmax (log2 domain); lane column = query head, rows kb*4 + i = positions
        float sc[4];
        float mx = kNegBig;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            float x = sacc[i] * p.scale2;
            if (__builtin_isnan(x)) x = kNegBig;
            sc[i] = tbase + kb * 4 + i < end ? x : -__builtin_inff();
            mx = fmaxf(mx, sc[i]);
        }
        mx = col_max4(mx);  // over the 4 lane blocks: the 16 positions of the tile
        // Lazy reference max: the accumulators move to a new reference (and are rescaled) only
        // when some head's tile max exceeds its reference by more than 2^8 (a wave-uniform
        // branch, rarely taken after the first tile); weights stay <= 256 in between.
        if (__builtin_amdgcn_ballot_w64(mx > m_run + kLazy2) != 0) {
            const float m_new = fmaxf(m_run, mx);
            const float da = m_run - m_new;
            const float alpha = da < kCut2 ? 0.0f : exp2_fast(da);
            l_run *= alpha;
#pragma unroll
            for (int dt = 0; dt < Gm::DTILES; ++dt) o[dt] *= alpha;
            m_run = m_new;
        }
        h4 pf;
        float psum = 0.0f;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const float df = sc[i] - m_run;  // -inf for masked rows
            const _Float16 eh = (_Float16)(df < kCut2 ? 0.0f : exp2_fast(df));
            pf[i] = eh;
            psum += (float)eh;
        }
        l_run += psum;

        // O^T += V^T P^T over the 16 positions (k = kb*4 + i); V^T by one transposing LDS read
#pragma unroll
        for (int dt = 0; dt < Gm::DTILES; ++dt) {
            const h4 va = lds_read_tr16(vl + (kb * 4 + (col >> 2)) * Gm::LROW + Gm::slot(2 * dt + ((col & 3) >> 1)) * 16 +
                                        (col & 1) * 8);
            o[dt] = mfma16x16x16(va, pf, o[dt]);
        }
        __builtin_amdgcn_wave_barrier();
    };

    // uniform trip count: groups of N tiles of this wave (tiles wave, wave + W, ...).
    // Long splits keep one tile in flight per wave (more congests HBM); short ones, whose
    // waves have at most four tiles, issue them all at once (one memory latency).
    const int my_tiles = ntiles > wt ? (ntiles - wt + WT - 1) / WT : 0;
    auto stream = [&](auto n_tag) {
        constexpr int N = decltype(n_tag)::value;
        Stage st[N];
        const int groups = (my_tiles + N - 1) / N;
        if (ROPE) load_inputs();
        // unconditional, like the loads above (a wave without tiles reads nothing: its
        // tiles lie past the split's end)
#pragma unroll
        for (int s = 0; s < N; ++s) load_tile(st[s], wt + s * WT);
        if (!ROPE) load_inputs();
        {
            // the newest load, so that no wait for the others covers it. Agent-coherent (sc1)
            // like the relaxed agent-scope atomic load it replaces; size 0 (a zero, no
            // access) for the workgroups that do not merge
            const __amdgpu_buffer_rsrc_t rb = coherent_rsrc(cnt + kCounterStride / 2, needs_base ? 4u : 0u);
            base = (unsigned)__builtin_amdgcn_raw_buffer_load_b32(rb, 0, 0, kCpolSc1);
        }
        using Whole = std::integral_constant<int, 0>;
        if constexpr (ROPE && !Q8 && N > 1 && !QREG) {
            // Paged short splits (all of a wave's tiles in flight at once): the first tile goes
            // into LDS, and its stage's refill is issued, before the q rotation (whose barrier
            // it would otherwise wait behind); its QK then waits for the rotated q. (With one
            // tile in flight per wave, measured 0.2 us slower at 32k: not used.) Contiguous
            // caches rotate in registers first, while the first tiles are in flight.
            if (groups > 0) consume(st[0], wt, wt + N * WT, std::integral_constant<int, 1>{});
            prepare();
            stamp(2);
            if (groups > 0) {
                consume(st[0], wt, wt + N * WT, std::integral_constant<int, 2>{});
#pragma unroll
                for (int s = 1; s < N; ++s) consume(st[s], wt + s * WT, wt + (N + s) * WT, Whole{});
            }
            for (int gi = 1; gi < groups; ++gi) {
#pragma unroll
                for (int s = 0; s < N; ++s) {
                    const int ts = wt + (gi * N + s) * WT;
                    consume(st[s], ts, ts + N * WT, Whole{});
                }
            }
        } else {
            prepare();
            stamp(2);
            for (int gi = 0; gi < groups; ++gi) {
#pragma unroll
                for (int s = 0; s < N; ++s) {
                    const int ts = wt + (gi * N + s) * WT;
                    consume(st[s], ts, ts + N * WT, Whole{});
                }
            }
        }
    };
    constexpr int kShort = PAGED ? kShortStagesPaged : kShortStages;
    if ((ntiles + WT - 1) / WT <= kShort)
        stream(std::integral_constant<int, kShort>{});
    else
        stream(std::integral_constant<int, NST>{});

    stamp(3);
    // ---- combine the W waves of the workgroup through LDS ----
    // (with a region of its own, each wave writes its state without waiting for the others;
    // over the tiles, every wave must be done reading its tiles first)
    l_run = col_sum4(l_run);
    if constexpr (Gm::COMB_OFF == 0) __syncthreads();
    float* cm = reinterpret_cast<float*>(smem + Gm::COMB_OFF);  // [W][16]
    float* cl = cm + W * 16;                          // [W][16]
    float* co = cl + W * 16;                          // [W][16][CROW]
    if (kb == 0) {
        cm[wave * 16 + col] = m_run;
        cl[wave * 16 + col] = l_run;
    }
#pragma unroll
    for (int dt = 0; dt < Gm::DTILES; ++dt)
        *reinterpret_cast<f4*>(co + (wave * 16 + col) * Gm::CROW + dt * 16 + kb * 4) = o[dt];
    __syncthreads();

    // one thread per (head, 4 consecutive output columns)
    const int gcount = min(16, p.G - gb * 16);
    const __amdgpu_buffer_rsrc_t rpo = coherent_rsrc(p.part_o, 0x7fffffff);
    const __amdgpu_buffer_rsrc_t rpml = coherent_rsrc(p.part_ml, 0x7fffffff);
    // (KPW = 2: the first half of the index range is kv head 2x with waves [0, WT), the
    // second kv head 2x + 1 with waves [WT, 2 WT))
    for (int idx = tid; idx < KPW * gcount * (D / 4); idx += NT) {
        const int hf = KPW == 2 ? idx / (gcount * (D / 4)) : 0;
        const int rem = idx - hf * gcount * (D / 4);
        const int gg = rem / (D / 4), d4 = rem % (D / 4);
        const float* hm = cm + hf * WT * 16;
        const float* hl = cl + hf * WT * 16;
        const float* ho = co + hf * WT * 16 * Gm::CROW;
        float M = hm[gg];
#pragma unroll
        for (int w = 1; w < WT; ++w) M = fmaxf(M, hm[w * 16 + gg]);
        float L = 0.0f;
        f4 O = f4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int w = 0; w < WT; ++w) {
            const float df = hm[w * 16 + gg] - M;
            const float wgt = df < kCut2 ? 0.0f : exp2_fast(df);
            L += wgt * hl[w * 16 + gg];
            O += wgt * *reinterpret_cast<const f4*>(ho + (w * 16 + gg) * Gm::CROW + 4 * d4);
        }
        const int hh = ((group / p.ngb) * KPW + hf) * p.G + gb * 16 + gg;
        const size_t row = (size_t)b * p.Hq + hh;
        if (nsp == 1) {
            h4 r;
#pragma unroll
            for (int i = 0; i < 4; ++i) r[i] = out_half(L > 1e-12f ? O[i] / L : 0.0f);
            store_out4(p, row, D, d4, r);
        } else {
            // written through to the device coherence point (sc1) for the merging workgroup,
            // or (XCD-local merge) into this XCD's L2, where the mergers of the group read them
            const size_t slot = row * p.nsplit_grid + split;
            if (!PAGED && !Q8 && p.local_merge) {
                st_pol4<0>(rpo, (uint32_t)((slot * D + 4 * d4) * 4), O);
                if (d4 == 0) st_pol2<0>(rpml, (uint32_t)(slot * 8), float2{M, L});
            } else {
                st_coherent4(rpo, (uint32_t)((slot * D + 4 * d4) * 4), O);
                if (d4 == 0) st_coherent2(rpml, (uint32_t)(slot * 8), float2{M, L});
            }
        }
    }

    stamp(4);
    // the merge group's head rows: one kv head's head block, or (KPW = 2) both heads of the pair
    const size_t mrow0 = (size_t)b * p.Hq + (size_t)(group / p.ngb) * KPW * p.G + gb * 16;
    const int mrows = KPW == 2 ? 2 * p.G : gcount;
    // rotated q back into the q buffer once no other workgroup of the group reads it
    auto write_q = [&]() {
        if (ROPE && gvalid) {
            uint16_t* qrow = const_cast<uint16_t*>(p.q) + ((size_t)b * p.Hq + head) * D;
#pragma unroll
            for (int s = 0; s < Gm::KSTEPS; ++s) *reinterpret_cast<h8*>(qrow + s * 32 + kb * 8) = qf[s];
        }
    };
    if (nsp == 1) write_q();

    // Fused merge. Every workgroup of this (sequence, kv head, head block) adds 1 to the
    // group's arrival counter once its partials are stored. The counter is never reset: a
    // launch is complete when it has grown by nsp over the group's base, which the
    // workgroup that merges (merger 0) then advances by nsp for the next launch.
    // Fixed-merger form (grids that fit on the device at once): nobody waits for the
    // atomic. The mergers are the last nslice splits of the group, i.e. the workgroups
    // dispatched last (workgroups are dispatched in increasing id order): each waits until
    // the counter is complete, which only needs workgroups dispatched before it, then
    // merges its column slice. Merger 0 also writes the rotated q back.
    // Last-arriver form (larger grids, where a waiting merger would hold a slot that
    // later workgroups need): the atomic returns the count before this arrival, and the
    // workgroup that completes the count merges every column.
    if (nsp > 1 && p.counters) {
        // The partials were written through to the device coherence point (sc1 stores);
        // wait until every one of them has completed before this workgroup is counted.
        wait_vmem();
        __syncthreads();
        stamp(5);
        if (!PAGED && !Q8 && p.local_merge) {
            // XCD-local form (every workgroup of the group runs on one XCD; the launcher sets it
            // only for fixed mergers and grids whose groups map to one XCD each): the partials
            // are in this XCD's L2 (completed, above); the split's flag word, also a plain
            // store, then says so with the launch's tag (the group's target count, base + nsp,
            // a value no earlier launch on this workspace left there). The mergers poll the
            // flags with loads that miss the CU's L1 (sc0) and read the partials the same way:
            // no atomic, and no round trip beyond the XCD's L2.
            const unsigned target = base + (unsigned)nsp;
            const size_t frow = ((size_t)b * ngroups + group) * p.nsplit_grid;
            const __amdgpu_buffer_rsrc_t rfl = coherent_rsrc(p.flags + frow, (uint32_t)p.nsplit_grid * 4u);
            if (tid == 0) st_pol1<0>(rfl, (uint32_t)split * 4u, target);
            if (mk < 0) return;
            __shared__ int gave_up_local;
            if (wave == 0) {
                // bounded like wait_count; a merger that gives up sets the sticky error bit
                const uint64_t t0 = __builtin_amdgcn_s_memrealtime();
                bool done = false;
                while (true) {
                    // drop this CU's L1 copies first, so the flags (and, after the last round,
                    // the partials) are read from the XCD's L2, whatever the load policy's L1
                    // behaviour; a vector-cache invalidate, completed before the loads
                    asm volatile("buffer_inv sc0\n\ts_waitcnt vmcnt(0)" ::: "memory");
                    bool ready = true;
                    for (int j = lane; j < nsp; j += 64) ready = ready && ld_pol1<kCpolSc0>(rfl, (uint32_t)j * 4u) == target;
                    if (__builtin_amdgcn_ballot_w64(!ready) == 0) {
                        done = true;
                        break;
                    }
                    if (__builtin_amdgcn_s_memrealtime() - t0 > kSpinTicks) break;
                }
                if (lane == 0) {
                    gave_up_local = !done;
                    if (!done)
                        __hip_atomic_fetch_or(reinterpret_cast<unsigned*>(p.counters) + kStatusWord, kStatusMergeTimeout,
                                              __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                }
            }
            __syncthreads();
            stamp(6);
            if (gave_up_local) return;
            merge_slice<D, NT, true>(p, mrow0, mrows, nsp, mk, nslice);
#if FA_STAMPS
            wait_vmem();
            stamp(7);
#endif
            if (mk == 0) {
                write_q();  // every workgroup of the group has read q by now
                // counter and base advance together, so the other forms find them equal
                if (tid == 0) {
                    __hip_atomic_fetch_add(cnt, (unsigned)nsp, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                    __hip_atomic_store(cnt + kCounterStride / 2, target, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                }
            }
            return;
        }
        if (last_arriver) {
            __shared__ int is_last;
            if (tid == 0)
                is_last = __hip_atomic_fetch_add(cnt, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) - base ==
                          (unsigned)nsp - 1u;
            __syncthreads();
            stamp(6);
            if (!is_last) return;
            merge_any<D, NT>(p, mrow0, mrows, nsp);
#if FA_STAMPS
            wait_vmem();
            stamp(7);
#endif
            write_q();  // every workgroup of the group has read q by now
            if (tid == 0) __hip_atomic_store(cnt + kCounterStride / 2, base + (unsigned)nsp, __ATOMIC_RELAXED,
                                             __HIP_MEMORY_SCOPE_AGENT);
            return;
        }
        if (tid == 0) __hip_atomic_fetch_add(cnt, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        if (mk < 0) return;
        // a merger that gives up waiting sets the workspace's sticky error bit (a vector
        // atomic) and merges nothing: neither the output, nor q, nor the base is written
        __shared__ int gave_up;
        if (tid == 0) {
            gave_up = !wait_count(cnt, base + (unsigned)nsp);
            if (gave_up)
                __hip_atomic_fetch_or(reinterpret_cast<unsigned*>(p.counters) + kStatusWord, kStatusMergeTimeout,
                                      __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
        __syncthreads();
        stamp(6);
        if (gave_up) return;
        merge_slice<D, NT>(p, mrow0, mrows, nsp, mk, nslice);
#if FA_STAMPS
        wait_vmem();
        stamp(7);
#endif
        if (mk == 0) {
            write_q();  // every workgroup of the group has read q by now
            if (tid == 0) __hip_atomic_store(cnt + kCounterStride / 2, base + (unsigned)nsp, __ATOMIC_RELAXED,
                                             __HIP_MEMORY_SCOPE_AGENT);
        }
    }
}

// Second pass of the two-kernel path: one workgroup per (sequence, head).
template <int D, bool PAGED>
__global__ __launch_bounds__(kThreads) void fa_merge_kernel(DecodeParams p) {
    const int row = blockIdx.x;  // b * Hq + head
    const int S = context_len(p, row / p.Hq, PAGED);
    const int nsp = split_count(S, p.min_chunk, p.max_splits);
    if (p.single || nsp <= 1) return;  // the decode kernel wrote the output
    merge_any<D, kThreads>(p, (size_t)row, 1, nsp);
}

template <int D, bool PAGED, bool Q8, int KPW, int WOV = 0, int NSTQ = kStagesQ8>
int launch_k(const DecodeParams& p_in, int batch, hipStream_t stream) {
    DecodeParams p = p_in;
    p.split_major = split_major_default();
    const dim3 grid(p.Hkv / KPW * p.ngb, p.single ? 1 : p.nsplit_grid, batch);
    const dim3 block((WOV ? WOV : waves_for(PAGED, Q8, KPW)) * 64);
    // fixed mergers while the whole grid can be resident at once, else the last arriver merges
    const size_t resident = (size_t)device_cus() * (WOV ? 1 : wgs_per_cu(PAGED, Q8, KPW));
    p.merge_slices = (size_t)grid.x * grid.y * grid.z <= resident ? kMergeSlices : 0;
    // XCD-local merge: fixed mergers, contiguous fp16 caches, groups placed one XCD each
    // (workgroup ids are dealt to the 8 XCDs in turn, and a group's ids are congruent modulo
    // the group count, a multiple of 8), and the caller's switch (FRIDAY_ATTN_LOCAL_MERGE)
    p.local_merge = (!PAGED && !Q8 && !p.single && p.counters && p.flags && p.merge_slices > 0 && !p.split_major &&
                     grid.x % 8 == 0 && grid.z == 1 && local_merge_default() && local_placement_ok(stream))
                        ? 1
                        : 0;
    if (p.rope_table) {
        if (!p.counters || (PAGED && Q8)) return -2;  // the step needs the fused merge; no int8 pages
        hipLaunchKernelGGL((fa_decode_kernel<D, PAGED, Q8, Q8 ? NSTQ : kStages, true, KPW, WOV>), grid, block, 0,
                           stream, p);
        return hipGetLastError() == hipSuccess ? 0 : -1;
    }
    hipLaunchKernelGGL((fa_decode_kernel<D, PAGED, Q8, Q8 ? NSTQ : kStages, false, KPW, WOV>), grid, block, 0, stream,
                       p);
    if (hipGetLastError() != hipSuccess) return -1;
    if (!p.single && !p.counters) {
        hipLaunchKernelGGL((fa_merge_kernel<D, PAGED>), dim3(batch * p.Hq), dim3(kThreads), 0, stream, p);
        if (hipGetLastError() != hipSuccess) return -1;
    }
    return 0;
}

// kv heads per workgroup: the host's choice (DecodeParams::kpw, which also set the split
// bound); pairs only for contiguous caches with one head block per kv head
template <int D, bool PAGED, bool Q8>
int launch_t(const DecodeParams& p, int batch, hipStream_t stream) {
    if constexpr (!PAGED) {
        if (p.kpw == 2) {
            if (p.ngb != 1 || p.Hkv % 2) return -2;
            return launch_k<D, PAGED, Q8, 2>(p, batch, stream);
        }
        // contiguous int8, one kv head per workgroup: 4 waves, two tiles in flight each
        // (FRIDAY_ATTN_Q8_DEEP = 1; the default is 8 waves with one)
        if constexpr (Q8) if (q8_deep_default()) return launch_k<D, PAGED, Q8, 1, 4, 2>(p, batch, stream);
    }
    return launch_k<D, PAGED, Q8, 1>(p, batch, stream);
}

__global__ void fa_zero_kernel(uint32_t* p, size_t n) {
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x) p[i] = 0;
}

// Placement check of the XCD-local merge: every workgroup of a (groups x splits) grid
// records the XCD it runs on (HW_REG_XCC_ID) in a file-scope array (no allocation).
constexpr int kProbeX = 64, kProbeY = 32;
__device__ unsigned g_xcc_probe[kProbeX * kProbeY];
__global__ void fa_xcc_probe_kernel(unsigned* xcc) {
    if (threadIdx.x == 0) xcc[blockIdx.x + gridDim.x * blockIdx.y] = __builtin_amdgcn_s_getreg((3 << 11) | 20);
}

}  // namespace

// Whether the workgroups of each group (grid x, a multiple of 8 columns) of a decode-shaped
// grid run on one XCD on the current device: probed once per device (a 64 x 32 grid, 16
// launches on the caller's stream, which is synchronised) and remembered. Not probed while
// `stream` is capturing: the caller then uses the counter form.
bool local_placement_ok(hipStream_t stream) {
    static std::mutex mu;
    static int state[64] = {};  // 0 unknown, 1 ok, -1 not
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return false;
    std::lock_guard<std::mutex> lock(mu);
    if (state[dev]) return state[dev] > 0;
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    if (hipStreamIsCapturing(stream, &cs) != hipSuccess || cs != hipStreamCaptureStatusNone) return false;
    void* d = nullptr;
    bool ok = hipGetSymbolAddress(&d, HIP_SYMBOL(g_xcc_probe)) == hipSuccess;
    std::vector<unsigned> h(kProbeX * kProbeY);
    for (int r = 0; ok && r < 16; ++r) {
        hipLaunchKernelGGL(fa_xcc_probe_kernel, dim3(kProbeX, kProbeY), dim3(64), 0, stream, static_cast<unsigned*>(d));
        ok = hipGetLastError() == hipSuccess &&
             hipMemcpyAsync(h.data(), d, sizeof(unsigned) * h.size(), hipMemcpyDeviceToHost, stream) == hipSuccess &&
             hipStreamSynchronize(stream) == hipSuccess;
        // workgroup ids are x + 64 y: every column x on one XCD for all y
        for (int x = 0; ok && x < kProbeX; ++x)
            for (int y = 1; ok && y < kProbeY; ++y) ok = h[x + kProbeX * y] == h[x];
    }
    state[dev] = ok ? 1 : -1;
    return ok;
}

int launch_zero_fill(void* ptr, size_t bytes, hipStream_t stream) {
    const size_t n = bytes / 4;
    const int blocks = (int)std::min<size_t>((n + 255) / 256, 4096);
    hipLaunchKernelGGL(fa_zero_kernel, dim3(blocks > 0 ? blocks : 1), dim3(256), 0, stream, static_cast<uint32_t*>(ptr), n);
    return hipGetLastError() == hipSuccess ? 0 : -1;
}

int launch_decode(const DecodeParams& p, int head_dim, int batch, bool paged, bool q8, hipStream_t stream) {
    if (head_dim == 128) {
        if (paged) return q8 ? -2 : launch_t<128, true, false>(p, batch, stream);
        return q8 ? launch_t<128, false, true>(p, batch, stream) : launch_t<128, false, false>(p, batch, stream);
    }
    if (head_dim == 64) {
        if (paged) return q8 ? -2 : launch_t<64, true, false>(p, batch, stream);
        return q8 ? launch_t<64, false, true>(p, batch, stream) : launch_t<64, false, false>(p, batch, stream);
    }
    return -2;
}

}  // namespace fa

#if FA_STAMPS
// Stamps build only: point the decode kernels' phase timestamps at `buf` (device memory of
// 32 64-bit words per workgroup of the launches that follow; null switches them off).
extern "C" int friday_attn_debug_stamps(void* buf) {
    return hipMemcpyToSymbol(HIP_SYMBOL(fa::g_stamps), &buf, sizeof(buf)) == hipSuccess ? 0 : -1;
}
#endif
