// Causal chunked-prefill attention on gfx950 MFMA.
//
// Semantics: launchPrefillAttention (attention_kernels.h:36-50, .cu:513-684):
// query t of the chunk sits at position p0 + t (p0 = *d_pos0) and attends to
// cache positions [0, p0 + t]; NaN score -> -1e30, exp cut off below -50 from
// the running max, fp32 accumulation, output NaN -> 0, clamp, RNE fp16. Row t
// equals decode attention with S = p0 + t + 1 up to the order of fp32 additions.
//
// Work decomposition: rows r = t * G + g of one kv head (all query heads of the GQA group
// for every token share its K/V).
// fa_prefill_dma_kernel (every fp16 / bf16 call, and int8 calls with 4-byte aligned scale
// arrays): a workgroup of eight waves owns up to six 16-row tiles in two groups of four
// waves; stages of 128 keys are copied global -> LDS by global_load_lds_dwordx4 (two
// stage buffers, the next stage in flight during this one's MFMAs), each wave of a group
// takes 32 keys of the stage for all of its group's row tiles, and the four key slices'
// softmax states merge through LDS at the end. int8 stages are copied raw and decoded to
// fp16 in LDS by the whole workgroup before the MFMAs.
// fa_prefill_kernel (int8 scale arrays off 4-byte alignment): 128 rows (4 waves x 32),
// K/V staged through registers in 32-position tiles:
//   K tile row-major            -> A operand of S^T = K Q^T   (ds_read_b128)
//   V tile transposed, with the positions of one lane block stored together
//                               -> A operand of O^T += V^T P^T (ds_read_b128)
// Both keep Q^T, O^T and the softmax state in registers.
#include "fa_common.hpp"
#include "fa_internal.hpp"

#include <climits>
#include <cstdlib>
#include <type_traits>

namespace fa {
namespace {

constexpr int kPfWaves = 4;
constexpr int kPfThreads = kPfWaves * 64;
constexpr int kPfRT = 2;                        // 16-row tiles per wave
constexpr int kPfRowsWave = 16 * kPfRT;
constexpr int kPfRowsWG = kPfRowsWave * kPfWaves;  // 128
constexpr int kPfTile = 32;                     // key positions per tile

template <int D, bool Q8>
struct PfGeo {
    static constexpr int KROW = D * 2 + 16;              // K tile row stride (bytes)
    static constexpr int VTROW = kPfTile * 2 + 16;       // V^T row stride (bytes), one row per d
    static constexpr int K_LDS = kPfTile * KROW;
    static constexpr int V_LDS = D * VTROW;
    static constexpr int KSTEPS = D / 32;
    static constexpr int DTILES = D / 16;
    static constexpr int ROWB = Q8 ? D : 2 * D;          // cache bytes per kv-head row
    static constexpr int CPR = ROWB / 16;                // 16 B chunks per row
    static constexpr int RPR = kPfThreads / CPR;         // rows per round
    static constexpr int ROUNDS = (kPfTile + RPR - 1) / RPR;
};

// V^T column of tile position p: the 8 positions that lane block kb feeds to one
// MFMA (p = kb*4+j and 16+kb*4+j, j < 4) are stored contiguously.
__device__ __forceinline__ int vt_col(int p) { return ((p & 15) >> 2) * 8 + (p >> 4) * 4 + (p & 3); }

template <int D, bool Q8>
__global__ __launch_bounds__(kPfThreads) void fa_prefill_kernel(PrefillParams p) {
    using Gm = PfGeo<D, Q8>;
    __shared__ __align__(16) unsigned char s_k[Gm::K_LDS];
    __shared__ __align__(16) unsigned char s_vt[Gm::V_LDS];

    const int R = p.T * p.G;
    const int rtile = gridDim.x - 1 - blockIdx.x;  // heavier (later) rows first
    const int kvh = blockIdx.y;
    const int row0 = rtile * kPfRowsWG;
    const int p0 = *p.d_pos0;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int col = lane & 15, kb = lane >> 4;
    const int qd = p.Hq * D;
    const int kv_dim = p.Hkv * D;

    // rows of this lane (one per 16-row tile) and their causal limits
    int lim[kPfRT];
    h8 qf[kPfRT][Gm::KSTEPS];
#pragma unroll
    for (int rt = 0; rt < kPfRT; ++rt) {
        const int r = row0 + wave * kPfRowsWave + rt * 16 + col;
        const bool valid = r < R;
        const int t = valid ? r / p.G : 0, g = valid ? r % p.G : 0;
        lim[rt] = valid ? p0 + t : -1;
        const uint16_t* qrow = p.q + (size_t)t * qd + (size_t)(kvh * p.G + g) * D;
#pragma unroll
        for (int s = 0; s < Gm::KSTEPS; ++s) {
            u4 raw = valid ? *reinterpret_cast<const u4*>(qrow + s * 32 + kb * 8) : u4{0, 0, 0, 0};
            qf[rt][s] = *reinterpret_cast<h8*>(&raw);
        }
    }
    const int wg_last = min(row0 + kPfRowsWG, R) - 1;
    const int wv_last = min(row0 + wave * kPfRowsWave + kPfRowsWave, R) - 1;
    const int kend = p0 + wg_last / p.G + 1;                              // keys [0, kend) for the workgroup
    const int wend = wv_last >= row0 + wave * kPfRowsWave ? p0 + wv_last / p.G + 1 : 0;  // for this wave
    const int ntiles = (kend + kPfTile - 1) / kPfTile;

    float m_run[kPfRT], l_run[kPfRT];
    f4 o[kPfRT][Gm::DTILES];
#pragma unroll
    for (int rt = 0; rt < kPfRT; ++rt) {
        m_run[rt] = kNegBig;
        l_run[rt] = 0.0f;
#pragma unroll
        for (int i = 0; i < Gm::DTILES; ++i) o[rt][i] = f4{0.f, 0.f, 0.f, 0.f};
    }

    const char* kbase = static_cast<const char*>(p.k) + (size_t)kvh * Gm::ROWB;
    const char* vbase = static_cast<const char*>(p.v) + (size_t)kvh * Gm::ROWB;
    const size_t rowb = (size_t)kv_dim * (Q8 ? 1 : 2);
    const int lrow = tid / Gm::CPR, lchunk = tid % Gm::CPR;
    u4 kr[Gm::ROUNDS], vr[Gm::ROUNDS];
    float ksc[Gm::ROUNDS], vsc[Gm::ROUNDS];

    auto load_tile = [&](int kt) {
#pragma unroll
        for (int r = 0; r < Gm::ROUNDS; ++r) {
            const int pr = r * Gm::RPR + lrow;
            const int pos = kt * kPfTile + pr;
            if (pr < kPfTile && pos < kend) {
                kr[r] = *(reinterpret_cast<const u4*>(kbase + (size_t)pos * rowb) + lchunk);
                vr[r] = *(reinterpret_cast<const u4*>(vbase + (size_t)pos * rowb) + lchunk);
                if (Q8) {
                    const size_t si = ((size_t)pos * kv_dim + (size_t)kvh * D + lchunk * 16) / 32;
                    ksc[r] = (float)*reinterpret_cast<const _Float16*>(p.k_scale + si);
                    vsc[r] = (float)*reinterpret_cast<const _Float16*>(p.v_scale + si);
                }
            } else {
                kr[r] = u4{0, 0, 0, 0};
                vr[r] = u4{0, 0, 0, 0};
                if (Q8) { ksc[r] = 0.f; vsc[r] = 0.f; }
            }
        }
    };
    auto store_tile = [&]() {
#pragma unroll
        for (int r = 0; r < Gm::ROUNDS; ++r) {
            const int pr = r * Gm::RPR + lrow;
            if (pr >= kPfTile) continue;
            h8 kv[2], vv[2];
            int nparts;
            if (Q8) {
                const int8_t* kc = reinterpret_cast<const int8_t*>(&kr[r]);
                const int8_t* vc = reinterpret_cast<const int8_t*>(&vr[r]);
#pragma unroll
                for (int j = 0; j < 8; ++j) {
                    kv[0][j] = (_Float16)((float)kc[j] * ksc[r]);
                    kv[1][j] = (_Float16)((float)kc[8 + j] * ksc[r]);
                    vv[0][j] = (_Float16)((float)vc[j] * vsc[r]);
                    vv[1][j] = (_Float16)((float)vc[8 + j] * vsc[r]);
                }
                nparts = 2;
            } else {
                kv[0] = *reinterpret_cast<h8*>(&kr[r]);
                vv[0] = *reinterpret_cast<h8*>(&vr[r]);
                nparts = 1;
            }
            const int d0 = lchunk * (Q8 ? 16 : 8);
            const int c = vt_col(pr);
#pragma unroll
            for (int part = 0; part < 2; ++part) {
                if (part >= nparts) break;
                *reinterpret_cast<h8*>(s_k + pr * Gm::KROW + (d0 + part * 8) * 2) = kv[part];
#pragma unroll
                for (int j = 0; j < 8; ++j)
                    *reinterpret_cast<_Float16*>(s_vt + (d0 + part * 8 + j) * Gm::VTROW + c * 2) = vv[part][j];
            }
        }
    };

    if (ntiles > 0) load_tile(0);
    for (int kt = 0; kt < ntiles; ++kt) {
        store_tile();
        __syncthreads();
        if (kt + 1 < ntiles) load_tile(kt + 1);
        const int tbase = kt * kPfTile;
        if (tbase < wend) {
            // S^T[pos][row] for two 16-position m-tiles x two 16-row tiles
            f4 sacc[kPfRT][2];
#pragma unroll
            for (int rt = 0; rt < kPfRT; ++rt) sacc[rt][0] = sacc[rt][1] = f4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int mt = 0; mt < 2; ++mt) {
#pragma unroll
                for (int s = 0; s < Gm::KSTEPS; ++s) {
                    const h8 a = *reinterpret_cast<const h8*>(s_k + (mt * 16 + col) * Gm::KROW + (s * 32 + kb * 8) * 2);
#pragma unroll
                    for (int rt = 0; rt < kPfRT; ++rt) sacc[rt][mt] = mfma16x16x32(a, qf[rt][s], sacc[rt][mt]);
                }
            }
            h8 pf[kPfRT];
            float alpha[kPfRT];
#pragma unroll
            for (int rt = 0; rt < kPfRT; ++rt) {
                float sc[8];
                float mx = kNegBig;
#pragma unroll
                for (int j = 0; j < 8; ++j) {
                    const int mt = j >> 2, i = j & 3;
                    float x = sacc[rt][mt][i] * p.scale2;
                    if (__builtin_isnan(x)) x = kNegBig;
                    const bool valid = tbase + mt * 16 + kb * 4 + i <= lim[rt];
                    sc[j] = valid ? x : -__builtin_inff();
                    mx = fmaxf(mx, sc[j]);
                }
                mx = wave_max_xor(mx, 16);
                mx = wave_max_xor(mx, 32);
                const float m_new = fmaxf(m_run[rt], mx);
                const float da = m_run[rt] - m_new;
                alpha[rt] = da < kCut2 ? 0.0f : exp2_fast(da);
                float psum = 0.0f;
#pragma unroll
                for (int j = 0; j < 8; ++j) {
                    const float df = sc[j] - m_new;
                    const float e = df < kCut2 ? 0.0f : exp2_fast(df);
                    const _Float16 eh = (_Float16)e;
                    pf[rt][j] = eh;
                    psum += (float)eh;
                }
                l_run[rt] = l_run[rt] * alpha[rt] + psum;
                m_run[rt] = m_new;
            }
#pragma unroll
            for (int dt = 0; dt < Gm::DTILES; ++dt) {
                const h8 va = *reinterpret_cast<const h8*>(s_vt + (dt * 16 + col) * Gm::VTROW + kb * 16);
#pragma unroll
                for (int rt = 0; rt < kPfRT; ++rt) o[rt][dt] = mfma16x16x32(va, pf[rt], o[rt][dt] * alpha[rt]);
            }
        }
        __syncthreads();
    }

    // epilogue: lane holds O^T[d = dt*16 + kb*4 + i][row col] of each row tile
#pragma unroll
    for (int rt = 0; rt < kPfRT; ++rt) {
        float L = wave_sum_xor(l_run[rt], 16);
        L = wave_sum_xor(L, 32);
        const int r = row0 + wave * kPfRowsWave + rt * 16 + col;
        if (r >= R) continue;
        const int t = r / p.G, g = r % p.G;
        _Float16* orow = reinterpret_cast<_Float16*>(p.out) + (size_t)t * qd + (size_t)(kvh * p.G + g) * D;
#pragma unroll
        for (int dt = 0; dt < Gm::DTILES; ++dt) {
            h4 v;
#pragma unroll
            for (int i = 0; i < 4; ++i) v[i] = out_half(L > 1e-12f ? o[rt][dt][i] / L : 0.0f);
            *reinterpret_cast<h4*>(orow + dt * 16 + kb * 4) = v;
        }
    }
}


// ---------------------------------------------------------------------------
// fp16 caches: LDS-DMA pipeline.
//
// A workgroup owns RA + RB 16-row tiles of one kv head (rows r = t*G + g) and streams
// the head's keys in stages of 128 positions through a two-stage LDS ring that
// global_load_lds_dwordx4 fills directly (no register staging). Its eight waves form
// two groups: group 0 holds the first RA row tiles, group 1 the next RB. Within a
// group, each of the four waves takes 32 keys of every stage for all of the group's
// row tiles, so every K/V fragment it reads from LDS feeds RA (or RB) MFMAs; the four
// waves' softmax states are merged through LDS at the end. With 128 KB of LDS per
// workgroup a CU runs one workgroup, i.e. two waves per SIMD (one of each group): while
// one wave runs its softmax on the vector unit, the other can issue its MFMAs. K and V rows stay row-major in LDS with the 16-byte chunks of row
// r stored at slot chunk ^ (r % CPR), which makes the MFMA operand reads free of bank
// conflicts; V^T comes from the transposing LDS read (ds_read_b64_tr_b16).
constexpr int kP2Slices = 4;                // key slices of a stage (one wave each per group)
constexpr int kP2Groups = 2;                // row-tile groups sharing every stage
constexpr int kP2Waves = kP2Slices * kP2Groups;
constexpr int kP2Threads = kP2Waves * 64;
// Group 0 issues every stage copy: it starts a stage behind group 1, whose QK MFMAs and
// softmax then overlap group 0's copy issue, which waits on the memory pipeline.
constexpr int kP2DmaWaves = kP2Slices;
constexpr int kP2KW = 32;                   // keys per wave per stage
constexpr int kP2KS = kP2KW * kP2Slices;    // keys per stage (128)
constexpr float kLazy = 8.0f;               // log2 slack of the reference max (weights <= 256)

template <int D>
struct P2Geo {
    static constexpr int ROWB = D * 2;                 // bytes of one K/V row
    static constexpr int CPR = ROWB / 16;              // 16-byte chunks per row
    static constexpr int RPI = 64 / CPR;               // rows per wave DMA instruction
    static constexpr int STAGE_K = kP2KS * ROWB;       // bytes of the K (or V) part of a stage
    static constexpr int STAGE = 2 * STAGE_K;
    static constexpr int NI = kP2KS / RPI / kP2DmaWaves;  // DMA instructions per wave per tensor and stage
    static constexpr int KSTEPS = D / 32;
    static constexpr int DTILES = D / 16;
    static constexpr int OROW = D + 4;                 // combine row stride (floats)
    static constexpr int CREG_BYTES = 4 * (2 * kP2Slices * 16 + kP2Slices * 16 * OROW);  // one group's merge area
    // LDS slot of 16-byte chunk c of row r: c ^ swz(r). swz is a bijection on r % CPR, so the
    // K operand reads (16 consecutive rows, one chunk) hit 16 distinct slots; and the four
    // rows a..a+3 (a % 4 == 0) of a V^T read get swz values that differ above bit 0, so their
    // chunk pairs (2 dt, 2 dt + 1) land in 8 distinct slots (r % CPR alone gave 2-way
    // bank conflicts there).
    static __device__ __forceinline__ int swz(int r) { return ((r & (CPR / 2 - 1)) << 1) | ((r / (CPR / 2)) & 1); }
};

// int8 caches: raw stage = the codes of K and V (row-major, kP2KS rows of D bytes each)
// followed by their fp16 scales (D/32 per row), copied by DMA as they lie in memory.
template <int D>
struct P2RawGeo {
    static constexpr int ROWB = D;                     // code bytes of one row
    static constexpr int CPR = ROWB / 16;              // 16-byte chunks per row
    static constexpr int RPI = 64 / CPR;               // rows per wave DMA instruction
    static constexpr int PART = kP2KS * ROWB;          // codes of K (or V) in a stage
    static constexpr int SROWB = D / 16;               // scale bytes of one row
    static constexpr int SDW = SROWB / 4;              // scale dwords of one row
    static constexpr int SPART = kP2KS * SROWB;        // scales of K (or V) in a stage
    static constexpr int NI = kP2KS / RPI / kP2DmaWaves;  // code DMA instructions per wave per tensor
    static constexpr int SI = SPART / 4 / 64;          // scale DMA instructions per tensor (one per wave)
    static constexpr int RAW = 2 * PART + 2 * SPART;
    static constexpr int NCH = 2 * kP2KS * CPR;        // 16-code chunks of a stage (K and V)
    static_assert(SI >= 1 && SI <= kP2DmaWaves && SPART % 256 == 0, "scale copy shape");
    static_assert(NCH % kP2Threads == 0, "decode shape");
};

// One wave-wide global -> LDS copy (global_load_lds_dwordx4): lane l moves 16 bytes
// from base + off (base wave-uniform, off its own) to lds + 16*l (lds wave-uniform).
// Issued from inline assembly: the compiler would otherwise drain every such copy before
// any later LDS read, including reads of the other stage buffer; the kernel waits for
// the copies itself (s_waitcnt vmcnt(0) + barrier) before reading the stage they fill.
typedef __attribute__((address_space(3))) unsigned char lds_u8;
__device__ __forceinline__ void dma16(const char* base, uint32_t off, lds_u8* lds) {
    asm volatile("s_mov_b32 m0, %0\n\tglobal_load_lds_dwordx4 %1, %2" ::"s"((uint32_t)(size_t)lds), "v"(off), "s"(base)
                 : "memory");
}

// The same copy for 4 bytes per lane (global_load_lds_dword): lane l's dword lands at lds + 4*l.
__device__ __forceinline__ void dma4(const char* base, uint32_t off, lds_u8* lds) {
    asm volatile("s_mov_b32 m0, %0\n\tglobal_load_lds_dword %1, %2" ::"s"((uint32_t)(size_t)lds), "v"(off), "s"(base)
                 : "memory");
}

// Bytes of the LDS buffers: fp16 caches use two fp16 stages (stage0, stage1); int8
// caches use one fp16 stage (stage0, decoded from the raw stage in use) and two raw
// stages (stage1, stage2), the first also holding group 1's merge area.
template <int D, bool Q8>
struct P2Lds {
    static constexpr int B0 = P2Geo<D>::STAGE;
    static constexpr int RAWB = P2RawGeo<D>::RAW > P2Geo<D>::CREG_BYTES ? P2RawGeo<D>::RAW : P2Geo<D>::CREG_BYTES;
    static constexpr int B1 = Q8 ? RAWB : P2Geo<D>::STAGE;
    static constexpr int B2 = Q8 ? RAWB : 16;
};

template <int D, int RA, int RB, bool Q8, bool BF>
__global__ __launch_bounds__(kP2Threads) void fa_prefill_dma_kernel(PrefillParams p) {
    static_assert(!(Q8 && BF), "int8 caches decode to fp16");
    using Gm = P2Geo<D>;
    using Rg = P2RawGeo<D>;
    using Lb = P2Lds<D, Q8>;
    constexpr int RT = RA;  // state arrays per lane (group 1 uses the first RB entries)
    static_assert(RB <= RA, "group 0 holds the larger share");
    // distinct stage buffers (not one array indexed by the tile's parity): the compiler
    // then sees that the DMA into one stage does not alias the LDS reads of the other
    __shared__ __align__(16) unsigned char stage0[Lb::B0];
    __shared__ __align__(16) unsigned char stage1[Lb::B1];
    __shared__ __align__(16) unsigned char stage2[Lb::B2];

    // grid x = kv head, y = row block (heaviest first): consecutive workgroup ids walk the
    // kv heads, so with round-robin placement over the XCDs one kv head's blocks share an
    // XCD and its L2 copy of K/V
    const int kvh = blockIdx.x;
    const int rb = gridDim.y - 1 - blockIdx.y;
    const int R = p.T * p.G;
    const int p0 = *p.d_pos0;
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int grp = wave / kP2Slices;  // row-tile group
    const int sl = wave % kP2Slices;   // key slice of every stage
    const int col = lane & 15, kb = lane >> 4;
    const int qd = p.Hq * D;
    const int wg_row0 = rb * (RA + RB) * 16;
    const int row0 = wg_row0 + grp * RA * 16;  // the group's first row
    const int ntl = grp == 0 ? RA : RB;        // the group's row tiles

    // Q^T fragments and causal limits of this lane's rows (one per row tile)
    h8 qf[RT][Gm::KSTEPS];
    int lim[RT];
#pragma unroll
    for (int rt = 0; rt < RT; ++rt) {
        const int r = row0 + rt * 16 + col;
        const bool valid = rt < ntl && r < R;
        const int rr = valid ? r : R - 1;
        const int t = rr / p.G, g = rr % p.G;
        lim[rt] = valid ? p0 + t : -1;
        const uint16_t* qrow = p.q + (size_t)t * qd + (size_t)(kvh * p.G + g) * D;
#pragma unroll
        for (int s = 0; s < Gm::KSTEPS; ++s) {
            const u4 raw = *reinterpret_cast<const u4*>(qrow + s * 32 + kb * 8);
            qf[rt][s] = *reinterpret_cast<const h8*>(&raw);
        }
    }
    // settle the q loads here: the compiler would otherwise wait for them at their first
    // use inside the stage loop, in every iteration, behind the stage copies
#pragma unroll
    for (int rt = 0; rt < RT; ++rt)
#pragma unroll
        for (int s = 0; s < Gm::KSTEPS; ++s) asm volatile("" ::"v"(qf[rt][s]));
    const int last_row = min(wg_row0 + (RA + RB) * 16, R) - 1;
    const int kend = p0 + last_row / p.G + 1;  // keys [0, kend) for the workgroup
    const int ntiles = (kend + kP2KS - 1) / kP2KS;
    // first token of the group's first tile: slices up to it need no causal mask
    const int grp_lo = row0 < R ? p0 + row0 / p.G : INT_MAX;

    // DMA of one stage: wave w moves rows [w*NI*RPI, (w+1)*NI*RPI) of the K and V parts
    constexpr int CROWB = Q8 ? Rg::ROWB : Gm::ROWB;  // cache bytes of one kv-head row
    constexpr int CCPR = Q8 ? Rg::CPR : Gm::CPR;
    constexpr int CRPI = Q8 ? Rg::RPI : Gm::RPI;
    constexpr int CNI = Q8 ? Rg::NI : Gm::NI;
    const size_t rowb = (size_t)p.Hkv * CROWB;
    const char* kbase = static_cast<const char*>(p.k) + (size_t)kvh * CROWB;
    const char* vbase = static_cast<const char*>(p.v) + (size_t)kvh * CROWB;
    const int drow = lane / CCPR, dslot = lane % CCPR;
    // this lane's byte offsets (row, chunk) within a stage, one per DMA instruction; fp16
    // rows land with their chunks swizzled, int8 rows as they are (the decode pass swizzles)
    uint32_t doff[CNI];
#pragma unroll
    for (int i = 0; i < CNI; ++i) {
        const int r = (wave * CNI + i) * CRPI + drow;
        doff[i] = (uint32_t)(r * (int)rowb + (Q8 ? dslot : (dslot ^ Gm::swz(r))) * 16);
    }
    lds_u8* const lds0 = (lds_u8*)(Q8 ? stage1 : stage0);
    lds_u8* const lds1 = (lds_u8*)(Q8 ? stage2 : stage1);
    // int8 scales: the row's D/32 fp16 scales are contiguous ([pos][kv_dim/32] layout)
    const size_t srowb = (size_t)p.Hkv * Rg::SROWB;
    const char* ksbase = reinterpret_cast<const char*>(p.k_scale) + (size_t)kvh * Rg::SROWB;
    const char* vsbase = reinterpret_cast<const char*>(p.v_scale) + (size_t)kvh * Rg::SROWB;
    const int srow = (wave * 64 + lane) / Rg::SDW;  // scale row of this lane's dword (waves < SI)
    const uint32_t soff = (uint32_t)(srow * (int)srowb + ((wave * 64 + lane) % Rg::SDW) * 4);
    auto issue = [&](int tile, auto stage_tag) __attribute__((always_inline)) {
        if (wave >= kP2DmaWaves) return;
        lds_u8* st = decltype(stage_tag)::value ? lds1 : lds0;
        // uniform base: the tile's first key
        const size_t tile0 = (size_t)tile * kP2KS * rowb;
        const char* kt = kbase + tile0;
        const char* vt = vbase + tile0;
        const int rmax = kend - 1 - tile * kP2KS;  // rows past it re-read the last key
        constexpr int VOFF = Q8 ? Rg::PART : Gm::STAGE_K;  // V part of the stage
        if (rmax >= kP2KS - 1) {
#pragma unroll
            for (int i = 0; i < CNI; ++i) {
                lds_u8* l = st + (wave * CNI + i) * CRPI * CROWB;
                dma16(kt, doff[i], l);
                dma16(vt, doff[i], l + VOFF);
            }
        } else {
#pragma unroll
            for (int i = 0; i < CNI; ++i) {
                const int r = (wave * CNI + i) * CRPI + drow;
                const uint32_t off = (uint32_t)(min(r, rmax) * (int)rowb + (Q8 ? dslot : (dslot ^ Gm::swz(r))) * 16);
                lds_u8* l = st + (wave * CNI + i) * CRPI * CROWB;
                dma16(kt, off, l);
                dma16(vt, off, l + VOFF);
            }
        }
        if constexpr (Q8) {
            if (wave < Rg::SI) {
                const size_t stile0 = (size_t)tile * kP2KS * srowb;
                const uint32_t off = rmax >= kP2KS - 1
                                         ? soff
                                         : (uint32_t)(min(srow, rmax) * (int)srowb + ((wave * 64 + lane) % Rg::SDW) * 4);
                lds_u8* l = st + 2 * Rg::PART + wave * 256;
                dma4(ksbase + stile0, off, l);
                dma4(vsbase + stile0, off, l + Rg::SPART);
            }
        }
    };
    // int8: the raw stage -> fp16 stage0 (same layout as the fp16 DMA: chunk slot
    // chunk ^ (row % CPR)); each 16-code chunk becomes two fp16 chunks (dequant16)
    auto decode = [&](const unsigned char* raw) __attribute__((always_inline)) {
        constexpr int NIT = Rg::NCH / kP2Threads;
        // chunks whose LDS reads are issued together: their latencies overlap; a larger batch
        // spills at the largest row-tile share
        constexpr int NB = 2;
        static_assert(NIT % NB == 0, "decode batches");
#pragma unroll 1
        for (int it0 = 0; it0 < NIT; it0 += NB) {
            u4 q[NB];
            float sc[NB];
#pragma unroll
            for (int b = 0; b < NB; ++b) {
                const int idx = (it0 + b) * kP2Threads + tid;
                const int ts = idx / (kP2KS * Rg::CPR);  // 0: K, 1: V
                const int rem = idx % (kP2KS * Rg::CPR);
                const int r = rem / Rg::CPR, c = rem % Rg::CPR;
                q[b] = *reinterpret_cast<const u4*>(raw + ts * Rg::PART + rem * 16);
                sc[b] = (float)*reinterpret_cast<const _Float16*>(raw + 2 * Rg::PART + ts * Rg::SPART +
                                                                   r * Rg::SROWB + (c >> 1) * 2);
            }
#pragma unroll
            for (int b = 0; b < NB; ++b) {
                const int idx = (it0 + b) * kP2Threads + tid;
                const int ts = idx / (kP2KS * Rg::CPR);
                const int rem = idx % (kP2KS * Rg::CPR);
                const int r = rem / Rg::CPR, c = rem % Rg::CPR;
                u4 lo, hi;
                dequant16(q[b], (_Float16)sc[b], lo, hi);  // sc[b] is an fp16 value: exact
                unsigned char* row = stage0 + ts * Gm::STAGE_K + r * Gm::ROWB;
                *reinterpret_cast<u4*>(row + (((2 * c) ^ Gm::swz(r)) * 16)) = lo;
                *reinterpret_cast<u4*>(row + (((2 * c + 1) ^ Gm::swz(r)) * 16)) = hi;
            }
        }
    };

    float m_run[RT];
    f4 o[RT][Gm::DTILES], ol[RT];
#pragma unroll
    for (int rt = 0; rt < RT; ++rt) {
        m_run[rt] = kNegBig;
        ol[rt] = f4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int i = 0; i < Gm::DTILES; ++i) o[rt][i] = f4{0.f, 0.f, 0.f, 0.f};
    }
    const h8 ones = BF ? bf16_splat_one() : h8{1, 1, 1, 1, 1, 1, 1, 1};
    const int wrow = sl * kP2KW;  // first stage row of this wave's keys

    // one stage's work for the group's N row tiles: S^T = K Q^T, online softmax, O^T += V^T P^T
    auto compute = [&](auto n_tag, const unsigned char* sk, const unsigned char* sv, int kpos0)
                       __attribute__((always_inline)) {
        constexpr int N = decltype(n_tag)::value;
        if constexpr (N > 0) {
            // K fragments (A of S^T = K Q^T) for both 16-key halves, shared by all row tiles
            h8 ka[2][Gm::KSTEPS];
#pragma unroll
            for (int mt = 0; mt < 2; ++mt) {
                const int r = wrow + mt * 16 + col;
#pragma unroll
                for (int s = 0; s < Gm::KSTEPS; ++s)
                    ka[mt][s] = *reinterpret_cast<const h8*>(sk + r * Gm::ROWB + (((4 * s + kb) ^ Gm::swz(r)) * 16));
            }
            // phase 1: S^T for every row tile (independent MFMA chains, no branches)
            f4 sacc[N][2];
#pragma unroll
            for (int rt = 0; rt < N; ++rt)
#pragma unroll
                for (int mt = 0; mt < 2; ++mt) {
                    sacc[rt][mt] = f4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
                    for (int s = 0; s < Gm::KSTEPS; ++s) sacc[rt][mt] = mma16<BF>(ka[mt][s], qf[rt][s], sacc[rt][mt]);
                }
            // phase 2: online softmax in the log2 domain; lane column = row, k-slots = keys.
            // x = raw score (its scale, scale * log2(e), is applied in the max and the weight
            // FMA); keys in a row's future -inf (only evaluated when the slice reaches past the
            // group's first row's position); the row max drops NaN scores, which then count as
            // -1e30 after scaling. The weights are taken against a reference max
            // m_run that only moves when the row max exceeds it by more than kLazy (then
            // the accumulators are rescaled): between moves the fp16 weights stay <= 2^kLazy.
            float x[N][8], mx[N];
            auto scores = [&](auto full_tag) __attribute__((always_inline)) {
                constexpr bool FULL = decltype(full_tag)::value;
#pragma unroll
                for (int rt = 0; rt < N; ++rt) {
                    float m = -__builtin_inff();
#pragma unroll
                    for (int j = 0; j < 8; ++j) {
                        const int mt = j >> 2, i = j & 3;
                        float v = sacc[rt][mt][i];
                        if (!FULL) v = kpos0 + mt * 16 + kb * 4 + i <= lim[rt] ? v : -__builtin_inff();
                        x[rt][j] = v;
                        m = fmaxf(m, v);
                    }
                    // max(s) * scale2 == max(s * scale2) exactly (scale2 > 0, rounding is monotone)
                    mx[rt] = fmaxf(col_max4(m) * p.scale2, kNegBig);
                }
            };
            const bool full = kpos0 + kP2KW - 1 <= grp_lo;
            if (full)
                scores(std::true_type{});
            else
                scores(std::false_type{});
            bool move = false;
#pragma unroll
            for (int rt = 0; rt < N; ++rt) move |= mx[rt] > m_run[rt] + kLazy;
            if (__builtin_expect(__any(move), 0)) {  // rare after the first stage
#pragma unroll
                for (int rt = 0; rt < N; ++rt) {
                    const float m_new = mx[rt] > m_run[rt] + kLazy ? mx[rt] : m_run[rt];
                    const float alpha = exp2_fast(m_run[rt] - m_new);
                    m_run[rt] = m_new;
#pragma unroll
                    for (int dt = 0; dt < Gm::DTILES; ++dt) o[rt][dt] *= alpha;
                    ol[rt] *= alpha;
                }
            }
            // weights exp2(s * scale2 - m_run) in one FMA. A NaN score counts as a scaled
            // score of -1e30: its exponent is clamped to -1e30 - m_run (weight 1 while no
            // finite score has moved m_run off -1e30, else 0); masked keys get weight 0.
            h8 pf[N];
#pragma unroll
            for (int rt = 0; rt < N; ++rt) {
                const float nb = kNegBig - m_run[rt];
#pragma unroll
                for (int j = 0; j < 8; ++j)
                    pf[rt][j] = to_p<BF>(exp2_fast(fmaxf(__builtin_fmaf(x[rt][j], p.scale2, -m_run[rt]), nb)));
            }
            if (!full) {
#pragma unroll
                for (int rt = 0; rt < N; ++rt)
#pragma unroll
                    for (int j = 0; j < 8; ++j)
                        if (x[rt][j] == -__builtin_inff()) pf[rt][j] = (_Float16)0.0f;
            }
            // V^T fragments (A of O^T += V^T P^T): k-slot j < 4 -> key kb*4 + j, j >= 4 -> 16 + kb*4 + j-4
            // (kept after the softmax: hoisted into the S phase they would not fit the registers)
            __builtin_amdgcn_sched_barrier(0);
            h8 va[Gm::DTILES];
            {
                const int r = wrow + kb * 4 + (col >> 2);
#pragma unroll
                for (int dt = 0; dt < Gm::DTILES; ++dt) {
                    const int d = dt * 16 + 4 * (col & 3);
                    const unsigned char* a = sv + r * Gm::ROWB + (((d >> 3) ^ Gm::swz(r)) * 16) + (d & 7) * 2;
                    const h4 lo = lds_read_tr16(a);
                    const h4 hi = lds_read_tr16(a + 16 * Gm::ROWB);
                    va[dt] = h8{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
                }
            }
            // phase 3: O^T += V^T P^T, and the row sums of the fp16 weights exactly as the PV
            // product sees them (P against a tile of ones)
#pragma unroll
            for (int rt = 0; rt < N; ++rt) {
#pragma unroll
                for (int dt = 0; dt < Gm::DTILES; ++dt) o[rt][dt] = mma16<BF>(va[dt], pf[rt], o[rt][dt]);
                ol[rt] = mma16<BF>(ones, pf[rt], ol[rt]);
            }
        }
    };

    auto step = [&](int tile, auto stage_tag, auto n_tag) __attribute__((always_inline)) {
        __builtin_amdgcn_sched_barrier(0);
        // the DMA of `tile` is the only one in flight: wait for it; after the barrier every
        // wave's part of the stage has landed and every wave is done with the other stage
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        __syncthreads();
        const unsigned char* sk = Q8 ? stage0 : (decltype(stage_tag)::value ? stage1 : stage0);
        const unsigned char* sv = sk + Gm::STAGE_K;
        // the next stage's DMA into the other buffer, in flight during this stage's compute
        if (tile + 1 < ntiles) issue(tile + 1, std::integral_constant<int, 1 - decltype(stage_tag)::value>{});
        if constexpr (Q8) {
            // every wave is done with the previous stage's fp16 tile (first barrier)
            decode(decltype(stage_tag)::value ? stage2 : stage1);
            __syncthreads();
        }
        const int kpos0 = tile * kP2KS + wrow;  // this wave's first key position
        compute(n_tag, sk, sv, kpos0);
    };
    using S0 = std::integral_constant<int, 0>;
    using S1 = std::integral_constant<int, 1>;
    // one copy of the stage loop per group share: the two groups run the same barriers, and
    // each copy is register-allocated on its own (a branch per stage inside one loop keeps
    // both shares' values live and spills when RA != RB)
    using NA = std::integral_constant<int, RA>;
    using NB = std::integral_constant<int, RB>;
    issue(0, S0{});
    if (RA == RB || grp == 0) {
        for (int tile = 0; tile < ntiles; tile += 2) {
            step(tile, S0{}, NA{});
            if (tile + 1 < ntiles) step(tile + 1, S1{}, NA{});
        }
    } else {
        for (int tile = 0; tile < ntiles; tile += 2) {
            step(tile, S0{}, NB{});
            if (tile + 1 < ntiles) step(tile + 1, S1{}, NB{});
        }
    }

    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();  // every wave is done reading the stages
    // ---- merge the key slices' states, one row tile per group at a time through LDS ----
    // group g uses stage buffer g: m [slices][16], l [slices][16], O [slices][16][OROW]
    static_assert(Gm::CREG_BYTES <= Lb::B0 && Gm::CREG_BYTES <= Lb::B1, "combine fits");
    float* cm = reinterpret_cast<float*>(grp ? stage1 : stage0);
    float* cl = cm + kP2Slices * 16;
    float* co = cl + kP2Slices * 16;
    const int gtid = tid % (kP2Slices * 64);
#pragma unroll
    for (int rt = 0; rt < RT; ++rt) {
        const bool act = rt < ntl;
        if (act) {
            if (kb == 0) {
                cm[sl * 16 + col] = m_run[rt];
                cl[sl * 16 + col] = ol[rt][0];
            }
#pragma unroll
            for (int dt = 0; dt < Gm::DTILES; ++dt)
                *reinterpret_cast<f4*>(co + (sl * 16 + col) * Gm::OROW + dt * 16 + kb * 4) = o[rt][dt];
        }
        __syncthreads();
        if (act) {
            for (int idx = gtid; idx < 16 * (D / 4); idx += kP2Slices * 64) {
                const int rr = idx / (D / 4), d4 = idx % (D / 4);
                const int r = row0 + rt * 16 + rr;
                if (r >= R) continue;
                float M = cm[rr];
#pragma unroll
                for (int w = 1; w < kP2Slices; ++w) M = fmaxf(M, cm[w * 16 + rr]);
                float L = 0.0f;
                f4 O = f4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
                for (int w = 0; w < kP2Slices; ++w) {
                    const float df = cm[w * 16 + rr] - M;
                    const float wt = df < kCut2 ? 0.0f : exp2_fast(df);
                    L += wt * cl[w * 16 + rr];
                    O += wt * *reinterpret_cast<const f4*>(co + (w * 16 + rr) * Gm::OROW + 4 * d4);
                }
                const int t = r / p.G, g = r % p.G;
                h4 v;
#pragma unroll
                for (int i = 0; i < 4; ++i) v[i] = out_elem<BF>(L > 1e-12f ? O[i] / L : 0.0f);
                *reinterpret_cast<h4*>(reinterpret_cast<_Float16*>(p.out) + (size_t)t * qd + (size_t)(kvh * p.G + g) * D + 4 * d4) = v;
            }
        }
        __syncthreads();
    }
}

template <int D, int RA, int RB, bool Q8, bool BF>
int launch_dma(const PrefillParams& p, hipStream_t stream) {
    const int R = p.T * p.G;
    constexpr int rows = (RA + RB) * 16;
    const dim3 grid(p.Hkv, (R + rows - 1) / rows);
    hipLaunchKernelGGL((fa_prefill_dma_kernel<D, RA, RB, Q8, BF>), grid, dim3(kP2Threads), 0, stream, p);
    return hipGetLastError() == hipSuccess ? 0 : -1;
}

// Row tiles per workgroup: about one workgroup per CU of the MI355X (256) for the
// whole launch; group 0 takes ceil(RT/2) of them, group 1 the rest, at most three per
// wave so that the registers of two waves per SIMD hold them (RT 1..6: (1,0), (1,1),
// (2,1), (2,2), (3,2), (3,3)).
template <int D, bool Q8, bool BF = false>
int launch_dma_rt(const PrefillParams& p, hipStream_t stream) {
    static const int forced = [] {
        const char* e = std::getenv("FRIDAY_ATTN_PREFILL_RT");
        return e && *e ? std::atoi(e) : 0;
    }();
    const long rows = (long)p.T * p.G * p.Hkv;
    int rt = forced > 0 ? forced : (int)((rows + 256 * 16 - 1) / (256 * 16));
    const int rt_max = 6;
    rt = rt < 1 ? 1 : (rt > rt_max ? rt_max : rt);
    switch (rt) {
        case 1: return launch_dma<D, 1, 0, Q8, BF>(p, stream);
        case 2: return launch_dma<D, 1, 1, Q8, BF>(p, stream);
        case 3: return launch_dma<D, 2, 1, Q8, BF>(p, stream);
        case 4: return launch_dma<D, 2, 2, Q8, BF>(p, stream);
        case 5: return launch_dma<D, 3, 2, Q8, BF>(p, stream);
        default: return launch_dma<D, 3, 3, Q8, BF>(p, stream);
    }
}

template <int D, bool Q8>
int launch_pf(const PrefillParams& p, hipStream_t stream) {
    const int R = p.T * p.G;
    const dim3 grid((R + kPfRowsWG - 1) / kPfRowsWG, p.Hkv);
    hipLaunchKernelGGL((fa_prefill_kernel<D, Q8>), grid, dim3(kPfThreads), 0, stream, p);
    return hipGetLastError() == hipSuccess ? 0 : -1;
}

}  // namespace

int launch_prefill(const PrefillParams& p, int head_dim, bool q8, hipStream_t stream) {
    // the int8 DMA copies the scales by dwords: a scale array off 4-byte alignment takes
    // the register-staged kernel
    const bool scale_dma = ((reinterpret_cast<uintptr_t>(p.k_scale) | reinterpret_cast<uintptr_t>(p.v_scale)) & 3) == 0;
    if (head_dim == 128)
        return !q8 ? launch_dma_rt<128, false>(p, stream)
                   : scale_dma ? launch_dma_rt<128, true>(p, stream) : launch_pf<128, true>(p, stream);
    if (head_dim == 64)
        return !q8 ? launch_dma_rt<64, false>(p, stream)
                   : scale_dma ? launch_dma_rt<64, true>(p, stream) : launch_pf<64, true>(p, stream);
    return -2;
}

int launch_prefill_bf16(const PrefillParams& p, int head_dim, hipStream_t stream) {
    if (head_dim == 128) return launch_dma_rt<128, false, true>(p, stream);
    if (head_dim == 64) return launch_dma_rt<64, false, true>(p, stream);
    return -2;
}

}  // namespace fa
