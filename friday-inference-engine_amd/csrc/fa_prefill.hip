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
// fa_prefill_dma_kernel: a workgroup of eight waves owns up to six 16-row tiles in two
// groups of four waves; stages of 128 keys are copied global -> LDS by
// global_load_lds_dwordx4 (two stage buffers, the next stage in flight during this one's
// MFMAs), each wave of a group takes 32 keys of the stage for all of its group's row tiles,
// and the four key slices' softmax states merge through LDS at the end. Q^T, O^T and the
// softmax state stay in registers. int8 caches: every wave copies its share of the next
// stage's codes raw into LDS and decodes it to fp16 itself while this stage's MFMAs run.
#include "fa_common.hpp"
#include "fa_internal.hpp"

#include <climits>
#include <cstdlib>
#include <type_traits>

namespace fa {
namespace {

// LDS-DMA pipeline.
//
// A workgroup owns RA + RB 16-row tiles of one kv head (rows r = t*G + g) and streams
// the head's keys in stages of 128 positions through a two-stage LDS ring that
// global_load_lds_dwordx4 fills directly (no register staging). Its eight waves form
// two groups: group 0 holds the first RA row tiles, group 1 the next RB. Within a
// group, each of the four waves takes 32 keys of every stage for all of the group's
// row tiles, so every K/V fragment it reads from LDS feeds RA (or RB) MFMAs; the four
// waves' softmax states are merged through LDS at the end. With 128 KB of LDS per
// workgroup (160 KB with the int8 raw codes) a CU runs one workgroup, i.e. two waves per
// SIMD (one of each group): while one wave runs its softmax on the vector unit, the other
// can issue its MFMAs. K and V rows stay row-major in LDS with the 16-byte chunks of row
// r stored at slot chunk ^ swz(r), which makes the MFMA operand reads free of bank
// conflicts; V^T comes from the transposing LDS read (ds_read_b64_tr_b16).

constexpr int kP2Slices = 4;                // key slices of a stage (one wave each per group)
constexpr int kP2Groups = 2;                // row-tile groups sharing every stage
constexpr int kP2Waves = kP2Slices * kP2Groups;
constexpr int kP2Threads = kP2Waves * 64;
// Every wave issues an equal share of each stage copy: its K rows right after the stage's
// barrier, its V rows once the wave's S^T MFMAs of the stage are issued. (Measured at
// config 4, p0 = 7680: 109.6-110.4 us; both parts at the barrier 111.7-111.9 us; group 0
// issuing all copies with K and V interleaved per instruction 117.8-119.0 us.)
constexpr int kP2DmaWaves = kP2Waves;
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

// int8 caches: each wave copies the codes of stage rows [16 w, 16 w + 16) of K and of V
// into a raw region of its own (row-major, D bytes per row) and decodes them itself, with
// the fp16 scales of its lanes' chunks loaded into registers.
template <int D>
struct P2RawGeo {
    static constexpr int ROWB = D;                     // code bytes of one row
    static constexpr int CPR = ROWB / 16;              // 16-code chunks per row
    static constexpr int RPI = 64 / CPR;               // rows per wave copy instruction
    static constexpr int WROWS = kP2KS / kP2Waves;     // stage rows per wave
    static constexpr int NI = WROWS / RPI;             // copy instructions per wave and tensor
    static constexpr int WAVE = 2 * WROWS * ROWB;      // raw bytes per wave (K rows, then V rows)
    static constexpr int RAW = kP2Waves * WAVE;
    static_assert(NI >= 1 && NI * RPI == WROWS, "copy shape");
};

// One wave-wide global -> LDS copy (global_load_lds_dwordx4): lane l moves 16 bytes
// from base + off (base wave-uniform, off its own) to lds + 16*l (lds wave-uniform).
// Issued from inline assembly: the compiler would otherwise drain every such copy before
// any later LDS read, including reads of the other stage buffer; the kernel waits for
// the copies itself (s_waitcnt vmcnt(0) + barrier) before reading the stage they fill.
// Non-temporal (nt): measured 2 % faster on int8 caches and at p0 = 0, the same elsewhere.
typedef __attribute__((address_space(3))) unsigned char lds_u8;
__device__ __forceinline__ void dma16(const char* base, uint32_t off, lds_u8* lds) {
    asm volatile("s_mov_b32 m0, %0\n\tglobal_load_lds_dwordx4 %1, %2 nt" ::"s"((uint32_t)(size_t)lds), "v"(off), "s"(base)
                 : "memory");
}

// The same copy for 4 bytes per lane (global_load_lds_dword): lane l's dword lands at lds + 4*l.
__device__ __forceinline__ void dma4(const char* base, uint32_t off, lds_u8* lds) {
    asm volatile("s_mov_b32 m0, %0\n\tglobal_load_lds_dword %1, %2" ::"s"((uint32_t)(size_t)lds), "v"(off), "s"(base)
                 : "memory");
}

// Bytes of the LDS buffers: two fp16 stages (stage0, stage1); int8 caches add the raw
// codes of one stage (stage2): 64 + 64 + 32 KiB at D = 128, the whole LDS of a CU.
template <int D, bool Q8>
struct P2Lds {
    static constexpr int B0 = P2Geo<D>::STAGE;
    static constexpr int B1 = P2Geo<D>::STAGE;
    static constexpr int B2 = Q8 ? P2RawGeo<D>::RAW : 16;
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
    // The q loads are settled once, right after the first stage copies are issued (below):
    // the compiler would otherwise wait for them at their first use inside the stage loop, in
    // every iteration, behind the stage copies; settling them here, before any copy is
    // issued, would put a whole q round trip in front of the first copy.
    auto settle_q = [&]() __attribute__((always_inline)) {
        // a full wait: the copies issued after the q loads are invisible to the compiler's
        // counting, so its partial waits would rely on the two kinds retiring in order
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
#pragma unroll
        for (int rt = 0; rt < RT; ++rt)
#pragma unroll
            for (int s = 0; s < Gm::KSTEPS; ++s) asm volatile("" ::"v"(qf[rt][s]));
    };
    const int last_row = min(wg_row0 + (RA + RB) * 16, R) - 1;
    const int kend = p0 + last_row / p.G + 1;  // keys [0, kend) for the workgroup
    const int ntiles = (kend + kP2KS - 1) / kP2KS;
    // first token of the group's first tile: slices up to it need no causal mask
    const int grp_lo = row0 < R ? p0 + row0 / p.G : INT_MAX;

    // fp16 stage copy: wave w moves rows [w*NI*RPI, (w+1)*NI*RPI) of the K part, then the same
    // rows of the V part, each 16-byte chunk to its swizzled slot. PART 1: K only, 2: V only.
    constexpr int CROWB = Q8 ? Rg::ROWB : Gm::ROWB;  // cache bytes of one kv-head row
    const size_t rowb = (size_t)p.Hkv * CROWB;
    const char* kbase = static_cast<const char*>(p.k) + (size_t)kvh * CROWB;
    const char* vbase = static_cast<const char*>(p.v) + (size_t)kvh * CROWB;
    const int drow = lane / Gm::CPR, dslot = lane % Gm::CPR;
    lds_u8* const lds0 = (lds_u8*)stage0;
    lds_u8* const lds1 = (lds_u8*)stage1;
    auto issue = [&](int tile, auto stage_tag, auto part_tag) __attribute__((always_inline)) {
        constexpr int PART = decltype(part_tag)::value;
        lds_u8* st = decltype(stage_tag)::value ? lds1 : lds0;
        // uniform base: the tile's first key
        const size_t tile0 = (size_t)tile * kP2KS * rowb;
        const char* kt = kbase + tile0;
        const char* vt = vbase + tile0;
        const int rmax = kend - 1 - tile * kP2KS;  // rows past it re-read the last key
        // (one form for every stage: a separate unclamped form for full stages, chosen by a
        // branch, measured 7 % slower at config 4, p0 = 7680)
        uint32_t off[Gm::NI];
#pragma unroll
        for (int i = 0; i < Gm::NI; ++i) {
            const int r = (wave * Gm::NI + i) * Gm::RPI + drow;
            off[i] = (uint32_t)(min(r, rmax) * (int)rowb + (dslot ^ Gm::swz(r)) * 16);
            if (PART != 2) dma16(kt, off[i], st + (wave * Gm::NI + i) * Gm::RPI * Gm::ROWB);
        }
        if (PART == 1) return;
#pragma unroll
        for (int i = 0; i < Gm::NI; ++i) dma16(vt, off[i], st + Gm::STAGE_K + (wave * Gm::NI + i) * Gm::RPI * Gm::ROWB);
    };
    // int8 stage copy: every wave loads the fp16 scales of the chunks its lanes decode into
    // registers, then moves its own rows [w*WROWS, (w+1)*WROWS) of K, then of V, into its raw
    // region (lane l's 16 codes at + 16 l of each instruction). (Config 4, int8, p0 = 7680:
    // 137.7 us; with K, V and the scales interleaved per row group 147 us.)
    const int qrow = lane / Rg::CPR, qch = lane % Rg::CPR;
    lds_u8* const rawl = (lds_u8*)stage2 + wave * Rg::WAVE;
    const int sdim = p.Hkv * (D / 32);  // scales per cache position
    const uint16_t* ksc = p.k_scale + (size_t)kvh * (D / 32) + (qch >> 1);
    const uint16_t* vsc = p.v_scale + (size_t)kvh * (D / 32) + (qch >> 1);
    uint16_t qsk[Rg::NI], qsv[Rg::NI];
    auto issue_q8 = [&](int tile) __attribute__((always_inline)) {
        const size_t tile0 = (size_t)tile * kP2KS * rowb;
        const char* kt = kbase + tile0;
        const char* vt = vbase + tile0;
        const int rmax = kend - 1 - tile * kP2KS;  // rows past it re-read the last key
        uint32_t off[Rg::NI];
#pragma unroll
        for (int i = 0; i < Rg::NI; ++i) {
            const int r = min(wave * Rg::WROWS + i * Rg::RPI + qrow, rmax);
            off[i] = (uint32_t)(r * (int)rowb + qch * 16);
            const size_t pos = (size_t)tile * kP2KS + r;
            qsk[i] = ksc[pos * sdim];
            qsv[i] = vsc[pos * sdim];
        }
#pragma unroll
        for (int i = 0; i < Rg::NI; ++i) dma16(kt, off[i], rawl + i * 1024);
#pragma unroll
        for (int i = 0; i < Rg::NI; ++i) dma16(vt, off[i], rawl + Rg::WROWS * Rg::ROWB + i * 1024);
    };
    // int8: this wave's raw rows -> the fp16 stage `dst` (the fp16 copy's layout: chunk c
    // of row r at slot c ^ swz(r)); each 16-code chunk becomes two fp16 chunks (dequant16).
    // Only this wave's own copies are read, so its own vmcnt wait covers them.
    auto decode_q8 = [&](unsigned char* dst) __attribute__((always_inline)) {
#pragma unroll
        for (int i = 0; i < Rg::NI; ++i) {
            const int r = wave * Rg::WROWS + i * Rg::RPI + qrow;
#pragma unroll
            for (int ts = 0; ts < 2; ++ts) {
                const u4 q = *reinterpret_cast<const u4*>((const unsigned char*)rawl + ts * Rg::WROWS * Rg::ROWB +
                                                          i * 1024 + lane * 16);
                const uint16_t sb = ts ? qsv[i] : qsk[i];
                u4 lo, hi;
                dequant16(q, __builtin_bit_cast(_Float16, sb), lo, hi);
                unsigned char* row = dst + ts * Gm::STAGE_K + r * Gm::ROWB;
                *reinterpret_cast<u4*>(row + (((2 * qch) ^ Gm::swz(r)) * 16)) = lo;
                *reinterpret_cast<u4*>(row + (((2 * qch + 1) ^ Gm::swz(r)) * 16)) = hi;
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
    // after_qk runs once the S^T MFMAs are issued
    auto compute = [&](auto n_tag, const unsigned char* sk, const unsigned char* sv, int kpos0, auto&& after_qk)
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
            after_qk();
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
                if constexpr (BF) {
                    const float nb = kNegBig - m_run[rt];
#pragma unroll
                    for (int j = 0; j < 8; ++j)
                        pf[rt][j] = to_p<BF>(exp2_fast(fmaxf(__builtin_fmaf(x[rt][j], p.scale2, -m_run[rt]), nb)));
                } else {
                    // the same rule on the fp16 weights, two per instruction: max(weight, w) with
                    // w the weight of a score of -1e30 (1 while m_run is -1e30, else 0, as
                    // exp2(-1e30 - m_run) rounds to 0) turns a NaN weight into w and keeps every
                    // other weight (>= 0) when w = 0. While m_run is -1e30 no finite score has been
                    // seen (it would have moved m_run), so the other weights then are those of
                    // masked keys, zeroed below, and of -inf scores, which the fp32 form also
                    // clamped to weight 1.
                    const uint32_t w = m_run[rt] == kNegBig ? 0x3C003C00u : 0u;
#pragma unroll
                    for (int j = 0; j < 8; ++j) pf[rt][j] = (_Float16)exp2_fast(__builtin_fmaf(x[rt][j], p.scale2, -m_run[rt]));
                    u4 pb = *reinterpret_cast<const u4*>(&pf[rt]);
#pragma unroll
                    for (int i = 0; i < 4; ++i) asm("v_pk_max_f16 %0, %1, %2" : "=v"(pb[i]) : "v"(pb[i]), "v"(w));
                    pf[rt] = *reinterpret_cast<const h8*>(&pb);
                }
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
        } else {
            after_qk();  // a group without row tiles still issues its share of the copies
        }
    };

    auto step = [&](int tile, auto stage_tag, auto n_tag) __attribute__((always_inline)) {
        __builtin_amdgcn_sched_barrier(0);
        constexpr int B = decltype(stage_tag)::value;
        const int kpos0 = tile * kP2KS + wrow;  // this wave's first key position
        if constexpr (Q8) {
            // stage `tile` is in fp16 buffer B (decoded by every wave, then a barrier).
            // After this stage's MFMAs are issued, the wave decodes its share of the next
            // stage (its own copies, landed during this stage) into the other buffer, which
            // every wave finished reading before the last barrier, and copies the stage
            // after it into its raw region; the decode's vector work overlaps the MFMAs.
            const unsigned char* sk = B ? stage1 : stage0;
            compute(n_tag, sk, sk + Gm::STAGE_K, kpos0, [] {});
            if (tile + 1 < ntiles) {
                asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
                decode_q8(B ? stage0 : stage1);
                if (tile + 2 < ntiles) issue_q8(tile + 2);
            }
            __syncthreads();
        } else {
            // the DMA of `tile` is the only one in flight (at tile 0 with prefetch2, tile 1's
            // too): wait for it; after the barrier every wave's part of the stage has landed and
            // every wave is done with the other stage
            asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
            __syncthreads();
            const unsigned char* sk = B ? stage1 : stage0;
            // the next stage's DMA into the other buffer, in flight during this stage's compute:
            // the K part of the next stage first, its V part once this stage's S^T MFMAs are
            // issued (measured 1 % faster than both at once at config 4, p0 = 7680); with
            // prefetch2, stage 1 went out with stage 0 at the start
            using SN = std::integral_constant<int, 1 - B>;
            const bool next = tile + 1 < ntiles && !(tile == 0 && p.prefetch2);
            if (next) issue(tile + 1, SN{}, std::integral_constant<int, 1>{});
            compute(n_tag, sk, sk + Gm::STAGE_K, kpos0, [&] {
                if (next) issue(tile + 1, SN{}, std::integral_constant<int, 2>{});
            });
        }
    };
    using S0 = std::integral_constant<int, 0>;
    using S1 = std::integral_constant<int, 1>;
    // one copy of the stage loop per group share: the two groups run the same barriers, and
    // each copy is register-allocated on its own (a branch per stage inside one loop keeps
    // both shares' values live and spills when RA != RB)
    using NA = std::integral_constant<int, RA>;
    using NB = std::integral_constant<int, RB>;
    if constexpr (Q8) {
        issue_q8(0);
        settle_q();  // q and stage 0's codes and scales were in flight together
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        decode_q8(stage0);
        if (ntiles > 1) issue_q8(1);
        __syncthreads();
    } else {
        // both stage buffers are free at the start: with prefetch2 the copy of stage 1 goes
        // out right behind stage 0's, so the first wait covers both and the copy of stage 2
        // is the first to overlap a stage's compute (one copy latency less per launch; the
        // waits stay full vmcnt(0) waits)
        issue(0, S0{}, std::integral_constant<int, 0>{});
        if (p.prefetch2 && ntiles > 1) issue(1, S1{}, std::integral_constant<int, 0>{});
        settle_q();  // q and the first copies were in flight together
    }
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
int launch_dma_rt(const PrefillParams& p_in, hipStream_t stream) {
    // FRIDAY_ATTN_PREFILL_PREFETCH2 = 0 turns the two-stage start off
    static const int prefetch2 = [] {
        const char* e = std::getenv("FRIDAY_ATTN_PREFILL_PREFETCH2");
        return e && *e ? std::atoi(e) != 0 : 1;
    }();
    PrefillParams p = p_in;
    p.prefetch2 = Q8 ? 0 : prefetch2;
    static const int forced = [] {
        const char* e = std::getenv("FRIDAY_ATTN_PREFILL_RT");
        return e && *e ? std::atoi(e) : 0;
    }();
    const long rows = (long)p.T * p.G * p.Hkv;
    const size_t cu16 = (size_t)device_cus() * 16;  // one row tile per CU and wave group
    int rt = forced > 0 ? forced : (int)((rows + cu16 - 1) / cu16);
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


}  // namespace

int launch_prefill(const PrefillParams& p, int head_dim, bool q8, hipStream_t stream) {
    if (head_dim == 128) return !q8 ? launch_dma_rt<128, false>(p, stream) : launch_dma_rt<128, true>(p, stream);
    if (head_dim == 64) return !q8 ? launch_dma_rt<64, false>(p, stream) : launch_dma_rt<64, true>(p, stream);
    return -2;
}

int launch_prefill_bf16(const PrefillParams& p, int head_dim, hipStream_t stream) {
    if (head_dim == 128) return launch_dma_rt<128, false, true>(p, stream);
    if (head_dim == 64) return launch_dma_rt<64, false, true>(p, stream);
    return -2;
}

}  // namespace fa
