// Prefill projection GEMM on gfx950: Y[t][n] = sum_k W[n][k] x_t[k] for T tokens, W in a
// GGUF K-quant / Q8_0 row layout, x in the int8 activation format of the decode GEMV
// (int8 per value, one fp32 scale per 32 values), plus the activation quantiser that
// makes that format. The reference computes per-32-value integer dot products on int8
// tensor cores and scales each in fp32 (prefill_kernels.cu:173-327); on CDNA that
// per-block scaling is vector work six times the matrix work, so here both operands are
// decoded once per workgroup into fp16 tiles in LDS (each value rounded once from its
// exact fp32 form; activations as q times their scale rounded to fp16) and a single fp16
// MFMA chain with fp32 accumulation runs over K.
//
// Tiling: a workgroup owns BN weight rows x BT tokens (256 x 128, 128 x 128 or 64 x 64,
// chosen by how well the grid fills the chip); its waves own 32 x 32 tiles of
// v_mfma_f32_32x32x16_f16 (2 x 2 of them, or one). K advances in stages of 64 values
// through two LDS buffers: while the MFMAs consume one, the raw bytes of the next stage are
// decoded into the other and those of the stage after it are in flight.
//
// Also here: the decode GEMV with int8 activations (gemvQ8), on the same block decoders.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdint>
#include <cstdlib>

#include "fa_common.hpp"
#include "fa_internal.hpp"

namespace fa {
namespace {

constexpr int kGBK = 64;  // K values per stage (two 32-value blocks)
constexpr int kGRowB = kGBK * 2;  // bytes of one fp16 tile row in LDS

// One wave-wide global -> LDS copy of 16 bytes per lane (global_load_lds_dwordx4): lane l
// moves base + off to lds + 16 l (base and lds wave-uniform). Issued from inline assembly,
// so that the compiler does not drain it before unrelated LDS accesses.
typedef __attribute__((address_space(3))) unsigned char gm_lds_u8;
// The LDS address goes through readfirstlane: it is wave-uniform, but the compiler may hold
// it in a VGPR (e.g. when derived from a boolean), which the SGPR operand cannot take.
__device__ __forceinline__ uint32_t lds_sgpr(const void* lds) {
    return (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)(size_t)lds);
}
__device__ __forceinline__ void gm_dma16(const void* base, uint32_t off, gm_lds_u8* lds) {
    asm volatile("s_mov_b32 m0, %0\n\tglobal_load_lds_dwordx4 %1, %2" ::"s"(lds_sgpr((const void*)lds)), "v"(off), "s"(base)
                 : "memory");
}

typedef _Float16 h8v __attribute__((ext_vector_type(8)));
typedef float f16v __attribute__((ext_vector_type(16)));

__device__ __forceinline__ float half_bits(uint32_t h) {
    return (float)__builtin_bit_cast(_Float16, (uint16_t)h);
}
__device__ __forceinline__ uint32_t ld32(const uint8_t* p) { return *reinterpret_cast<const uint32_t*>(p); }
__device__ __forceinline__ uint32_t ld16(const uint8_t* p) { return *reinterpret_cast<const uint16_t*>(p); }

// N 4-byte words from a 2-byte aligned address p, with aligned dword loads: from p itself
// when it is 4-byte aligned, else from p - 2 plus one 2-byte load of the tail, the words
// realigned by v_alignbyte. Reads stay within [p - 2, p + 4N): the 2 bytes before p lie in
// the same buffer (its base is 4-byte aligned and p is not).
template <int N>
__device__ __forceinline__ void ld_span_a2(const uint8_t* p, uint32_t (&out)[N]) {
    const bool mis = (reinterpret_cast<uintptr_t>(p) & 2) != 0;
    const uint32_t* a = reinterpret_cast<const uint32_t*>(p - (mis ? 2 : 0));
    uint32_t t[N + 1];
#pragma unroll
    for (int i = 0; i < N; ++i) t[i] = a[i];
    t[N] = mis ? (uint32_t)*reinterpret_cast<const uint16_t*>(a + N) : 0u;
#pragma unroll
    for (int i = 0; i < N; ++i) out[i] = mis ? __builtin_amdgcn_alignbyte(t[i + 1], t[i], 2) : t[i];
}

// One 32-value block of a weight row: byte l of u (unsigned) maps to ws[l/16] * byte + c[l/16].
// Offsets of the signed kinds are folded into c (c = -off * ws, exact: off is a power of 2),
// the mins of Q2_K / Q4_K / Q5_K are c = -min.
struct WBlock {
    uint32_t u[8];
    float ws[2], c[2];
};

// Word i / 4 of the 12 scale bytes (s0, s1, s2), chosen with bit masks: a select on a
// wave-uniform index becomes a branch, which would split the stage's MFMAs from its decode.
__device__ __forceinline__ uint32_t pick3(int i, uint32_t s0, uint32_t s1, uint32_t s2) {
    const uint32_t m0 = 0u - (uint32_t)(i < 4), m2 = 0u - (uint32_t)(i >= 8);
    return (s0 & m0) | (s1 & ~(m0 | m2)) | (s2 & m2);
}

// get_scale_min_k4: 6-bit scale and min of block j (0..7) of a Q4_K / Q5_K superblock
__device__ __forceinline__ void scale_min_k4(int j, uint32_t s0, uint32_t s1, uint32_t s2, int& sc, int& m) {
    auto byte = [&](int i) { return (int)((pick3(i, s0, s1, s2) >> (8 * (i & 3))) & 0xFF); };
    // (a scalar branch on the stage-uniform j: measured faster than blending both forms)
    if (j < 4) {
        sc = byte(j) & 63;
        m = byte(j + 4) & 63;
    } else {
        sc = (byte(j + 4) & 0xF) | ((byte(j - 4) >> 6) << 4);
        m = (byte(j + 4) >> 4) | ((byte(j) >> 6) << 4);
    }
}

// Raw words of block `blk` (0..K/32-1) of one weight row, per GGML layout:
//   Q2_K  scales[16] qs[64] d dmin              84 B / 256, q = 2 bits, per-16 4-bit scale & min
//   Q3_K  hmask[32] qs[64] scales[12] d         110 B, q = 2 bits + hmask bit - 4, per-16 6-bit scale - 32
//   Q4_K  d dmin scales[12] qs[128]             144 B, q = nibble, per-32 6-bit scale & min
//   Q5_K  d dmin scales[12] qh[32] qs[128]      176 B, q = nibble + qh bit << 4
//   Q6_K  ql[128] qh[64] scales[16] d           210 B, q = nibble + 2 bits << 4 - 32, per-16 int8 scale
//   Q8_0  d qs[32]                              34 B / 32, q = int8
// (dequant32, prefill_kernels.cu:57-144; dequantizeRow, cpu_kquants.cpp:227-280).
// load_wraw only issues the loads; decode_wraw does the bit work once they are needed, so
// the loads of the next stage stay in flight across this stage's MFMAs.
struct WRaw {
    uint32_t a[8], b[8];  // the block's quant bits (qs / ql) and high bits (hmask / qh)
    uint32_t s[3];        // packed scales
    uint32_t d;           // fp16 d (and dmin)
};

template <int KIND>
__device__ __forceinline__ void load_wraw(const uint8_t* row, int blk, WRaw& r) {
    const int sb = blk >> 3, j = blk & 7;
    if constexpr (KIND == kKqQ2K) {
        const uint8_t* b = row + (size_t)sb * 84;
        const int h = j >> 2, s = j & 3;
#pragma unroll
        for (int w = 0; w < 8; ++w) r.a[w] = ld32(b + 16 + 32 * h + 4 * w);
        r.s[0] = ld32(b + 8 * h + 4 * (s >> 1));
        r.d = ld32(b + 80);
    } else if constexpr (KIND == kKqQ3K) {
        const uint8_t* b = row + (size_t)sb * 110;
        const int h = j >> 2;
        ld_span_a2<8>(b + 32 + 32 * h, r.a);
        ld_span_a2<8>(b, r.b);
        ld_span_a2<3>(b + 96, r.s);
        r.d = ld16(b + 108);
    } else if constexpr (KIND == kKqQ4K || KIND == kKqQ5K) {
        constexpr bool Q5 = KIND == kKqQ5K;
        const uint8_t* b = row + (size_t)sb * (Q5 ? 176 : 144);
        const uint8_t* qs = b + (Q5 ? 48 : 16) + 32 * (j >> 1);
#pragma unroll
        for (int w = 0; w < 8; ++w) {
            r.a[w] = ld32(qs + 4 * w);
            if constexpr (Q5) r.b[w] = ld32(b + 16 + 4 * w);
        }
        r.s[0] = ld32(b + 4);
        r.s[1] = ld32(b + 8);
        r.s[2] = ld32(b + 12);
        r.d = ld32(b);
    } else if constexpr (KIND == kKqQ6K) {
        const uint8_t* b = row + (size_t)sb * 210;
        const int h = j >> 2, p = j & 3;
        ld_span_a2<8>(b + 64 * h + 32 * (p & 1), r.a);
        ld_span_a2<8>(b + 128 + 32 * h, r.b);
        r.s[0] = ld16(b + 192 + 8 * h + 2 * p);
        r.d = ld16(b + 208);
    } else {  // Q8_0
        const uint8_t* b = row + (size_t)blk * 34;
        ld_span_a2<8>(b + 2, r.a);
        r.d = ld16(b);
    }
}

template <int KIND>
__device__ __forceinline__ void decode_wraw(const WRaw& r, int blk, WBlock& o) {
    const int j = blk & 7;
    if constexpr (KIND == kKqQ2K) {
        const int s = j & 3;
#pragma unroll
        for (int w = 0; w < 8; ++w) o.u[w] = (r.a[w] >> (2 * s)) & 0x03030303u;
        const uint32_t scw = r.s[0] >> (16 * (s & 1));
        const float d = half_bits(r.d & 0xFFFF), dmin = half_bits(r.d >> 16);
#pragma unroll
        for (int c = 0; c < 2; ++c) {
            const int sc = (scw >> (8 * c)) & 0xFF;
            o.ws[c] = d * (float)(sc & 0xF);
            o.c[c] = -(dmin * (float)(sc >> 4));
        }
    } else if constexpr (KIND == kKqQ3K) {
        const int h = j >> 2, s = j & 3;
#pragma unroll
        for (int w = 0; w < 8; ++w) {
            const uint32_t lo = (r.a[w] >> (2 * s)) & 0x03030303u;
            const uint32_t hb = (r.b[w] >> (4 * h + s)) & 0x01010101u;
            o.u[w] = lo | (hb << 2);  // q + 4, 0..7
        }
        auto byte = [&](int i) {  // masks, not an indexed array (which would live in scratch)
            return (int)((pick3(i, r.s[0], r.s[1], r.s[2]) >> (8 * (i & 3))) & 0xFF);
        };
        const float d = half_bits(r.d);
#pragma unroll
        for (int c = 0; c < 2; ++c) {
            const int g = 8 * h + 2 * s + c;
            const int lo = g < 8 ? (byte(g) & 0xF) : (byte(g - 8) >> 4);
            const int hi = (byte(8 + (g & 3)) >> (2 * (g >> 2))) & 3;
            o.ws[c] = d * (float)((lo | (hi << 4)) - 32);
            o.c[c] = -4.0f * o.ws[c];
        }
    } else if constexpr (KIND == kKqQ4K || KIND == kKqQ5K) {
        const int hi = j & 1;
#pragma unroll
        for (int w = 0; w < 8; ++w) {
            uint32_t v = (r.a[w] >> (4 * hi)) & 0x0F0F0F0Fu;
            if constexpr (KIND == kKqQ5K) v |= ((r.b[w] >> j) & 0x01010101u) << 4;
            o.u[w] = v;
        }
        int sc, m;
        scale_min_k4(j, r.s[0], r.s[1], r.s[2], sc, m);
        o.ws[0] = o.ws[1] = half_bits(r.d & 0xFFFF) * (float)sc;
        o.c[0] = o.c[1] = -(half_bits(r.d >> 16) * (float)m);
    } else if constexpr (KIND == kKqQ6K) {
        const int p = j & 3;
#pragma unroll
        for (int w = 0; w < 8; ++w) {
            const uint32_t lo = (p < 2 ? r.a[w] : r.a[w] >> 4) & 0x0F0F0F0Fu;
            const uint32_t hb = (r.b[w] >> (2 * p)) & 0x03030303u;
            o.u[w] = lo | (hb << 4);  // q + 32, 0..63
        }
        const float d = half_bits(r.d);
#pragma unroll
        for (int c = 0; c < 2; ++c) {
            o.ws[c] = d * (float)(int8_t)((r.s[0] >> (8 * c)) & 0xFF);
            o.c[c] = -32.0f * o.ws[c];
        }
    } else {  // Q8_0
#pragma unroll
        for (int w = 0; w < 8; ++w) o.u[w] = r.a[w] ^ 0x80808080u;  // q + 128
        o.ws[0] = o.ws[1] = half_bits(r.d);
        o.c[0] = o.c[1] = -128.0f * o.ws[0];
    }
}

// byte i of w as a float (v_cvt_f32_ubyte{0..3})
__device__ __forceinline__ float ubyte(uint32_t w, int i) { return (float)((w >> (8 * i)) & 0xFF); }

// LDS tiles: row r of a tile holds 64 fp16 values (128 bytes, eight 16-byte chunks); chunk c
// is stored at slot c ^ ((r >> 1) & 7). A 16-byte access serves 16 lanes per cycle over a
// 256-byte bank window (two rows): the 16 rows a fragment read touches then land on 16
// distinct (row parity, slot) pairs, and so do the 8 rows x 2 halves of a tile write.
__device__ __forceinline__ int tile_off(int r, int chunk) { return r * kGRowB + ((chunk ^ ((r >> 1) & 7)) * 16); }

typedef _Float16 h2v __attribute__((ext_vector_type(2)));

// fp16(a * b + c) in one rounding, fp32 operands (v_fma_mix), into the low / high half of d
__device__ __forceinline__ uint32_t fma_mix_lo(float a, float b, float c) {
    uint32_t d;
    asm("v_fma_mixlo_f16 %0, %1, %2, %3" : "=v"(d) : "v"(a), "v"(b), "v"(c));
    return d;
}
__device__ __forceinline__ uint32_t fma_mix_hi(uint32_t d, float a, float b, float c) {
    asm("v_fma_mixhi_f16 %0, %1, %2, %3" : "+v"(d) : "v"(a), "v"(b), "v"(c));
    return d;
}

// 32 decoded weight values -> row r of an fp16 tile, chunks 4*half .. 4*half+3:
// value l = fp16(ws[l/16] * byte_l + c[l/16]) rounded once from the exact fp32 form
__device__ __forceinline__ void store_w32(unsigned char* tile, int r, int half, uint32_t (&u)[8],
                                          const float (&ws)[2], const float (&c)[2]) {
#pragma unroll
    for (int w = 0; w < 8; ++w) asm volatile("" : "+v"(u[w]));  // keep the masked words: one cvt per byte
#pragma unroll
    for (int ch = 0; ch < 4; ++ch) {
        uint32_t o[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const int l = 8 * ch + 2 * e;  // values l, l + 1 (bytes of word l / 4)
            const uint32_t wd = u[l >> 2];
            const float s = ws[l >> 4], cc = c[l >> 4];
            const float b0 = ubyte(wd, l & 3), b1 = ubyte(wd, (l & 3) + 1);
            o[e] = fma_mix_hi(fma_mix_lo(s, b0, cc), s, b1, cc);
        }
        *reinterpret_cast<uint4*>(tile + tile_off(r, 4 * half + ch)) = uint4{o[0], o[1], o[2], o[3]};
    }
}

// 32 int8 activations (two 16-byte words) and their fp32 scale -> row r of an fp16 tile:
// byte (q ^ 0x80) spliced under the fp16 exponent byte 0x66 is 1664 + q exactly; minus 1664
// (exact) times the scale rounded to fp16, in packed fp16 (one rounding of q * fp16(xd))
__device__ __forceinline__ void store_x32(unsigned char* tile, int r, int half, const uint4& xa, const uint4& xb,
                                          float xd) {
    const h2v s2 = h2v{(_Float16)xd, (_Float16)xd};
    const h2v bias = h2v{(_Float16)1664.0f, (_Float16)1664.0f};
    const uint32_t in[8] = {xa.x, xa.y, xa.z, xa.w, xb.x, xb.y, xb.z, xb.w};
#pragma unroll
    for (int ch = 0; ch < 4; ++ch) {
        uint32_t o[4];
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            const uint32_t u = in[2 * ch + i] ^ 0x80808080u;
            const uint32_t d0 = __builtin_amdgcn_perm(0x66666666u, u, 0x04010400u);  // bytes u0 66 u1 66
            const uint32_t d1 = __builtin_amdgcn_perm(0x66666666u, u, 0x04030402u);  // bytes u2 66 u3 66
            o[2 * i] = __builtin_bit_cast(uint32_t, (__builtin_bit_cast(h2v, d0) - bias) * s2);
            o[2 * i + 1] = __builtin_bit_cast(uint32_t, (__builtin_bit_cast(h2v, d1) - bias) * s2);
        }
        *reinterpret_cast<uint4*>(tile + tile_off(r, 4 * half + ch)) = uint4{o[0], o[1], o[2], o[3]};
    }
}

__device__ __forceinline__ uint16_t clamp_to_half_bits(float r) {
    if (__builtin_isnan(r)) r = 0.0f;
    r = fminf(fmaxf(r, -65504.0f), 65504.0f);
    return __builtin_bit_cast(uint16_t, (_Float16)r);
}

// storeY (prefill_kernels.cu:155-171): fp16 rounding, then + bias (fp32), then + residual
// (fp16), each sum with NaN -> 0 on its inputs and clamped to the fp16 range
__device__ __forceinline__ uint16_t epilogue(float acc, const float* bias, const uint16_t* res_row, int n) {
    uint16_t h = __builtin_bit_cast(uint16_t, (_Float16)acc);
    if (bias) {
        float t = half_bits(h), b = bias[n];
        if (__builtin_isnan(t)) t = 0.0f;
        if (__builtin_isnan(b)) b = 0.0f;
        h = clamp_to_half_bits(t + b);
    }
    if (res_row) {
        float t = half_bits(res_row[n]), a = half_bits(h);
        if (__builtin_isnan(t)) t = 0.0f;
        if (__builtin_isnan(a)) a = 0.0f;
        h = clamp_to_half_bits(t + a);
    }
    return h;
}

// The same with the bias and residual values loaded beforehand (present: hb / hr).
__device__ __forceinline__ uint16_t epilogue_pre(float acc, bool hb, float b, bool hr, uint16_t r) {
    uint16_t h = __builtin_bit_cast(uint16_t, (_Float16)acc);
    if (hb) {
        float t = half_bits(h);
        if (__builtin_isnan(t)) t = 0.0f;
        if (__builtin_isnan(b)) b = 0.0f;
        h = clamp_to_half_bits(t + b);
    }
    if (hr) {
        float t = half_bits(r), a = half_bits(h);
        if (__builtin_isnan(t)) t = 0.0f;
        if (__builtin_isnan(a)) a = 0.0f;
        h = clamp_to_half_bits(t + a);
    }
    return h;
}

// A decode-GEMV wave's epilogue operands, loaded when the wave starts (after its reduction
// they cost two more dependent round trips): bias[row] and res[row] through descriptors of
// size 0 when absent (zeros, no access; rows past N read zeros too).
struct GemvEpi {
    float b;
    uint16_t r;
};
__device__ __forceinline__ GemvEpi gemv_epi_load(const KqGemvParams& p, int row) {
    const __amdgpu_buffer_rsrc_t rb = uniform_rsrc(p.bias, p.bias ? (uint32_t)p.N * 4u : 0u);
    const __amdgpu_buffer_rsrc_t rr = uniform_rsrc(p.res, p.res ? (uint32_t)p.N * 2u : 0u);
    GemvEpi e;
    e.b = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rb, row * 4, 0, 0));
    e.r = (uint16_t)__builtin_amdgcn_raw_buffer_load_b16(rr, row * 2, 0, 0);
    return e;
}

// Workgroup shape: WVN x WVT waves, each owning TN x TT tiles of 32 x 32 (rows x tokens),
// so BN = 32 WVN TN weight rows and BT = 32 WVT TT tokens per workgroup. Staging: thread
// u < 2 BN decodes half u % 2 (32 values) of weight row u / 2 of each stage, thread
// u >= NT - 2 BT the same for token row (u - (NT - 2 BT)) / 2.
template <int KIND, int WVN, int WVT, int TN, int TT, bool XH>
__global__ __launch_bounds__(64 * WVN * WVT) void kq_gemm_kernel(KqGemmParams p) {
    constexpr int NT = 64 * WVN * WVT;
    constexpr int BN = 32 * WVN * TN, BT = 32 * WVT * TT;
    static_assert(2 * BN <= NT && 2 * BT <= NT, "one staging unit per thread and role");
    __shared__ __align__(16) unsigned char sw0[BN * kGRowB];
    __shared__ __align__(16) unsigned char sw1[BN * kGRowB];
    __shared__ __align__(16) unsigned char sx0[BT * kGRowB];
    __shared__ __align__(16) unsigned char sx1[BT * kGRowB];

    // workgroup -> (row block, token block): the token blocks of one row block get ids
    // that are equal mod 8, so with round-robin placement over the 8 XCDs they share an
    // XCD and its L2 copy of the weight rows
    const int nrb = (p.N + BN - 1) / BN, ntb = (p.T + BT - 1) / BT;
    const int id = blockIdx.x;
    // K split z = blockIdx.y covers the stages [sbeg, sbeg + nst) (all of K when ksplit = 1)
    const int z = blockIdx.y;
    const int sps = p.ksplit > 1 ? p.sps : p.K / kGBK;
    const int sbeg = z * sps;
    const int nst = min(p.K / kGBK - sbeg, sps);
    const int rb = (id % 8) + 8 * (id / (8 * ntb));
    const int tb = (id / 8) % ntb;
    if (rb >= nrb) return;  // padding of the last group of 8 row blocks
    const int n0 = rb * BN, t0 = tb * BT;

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wn = wave % WVN, wt = wave / WVN;

    // staging roles (wave-uniform: 2 BN and NT - 2 BT are multiples of 64)
    const bool w_role = tid < 2 * BN;
    const bool x_role = tid >= NT - 2 * BT;
    const int wr_ = tid >> 1, xr_ = (tid - (NT - 2 * BT)) >> 1, lh = tid & 1;
    const size_t row_bytes = p.row_bytes;
    const bool w_ok = w_role && n0 + wr_ < p.N;
    const bool x_ok = x_role && t0 + xr_ < p.T;
    const uint8_t* wrow = p.W + (size_t)(w_ok ? n0 + wr_ : 0) * row_bytes;
    const int8_t* xrow = p.xq + (size_t)(x_ok ? t0 + xr_ : 0) * p.K;
    const float* xdrow = p.xd + (size_t)(x_ok ? t0 + xr_ : 0) * (p.K / 32);
    // XH: the activations were dequantised to fp16 once for the whole call (dequant_x_kernel,
    // the same bits as store_x32). The x-role waves copy a stage's tile straight into LDS
    // (gm_dma16), 8 tile rows per instruction: lane l fills row 8i + l/8, slot l%8, i.e.
    // chunk (l%8) ^ ((row >> 1) & 7) of the row (tile_off's swizzle); rows past T re-read
    // row T - 1 (their outputs are not stored).
    constexpr int XWAVES = 2 * BT / 64;           // x-role waves
    constexpr int XNI = BT / 8 / XWAVES;          // copies per x-role wave and stage
    static_assert(XNI * XWAVES * 8 == BT, "x copy shape");
    const int xw = wave - (NT - 2 * BT) / 64;     // index among the x-role waves
    uint32_t xoff[XNI];
#pragma unroll
    for (int i = 0; i < XNI; ++i) {
        const int r = (xw * XNI + i) * 8 + (lane >> 3);
        const int t = min(t0 + r, p.T - 1);
        xoff[i] = (uint32_t)(((size_t)t * p.K + (((lane & 7) ^ ((r >> 1) & 7)) * 8)) * 2);
    }
    // every wave has a role when the tile shape gives one to every thread: then the role
    // tests are compile-time true (no branch splits the stage's MFMAs from its decode)
    const bool w_wave = 2 * BN >= NT ? true : (bool)__builtin_amdgcn_readfirstlane(w_role);
    const bool x_wave = NT - 2 * BT <= 0 ? true : (bool)__builtin_amdgcn_readfirstlane(x_role);

    // raw operands of one stage in registers; two sets, so that the loads of stage s + 2
    // are in flight across the MFMAs of stage s and the decode of stage s + 1
    struct Raw {
        WRaw w;
        uint4 xa, xb;
        float xs;
    };
    Raw raw0, raw1;
    // XH copy of stage st into the tile sx, issued one stage ahead. Every wave waits for all
    // of its vector memory operations (s_waitcnt vmcnt(0)) before the barrier that publishes
    // the stage: a partial count does not cover a global->LDS copy (measured: a ring of such
    // copies waited with constant partial counts read stale tiles now and then), and the full
    // wait costs nothing measurable here.
    auto load_xh = [&](int st, unsigned char* sx) __attribute__((always_inline)) {
        if (x_wave) {
            const uint16_t* base = p.xh + (size_t)st * kGBK;
#pragma unroll
            for (int i = 0; i < XNI; ++i) gm_dma16(base, xoff[i], (gm_lds_u8*)(sx + (xw * XNI + i) * 8 * kGRowB));
        }
    };
    auto wait_x = [&]() __attribute__((always_inline)) {
        if (XH) wait_vmem();
    };
    auto load_stage = [&](Raw& r, int st) __attribute__((always_inline)) {
        const int blk = st * (kGBK / 32) + lh;
        if (w_wave) load_wraw<KIND>(wrow, blk, r.w);
        if (!XH && x_wave) {
            r.xa = *reinterpret_cast<const uint4*>(xrow + 32 * blk);
            r.xb = *reinterpret_cast<const uint4*>(xrow + 32 * blk + 16);
            r.xs = xdrow[blk];
        }
    };
    auto store_stage = [&](const Raw& r, int st, unsigned char* sw, unsigned char* sx) __attribute__((always_inline)) {
        if (w_wave) {
            WBlock wb;
            decode_wraw<KIND>(r.w, st * (kGBK / 32) + lh, wb);
            if (!w_ok) {
                wb.ws[0] = wb.ws[1] = wb.c[0] = wb.c[1] = 0.0f;
            }
            store_w32(sw, wr_, lh, wb.u, wb.ws, wb.c);
        }
        if (!XH && x_wave) store_x32(sx, xr_, lh, r.xa, r.xb, x_ok ? r.xs : 0.0f);
    };

    f16v acc[TN][TT];
#pragma unroll
    for (int i = 0; i < TN; ++i)
#pragma unroll
        for (int j = 0; j < TT; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;

    auto compute = [&](const unsigned char* sw, const unsigned char* sx) __attribute__((always_inline)) {
#pragma unroll
        for (int kk = 0; kk < kGBK / 16; ++kk) {
            const int ch = 2 * kk + (lane >> 5);  // this lane's 8 K values of the 16
            h8v a[TN], b[TT];
#pragma unroll
            for (int i = 0; i < TN; ++i) {
                const int r = (wn * TN + i) * 32 + (lane & 31);
                a[i] = *reinterpret_cast<const h8v*>(sw + tile_off(r, ch));
            }
#pragma unroll
            for (int j = 0; j < TT; ++j) {
                const int r = (wt * TT + j) * 32 + (lane & 31);
                b[j] = *reinterpret_cast<const h8v*>(sx + tile_off(r, ch));
            }
#pragma unroll
            for (int i = 0; i < TN; ++i)
#pragma unroll
                for (int j = 0; j < TT; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a[i], b[j], acc[i][j], 0, 0, 0);
        }
    };

    // stage st: loads of st + 2 into the set that held st, MFMAs on LDS buffer st % 2,
    // decode of st + 1 (loaded one stage earlier) into the other buffer, barrier
    // (st counts from the split's first stage)
    // (XH: the activation copy of stage st + 1 is issued at the top of stage st, into the
    // buffer that stage st - 1 used, and waited for before the barrier that ends stage st)
    if (XH) load_xh(sbeg, sx0);
    load_stage(raw0, sbeg);
    if (nst > 1) load_stage(raw1, sbeg + 1);
    store_stage(raw0, sbeg, sw0, sx0);
    wait_x();
    __syncthreads();
    int st = 0;
    // steady state (every guard below true, no branch between a stage's MFMAs and the decode
    // of the next): measured 4-8 % faster than the guarded loop alone on Q4_K / Q2_K / Q3_K
    for (; st + 3 < nst; st += 2) {
        if (XH) load_xh(sbeg + st + 1, sx1);
        load_stage(raw0, sbeg + st + 2);
        compute(sw0, sx0);
        store_stage(raw1, sbeg + st + 1, sw1, sx1);
        wait_x();
        __syncthreads();
        if (XH) load_xh(sbeg + st + 2, sx0);
        load_stage(raw1, sbeg + st + 3);
        compute(sw1, sx1);
        store_stage(raw0, sbeg + st + 2, sw0, sx0);
        wait_x();
        __syncthreads();
    }
    for (; st < nst; st += 2) {
        if (XH && st + 1 < nst) load_xh(sbeg + st + 1, sx1);
        if (st + 2 < nst) load_stage(raw0, sbeg + st + 2);
        compute(sw0, sx0);
        if (st + 1 < nst) store_stage(raw1, sbeg + st + 1, sw1, sx1);
        wait_x();
        __syncthreads();
        if (st + 1 >= nst) break;
        if (XH && st + 2 < nst) load_xh(sbeg + st + 2, sx0);
        if (st + 3 < nst) load_stage(raw1, sbeg + st + 3);
        compute(sw1, sx1);
        if (st + 2 < nst) store_stage(raw0, sbeg + st + 2, sw0, sx0);
        wait_x();
        __syncthreads();
    }

    // K split: every split writes its accumulators as fp32 partials, float4 v of thread tid
    // at float4 index ((z * gridDim.x + id) * NV + v) * NT + tid, written through to the
    // device coherence point; the last of the tile's splits to arrive adds them in split
    // order (the same bits whichever split arrives last), applies the epilogue and re-arms
    // the tile's counter
    if (p.ksplit > 1) {
        constexpr int NV = TN * TT * 4;
        const __amdgpu_buffer_rsrc_t rp = coherent_rsrc(p.part, 0x7fffffff);
        auto off = [&](int zz, int v) { return (uint32_t)((((size_t)zz * gridDim.x + id) * NV + v) * NT + tid) * 16u; };
#pragma unroll
        for (int i = 0; i < TN; ++i)
#pragma unroll
            for (int j = 0; j < TT; ++j)
#pragma unroll
                for (int q = 0; q < 4; ++q)
                    st_coherent4(rp, off(z, (i * TT + j) * 4 + q),
                                 f4{acc[i][j][4 * q], acc[i][j][4 * q + 1], acc[i][j][4 * q + 2], acc[i][j][4 * q + 3]});
        __shared__ int s_last;
        wait_vmem();
        __syncthreads();
        if (tid == 0) {
            int* cnt = p.counters + (size_t)id * kCounterStride;
            const int prev = __hip_atomic_fetch_add(cnt, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            s_last = prev == p.ksplit - 1;
            if (s_last) __hip_atomic_store(cnt, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
        __syncthreads();
        if (!s_last) return;
#pragma unroll
        for (int i = 0; i < TN; ++i)
#pragma unroll
            for (int j = 0; j < TT; ++j)
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    const int v = (i * TT + j) * 4 + q;
                    const f4 mine = f4{acc[i][j][4 * q], acc[i][j][4 * q + 1], acc[i][j][4 * q + 2], acc[i][j][4 * q + 3]};
                    f4 tot = z == 0 ? mine : ld_coherent4(rp, off(0, v));
                    for (int zz = 1; zz < p.ksplit; ++zz) tot += zz == z ? mine : ld_coherent4(rp, off(zz, v));
#pragma unroll
                    for (int e = 0; e < 4; ++e) acc[i][j][4 * q + e] = tot[e];
                }
    }

    // acc[i][j][r]: weight row n0 + (wn TN + i) 32 + 8(r/4) + 4(lane/32) + r%4,
    // token t0 + (wt TT + j) 32 + lane%32
#pragma unroll
    for (int j = 0; j < TT; ++j) {
        const int t = t0 + (wt * TT + j) * 32 + (lane & 31);
        if (t >= p.T) continue;
        uint16_t* yrow = p.Y + (size_t)t * p.ldy;
        const uint16_t* rrow = p.res ? p.res + (size_t)t * p.ldy : nullptr;
#pragma unroll
        for (int i = 0; i < TN; ++i)
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int n = n0 + (wn * TN + i) * 32 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
                if (n < p.N) yrow[n] = epilogue(acc[i][j][r], p.bias, rrow, n);
            }
    }
}

// Decode GEMV with int8 activations (gemvQ8, hpc_k_quants.cu:440-700, 904-931): y = W x for
// one quantised activation vector, one wave per weight row (rows >= N from W2 into y2).
// Lane l takes the 32-value blocks l, l + 64, ... of the row; per block the integer dot
// products of each 16-value half with v_dot4_i32_i8 (exact, as the reference's dp4a) and
// the activation sums for the min / offset term, scaled in fp32; a wave sum; the storeQ8
// epilogue. HBM-bound: every weight byte is read once.
template <int KIND>
__global__ __launch_bounds__(256) void kq_gemv_kernel(KqGemvParams p) {
    const int lane = threadIdx.x & 63;
    int row = blockIdx.x * 4 + (threadIdx.x >> 6);
    const int rows = p.W2 ? 2 * p.N : p.N;
    if (row >= rows) return;  // the whole wave
    const uint8_t* W = p.W;
    uint16_t* y = p.y;
    if (p.W2 && row >= p.N) {
        W = p.W2;
        y = p.y2;
        row -= p.N;
    }
    const uint8_t* wrow = W + (size_t)row * p.row_bytes;
    const GemvEpi epi = gemv_epi_load(p, row);
    const int nblk = p.K / 32;
    float acc = 0.0f;
    for (int blk = lane; blk < nblk; blk += 64) {
        WRaw r;
        load_wraw<KIND>(wrow, blk, r);
        const uint4 xa = *reinterpret_cast<const uint4*>(p.xq + 32 * blk);
        const uint4 xb = *reinterpret_cast<const uint4*>(p.xq + 32 * blk + 16);
        const float dx = p.xd[blk];
        WBlock b;
        decode_wraw<KIND>(r, blk, b);
        const int x[8] = {(int)xa.x, (int)xa.y, (int)xa.z, (int)xa.w, (int)xb.x, (int)xb.y, (int)xb.z, (int)xb.w};
        int dot[2] = {0, 0}, xs[2] = {0, 0};
        float cs[2] = {b.c[0], b.c[1]};
#pragma unroll
        for (int w = 0; w < 8; ++w) {
            // Q8_0: the signed codes themselves (u = q + 128 would not fit a signed byte)
            const int wv = KIND == kKqQ80 ? (int)r.a[w] : (int)b.u[w];
            dot[w >> 2] = __builtin_amdgcn_sdot4(wv, x[w], dot[w >> 2], false);
            xs[w >> 2] = __builtin_amdgcn_sdot4(0x01010101, x[w], xs[w >> 2], false);
        }
        if (KIND == kKqQ80) cs[0] = cs[1] = 0.0f;
        acc += dx * (b.ws[0] * (float)dot[0] + cs[0] * (float)xs[0] + b.ws[1] * (float)dot[1] + cs[1] * (float)xs[1]);
    }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) acc += __shfl_xor(acc, off, 64);
    if (lane == 0) y[row] = epilogue_pre(acc, p.bias != nullptr, epi.b, p.res != nullptr, epi.r);
}

// LDS-staged decode GEMV: a workgroup of ROWS waves takes ROWS consecutive weight rows
// (contiguous bytes) and copies them into LDS in one burst of global->LDS copies (every copy
// in flight at once, no registers), optionally followed by the activations (XL); then each
// wave computes its row as kq_gemv_kernel does, reading the blocks from LDS. Rows start in
// LDS at the same offsets mod 4 as in memory, so the 2-byte aligned kinds use the same
// realigning loads.
typedef __attribute__((address_space(3))) unsigned char gv_lds_u8;
// The GEMV's copies (the weight rows, each read once per call, and the activations) are
// non-temporal (nt): measured 4-5 % faster on the 32B attn_output and 8B ffn_down shapes
// than the default policy.
__device__ __forceinline__ void dma16_nt(const void* base, uint32_t off, gv_lds_u8* lds) {
    asm volatile("s_mov_b32 m0, %0\n\tglobal_load_lds_dwordx4 %1, %2 nt" ::"s"(lds_sgpr((const void*)lds)), "v"(off), "s"(base)
                 : "memory");
}
__device__ __forceinline__ void dma4(const uint8_t* base, uint32_t off, gv_lds_u8* lds) {
    asm volatile("s_mov_b32 m0, %0\n\tglobal_load_lds_dword %1, %2 nt" ::"s"(lds_sgpr((const void*)lds)), "v"(off),
                 "s"(base)
                 : "memory");
}

// One weight row in LDS against the activations (xq, xd; LDS or global): lane l takes
// blocks l, l + 64, ...; returns the wave-summed fp32 dot product (every lane).
template <int KIND>
__device__ __forceinline__ float gemv_row(const unsigned char* wrow, const int8_t* xq, const float* xd, int nblk,
                                          int lane, int first = 0, int step = 64) {
    float acc = 0.0f;
    for (int blk = first + lane; blk < nblk; blk += step) {
        WRaw r;
        load_wraw<KIND>(wrow, blk, r);
        const uint4 xa = *reinterpret_cast<const uint4*>(xq + 32 * blk);
        const uint4 xb = *reinterpret_cast<const uint4*>(xq + 32 * blk + 16);
        const float dx = xd[blk];
        WBlock b;
        decode_wraw<KIND>(r, blk, b);
        const int x[8] = {(int)xa.x, (int)xa.y, (int)xa.z, (int)xa.w, (int)xb.x, (int)xb.y, (int)xb.z, (int)xb.w};
        int dot[2] = {0, 0}, xs[2] = {0, 0};
        float cs[2] = {b.c[0], b.c[1]};
#pragma unroll
        for (int w = 0; w < 8; ++w) {
            const int wv = KIND == kKqQ80 ? (int)r.a[w] : (int)b.u[w];
            dot[w >> 2] = __builtin_amdgcn_sdot4(wv, x[w], dot[w >> 2], false);
            xs[w >> 2] = __builtin_amdgcn_sdot4(0x01010101, x[w], xs[w >> 2], false);
        }
        if (KIND == kKqQ80) cs[0] = cs[1] = 0.0f;
        acc += dx * (b.ws[0] * (float)dot[0] + cs[0] * (float)xs[0] + b.ws[1] * (float)dot[1] + cs[1] * (float)xs[1]);
    }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) acc += __shfl_xor(acc, off, 64);
    return acc;
}

// Copy `span` bytes (a multiple of 4) from src (4-byte aligned) to lds with the nw waves of
// the workgroup: from a 16-byte aligned start, whole 1 KiB pieces by global_load_lds_dwordx4
// (lane l moves bytes 16l..16l+15; wave w takes pieces w, w + nw, ...), the rest (or
// everything, from a start off 16-byte alignment) in 256-byte pieces of global_load_lds_dword,
// lane l moving bytes 4l..4l+3, the tail re-reading the last word. LDS receives up to
// span rounded up to 256 bytes.
__device__ __forceinline__ void copy_span(const void* src, uint32_t span, gv_lds_u8* lds, int wave, int nw, int lane) {
    const uint32_t big = (reinterpret_cast<uintptr_t>(src) & 15) == 0 ? span / 1024 : 0;
    for (uint32_t i = wave; i < big; i += nw) dma16_nt(src, 1024 * i + 16 * lane, lds + 1024 * i);
    const uint32_t rest0 = 1024 * big;
    const uint32_t pieces = (span - rest0 + 255) / 256;
    for (uint32_t i = wave; i < pieces; i += nw)
        dma4(static_cast<const uint8_t*>(src), min(rest0 + 256 * i + 4 * lane, span - 4), lds + rest0 + 256 * i);
}

template <int KIND, int ROWS, bool XL, int WPR>
__global__ __launch_bounds__(64 * ROWS * WPR) void kq_gemv_lds_kernel(KqGemvParams p) {
    extern __shared__ __align__(16) unsigned char rows_lds[];
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int gpm = (p.N + ROWS - 1) / ROWS;  // row groups per matrix
    int g = blockIdx.x;
    const uint8_t* W = p.W;
    uint16_t* y = p.y;
    if (g >= gpm) {
        g -= gpm;
        W = p.W2;
        y = p.y2;
    }
    const int n0 = g * ROWS;
    const int nrows = min(ROWS, p.N - n0);
    // a multiple of 4 bytes: the launcher takes this kernel only when every group's rows are
    const uint32_t span = (uint32_t)(nrows * p.row_bytes);
    const uint8_t* src = W + (size_t)n0 * p.row_bytes;  // 4-byte aligned: W is, n0 is even, row_bytes even
    gv_lds_u8* lds = (gv_lds_u8*)rows_lds;
    constexpr int NW = ROWS * WPR;  // waves; wave w takes row w % ROWS, block slice w / ROWS
    const GemvEpi epi = gemv_epi_load(p, n0 + wave % ROWS);  // (rows past the group: unused)
    copy_span(src, span, lds, wave, NW, lane);
    // XL: the activations (xq: K bytes, 16-byte aligned; xd: K / 8 bytes) after the rows, at
    // xoff = ROWS row_bytes rounded up to 256
    const uint32_t xoff = ((ROWS * (uint32_t)p.row_bytes + 255) / 256) * 256;
    if constexpr (XL) {
        copy_span(p.xq, (uint32_t)p.K, lds + xoff, wave, NW, lane);
        copy_span(p.xd, (uint32_t)p.K / 8, lds + xoff + p.K, wave, NW, lane);
    }
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    const int rw = wave % ROWS, slice = wave / ROWS;
    const int8_t* xq = XL ? reinterpret_cast<const int8_t*>(rows_lds + xoff) : p.xq;
    const float* xd = XL ? reinterpret_cast<const float*>(rows_lds + xoff + p.K) : p.xd;
    float acc = 0.0f;
    if (rw < nrows)
        acc = gemv_row<KIND>(rows_lds + (size_t)rw * p.row_bytes, xq, xd, p.K / 32, lane, 64 * slice, 64 * WPR);
    if constexpr (WPR > 1) {
        // the slices of a row add in slice order (the same for every call); the partial sums
        // sit past the activations
        __shared__ float part[ROWS * WPR];
        if (lane == 0) part[wave] = acc;
        __syncthreads();
        if (slice != 0) return;
        acc = part[rw];
#pragma unroll
        for (int k = 1; k < WPR; ++k) acc += part[rw + k * ROWS];
    }
    if (rw >= nrows) return;
    const int row = n0 + rw;
    if (lane == 0) y[row] = epilogue_pre(acc, p.bias != nullptr, epi.b, p.res != nullptr, epi.r);
}

// quantize_x_q8_kernel semantics (hpc_k_quants.cu:386-400): 32 lanes per 32-value block,
// d = amax / 127 (correctly rounded), inv = d > 0 ? 1 / d : 0, q = clamp(rne(x * inv), +-127)
__global__ __launch_bounds__(256) void quantize_q8_rows_kernel(const uint16_t* __restrict__ x, int K,
                                                               int8_t* __restrict__ xq, float* __restrict__ xd) {
    const size_t row = blockIdx.y;
    const int idx = blockIdx.x * 256 + threadIdx.x;
    const int blk = idx >> 5;
    if (blk * 32 >= K) return;  // whole 32-lane groups leave together
    const float v = half_bits(x[row * K + idx]);
    float amax = fabsf(v);
#pragma unroll
    for (int off = 16; off > 0; off >>= 1) amax = fmaxf(amax, __shfl_xor(amax, off, 32));
    const float d = amax / 127.0f;
    const float inv = d > 0.0f ? 1.0f / d : 0.0f;
    int q = (int)__builtin_rintf(v * inv);
    q = q < -127 ? -127 : (q > 127 ? 127 : q);
    xq[row * K + idx] = (int8_t)q;
    if ((idx & 31) == 0) xd[row * (K / 32) + blk] = d;
}

// xq [n] int8 with xd [n / 32] -> xh [n] fp16, each value exactly as store_x32 forms it
// (fp16(1664 + q) - 1664, times fp16(xd), in packed fp16); 16 values per thread.
__global__ __launch_bounds__(256) void dequant_x_kernel(const int8_t* __restrict__ xq, const float* __restrict__ xd,
                                                        size_t n16, uint16_t* __restrict__ xh) {
    const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= n16) return;
    const uint4 q = reinterpret_cast<const uint4*>(xq)[i];
    const float d = xd[i >> 1];
    const h2v s2 = h2v{(_Float16)d, (_Float16)d};
    const h2v bias = h2v{(_Float16)1664.0f, (_Float16)1664.0f};
    const uint32_t in[4] = {q.x, q.y, q.z, q.w};
    uint32_t o[8];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        const uint32_t u = in[k] ^ 0x80808080u;
        const uint32_t d0 = __builtin_amdgcn_perm(0x66666666u, u, 0x04010400u);
        const uint32_t d1 = __builtin_amdgcn_perm(0x66666666u, u, 0x04030402u);
        o[2 * k] = __builtin_bit_cast(uint32_t, (__builtin_bit_cast(h2v, d0) - bias) * s2);
        o[2 * k + 1] = __builtin_bit_cast(uint32_t, (__builtin_bit_cast(h2v, d1) - bias) * s2);
    }
    uint4* dst = reinterpret_cast<uint4*>(xh) + 2 * i;
    dst[0] = uint4{o[0], o[1], o[2], o[3]};
    dst[1] = uint4{o[4], o[5], o[6], o[7]};
}

template <int WVN, int WVT, int TN, int TT, bool XH>
int launch_kq_shape_x(int kind, const KqGemmParams& p, hipStream_t stream) {
    constexpr int BN = 32 * WVN * TN, BT = 32 * WVT * TT;
    const int nrb = (p.N + BN - 1) / BN, ntb = (p.T + BT - 1) / BT;
    const dim3 grid(((nrb + 7) / 8) * 8 * ntb, p.ksplit), block(64 * WVN * WVT);
    switch (kind) {
        case kKqQ2K: hipLaunchKernelGGL((kq_gemm_kernel<kKqQ2K, WVN, WVT, TN, TT, XH>), grid, block, 0, stream, p); break;
        case kKqQ3K: hipLaunchKernelGGL((kq_gemm_kernel<kKqQ3K, WVN, WVT, TN, TT, XH>), grid, block, 0, stream, p); break;
        case kKqQ4K: hipLaunchKernelGGL((kq_gemm_kernel<kKqQ4K, WVN, WVT, TN, TT, XH>), grid, block, 0, stream, p); break;
        case kKqQ5K: hipLaunchKernelGGL((kq_gemm_kernel<kKqQ5K, WVN, WVT, TN, TT, XH>), grid, block, 0, stream, p); break;
        case kKqQ6K: hipLaunchKernelGGL((kq_gemm_kernel<kKqQ6K, WVN, WVT, TN, TT, XH>), grid, block, 0, stream, p); break;
        case kKqQ80: hipLaunchKernelGGL((kq_gemm_kernel<kKqQ80, WVN, WVT, TN, TT, XH>), grid, block, 0, stream, p); break;
        default: return -2;
    }
    return hipGetLastError() == hipSuccess ? 0 : -1;
}

template <int WVN, int WVT, int TN, int TT>
int launch_kq_shape(int kind, const KqGemmParams& p, hipStream_t stream) {
    if (p.xh) {
        const size_t n16 = (size_t)p.T * p.K / 16;
        hipLaunchKernelGGL(dequant_x_kernel, dim3((unsigned)((n16 + 255) / 256)), dim3(256), 0, stream, p.xq, p.xd, n16,
                           const_cast<uint16_t*>(p.xh));
        if (hipGetLastError() != hipSuccess) return -1;
        return launch_kq_shape_x<WVN, WVT, TN, TT, true>(kind, p, stream);
    }
    return launch_kq_shape_x<WVN, WVT, TN, TT, false>(kind, p, stream);
}

}  // namespace

// Tile shape: 256 x 128 (eight waves, one workgroup per CU) when that alone fills the
// device's CUs (256 on an MI355X), else 128 x 128 (four waves, two per CU) when it gives at least 1.5 workgroups per
// CU, else 64 x 64 (four waves, one tile each) so that small-N / large-K shapes still
// spread over the chip. FRIDAY_GEMM_TILE = 1 / 2 / 3 forces one of them.
// K split for shapes that fill neither tile: 128 x 128 tiles with the split count (2 to 8,
// at least 16 stages of 64 K values each) that best fills the workgroup slots (two per
// CU), the smaller count on ties. FRIDAY_GEMM_KSPLIT = 1 turns it off, n > 1 forces n.
KqPlan kq_gemm_plan(int T, int K, int N) {
    static const int forced = [] {
        const char* e = std::getenv("FRIDAY_GEMM_KSPLIT");
        return e && *e ? std::atoi(e) : 0;
    }();
    const size_t cbytes = (size_t)kKqMaxCounters * kCounterStride * 4;
    const bool xh = (size_t)T * K * 2 < ((size_t)1 << 32);  // the copies use 32-bit offsets
    const size_t xbytes = xh ? (((size_t)T * K * 2 + 255) / 256) * 256 : 0;
    KqPlan r{1, K / kGBK, xh, cbytes, cbytes + xbytes, cbytes + xbytes};
    auto wgs = [&](int bn, int bt) { return (long)((N + bn - 1) / bn) * ((T + bt - 1) / bt); };
    const int nst = K / kGBK;
    const long tiles = wgs(128, 128);
    const long cus = device_cus(), slots = 2 * cus;  // two 128 x 128 workgroups per CU
    int best = 1;
    if (forced > 1) {
        best = forced;
    } else if (forced == 0 && wgs(256, 128) < cus && 2 * tiles < 3 * cus) {
        double fill_best = 0.0;
        for (int sk = 2; sk <= 8 && nst / sk >= 16; ++sk) {
            const long n = tiles * sk;
            const double fill = (double)n / ((double)slots * ((n + slots - 1) / slots));
            if (fill > fill_best + 1e-9) fill_best = fill, best = sk;
        }
    }
    if (best <= 1 || nst < 2) return r;
    const int sps = (nst + best - 1) / best;
    const int ks = (nst + sps - 1) / sps;
    const long gx = ((N + 127) / 128 + 7) / 8 * 8 * ((T + 127) / 128);  // grid x of the 128 x 128 launch
    const size_t pbytes = (size_t)ks * gx * 256 * 64 * 4;               // 256 threads x 64 accumulators
    if (ks <= 1 || gx > kKqMaxCounters || pbytes >= ((size_t)1 << 31)) return r;  // 32-bit buffer offsets
    r.ksplit = ks;
    r.sps = sps;
    r.bytes = r.part_off + pbytes;
    return r;
}

int launch_kq_gemm(int kind, const KqGemmParams& p, hipStream_t stream) {
    static const int forced = [] {
        const char* e = std::getenv("FRIDAY_GEMM_TILE");
        return e && *e ? std::atoi(e) : 0;
    }();
    if (p.ksplit > 1) return launch_kq_shape<2, 2, 2, 2>(kind, p, stream);
    auto wgs = [&](int bn, int bt) { return (long)((p.N + bn - 1) / bn) * ((p.T + bt - 1) / bt); };
    int shape = forced;
    const long cus = device_cus();
    if (shape < 1 || shape > 4) shape = wgs(256, 128) >= cus ? 1 : (2 * wgs(128, 128) >= 3 * cus ? 2 : 3);
    if (shape == 1) return launch_kq_shape<4, 2, 2, 2>(kind, p, stream);
    if (shape == 2) return launch_kq_shape<2, 2, 2, 2>(kind, p, stream);
    if (shape == 4) return launch_kq_shape<2, 4, 2, 1>(kind, p, stream);
    return launch_kq_shape<2, 2, 1, 1>(kind, p, stream);
}

template <int ROWS, bool XL, int WPR = 1>
int launch_gemv_lds(int kind, const KqGemvParams& p, size_t lds, hipStream_t stream) {
    const dim3 grid(((p.N + ROWS - 1) / ROWS) * (p.W2 ? 2 : 1)), block(64 * ROWS * WPR);
    switch (kind) {
        case kKqQ2K: hipLaunchKernelGGL((kq_gemv_lds_kernel<kKqQ2K, ROWS, XL, WPR>), grid, block, lds, stream, p); break;
        case kKqQ3K: hipLaunchKernelGGL((kq_gemv_lds_kernel<kKqQ3K, ROWS, XL, WPR>), grid, block, lds, stream, p); break;
        case kKqQ4K: hipLaunchKernelGGL((kq_gemv_lds_kernel<kKqQ4K, ROWS, XL, WPR>), grid, block, lds, stream, p); break;
        case kKqQ5K: hipLaunchKernelGGL((kq_gemv_lds_kernel<kKqQ5K, ROWS, XL, WPR>), grid, block, lds, stream, p); break;
        case kKqQ6K: hipLaunchKernelGGL((kq_gemv_lds_kernel<kKqQ6K, ROWS, XL, WPR>), grid, block, lds, stream, p); break;
        case kKqQ80: hipLaunchKernelGGL((kq_gemv_lds_kernel<kKqQ80, ROWS, XL, WPR>), grid, block, lds, stream, p); break;
        default: return -2;
    }
    return hipGetLastError() == hipSuccess ? 0 : -1;
}

// The LDS-staged GEMV when its rows (and activations) fit in 64 KiB (two or more workgroups
// per CU) and every row group spans a multiple of 4 bytes, else one wave per row straight
// from memory. FRIDAY_GEMV_LDS = 0 forces the direct kernel; FRIDAY_GEMV_ROWS (2 / 4 / 8),
// FRIDAY_GEMV_XL (0 / 1) and FRIDAY_GEMV_WPR (1 / 2, with 4 rows) override the rows per
// workgroup, the activation staging and the waves per row.
int launch_kq_gemv(int kind, const KqGemvParams& p, hipStream_t stream) {
    static const int env_lds = [] {
        const char* e = std::getenv("FRIDAY_GEMV_LDS");
        return e && *e ? std::atoi(e) : 1;
    }();
    static const int env_rows = [] {
        const char* e = std::getenv("FRIDAY_GEMV_ROWS");
        return e && *e ? std::atoi(e) : 0;
    }();
    static const int env_xl = [] {
        const char* e = std::getenv("FRIDAY_GEMV_XL");
        return e && *e ? std::atoi(e) : -1;
    }();
    static const int env_wpr = [] {
        const char* e = std::getenv("FRIDAY_GEMV_WPR");
        return e && *e ? std::atoi(e) : 0;
    }();
    const int rows = p.W2 ? 2 * p.N : p.N;
    int nr = env_rows == 2 || env_rows == 4 || env_rows == 8 ? env_rows : 4;
    const bool span4 = p.row_bytes % 4 == 0 || p.N % 2 == 0;
    const size_t xbytes = (((size_t)p.K + p.K / 8 + 255) / 256) * 256;
    auto rows_bytes = [&](int r) { return ((r * p.row_bytes + 255) / 256) * 256; };
    while (nr > 2 && rows_bytes(nr) > 65536) nr /= 2;
    // activations in LDS when that keeps the workgroups per CU (160 KiB of LDS, at most 32
    // waves): measured 5 % faster at 32B attn_output, 3 % slower at 8B ffn_down where it
    // would cost a workgroup per CU
    auto per_cu = [&](size_t b) { return std::min<size_t>(32 / nr, 163840 / b); };
    bool xl = per_cu(rows_bytes(nr) + xbytes) >= per_cu(rows_bytes(nr)) && rows_bytes(nr) + xbytes <= 65536;
    if (env_xl >= 0) xl = env_xl != 0;
    const size_t lds = rows_bytes(nr) + (xl ? xbytes : 0);
    if (env_lds != 0 && span4 && lds <= 65536) {
        if (nr == 2) return xl ? launch_gemv_lds<2, true>(kind, p, lds, stream) : launch_gemv_lds<2, false>(kind, p, lds, stream);
        if (nr == 8) return xl ? launch_gemv_lds<8, true>(kind, p, lds, stream) : launch_gemv_lds<8, false>(kind, p, lds, stream);
        // two waves per row (alternate 64-block slices) for long rows: measured 6 % faster at
        // K = 14336 (448 blocks), 6 % slower at K = 5120 (160 blocks, half the lanes idle)
        const int wpr = env_wpr > 0 ? env_wpr : (p.K / 32 >= 384 ? 2 : 1);
        if (wpr == 2)
            return xl ? launch_gemv_lds<4, true, 2>(kind, p, lds, stream) : launch_gemv_lds<4, false, 2>(kind, p, lds, stream);
        return xl ? launch_gemv_lds<4, true>(kind, p, lds, stream) : launch_gemv_lds<4, false>(kind, p, lds, stream);
    }
    const dim3 grid((rows + 3) / 4), block(256);
    switch (kind) {
        case kKqQ2K: hipLaunchKernelGGL(kq_gemv_kernel<kKqQ2K>, grid, block, 0, stream, p); break;
        case kKqQ3K: hipLaunchKernelGGL(kq_gemv_kernel<kKqQ3K>, grid, block, 0, stream, p); break;
        case kKqQ4K: hipLaunchKernelGGL(kq_gemv_kernel<kKqQ4K>, grid, block, 0, stream, p); break;
        case kKqQ5K: hipLaunchKernelGGL(kq_gemv_kernel<kKqQ5K>, grid, block, 0, stream, p); break;
        case kKqQ6K: hipLaunchKernelGGL(kq_gemv_kernel<kKqQ6K>, grid, block, 0, stream, p); break;
        case kKqQ80: hipLaunchKernelGGL(kq_gemv_kernel<kKqQ80>, grid, block, 0, stream, p); break;
        default: return -2;
    }
    return hipGetLastError() == hipSuccess ? 0 : -1;
}

int launch_quantize_q8_rows(const uint16_t* x, int rows, int K, int8_t* xq, float* xd, hipStream_t stream) {
    const dim3 grid((K + 255) / 256, rows);
    hipLaunchKernelGGL(quantize_q8_rows_kernel, grid, dim3(256), 0, stream, x, K, xq, xd);
    return hipGetLastError() == hipSuccess ? 0 : -1;
}

}  // namespace fa
