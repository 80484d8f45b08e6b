// Prefill projection GEMM on gfx950: Y[t][n] = sum_k W[n][k] x_t[k] for T tokens, W in a
// GGUF K-quant / Q8_0 row layout, x in the int8 activation format of the decode GEMV
// (int8 per value, one fp32 scale per 32 values), plus the activation quantiser that
// makes that format. The reference computes per-32-value integer dot products on int8
// tensor cores and scales each in fp32 (prefill_kernels.cu:173-327); on CDNA that
// per-block scaling is vector work six times the matrix work, so here both operands are
// decoded once per workgroup into fp16 tiles in LDS (each value rounded once from its
// exact fp32 form) and a single fp16 MFMA chain with fp32 accumulation runs over K.
//
// Tiling: a workgroup of 256 threads owns 128 weight rows x 128 tokens; its four waves
// each own 64 x 64 (2 x 2 tiles of v_mfma_f32_32x32x16_f16). K advances in stages of 64
// values through two LDS buffers: while the MFMAs consume one, the raw bytes of the next
// stage are in flight in registers, then decoded into the other buffer.
#include <hip/hip_runtime.h>

#include <cstdint>

#include "fa_common.hpp"
#include "fa_internal.hpp"

namespace fa {
namespace {

constexpr int kGBN = 128;  // weight rows per workgroup
constexpr int kGBT = 128;  // tokens per workgroup
constexpr int kGBK = 64;   // K values per stage (two 32-value blocks)
constexpr int kGThreads = 256;
constexpr int kGRowB = kGBK * 2;  // bytes of one fp16 tile row in LDS

typedef _Float16 h8v __attribute__((ext_vector_type(8)));
typedef float f16v __attribute__((ext_vector_type(16)));

__device__ __forceinline__ float half_bits(uint32_t h) {
    return (float)__builtin_bit_cast(_Float16, (uint16_t)h);
}
__device__ __forceinline__ uint32_t ld32(const uint8_t* p) { return *reinterpret_cast<const uint32_t*>(p); }
// 4 bytes from a 2-byte aligned address (Q3_K, Q6_K and Q8_0 blocks are 2-byte aligned)
__device__ __forceinline__ uint32_t ld16x2(const uint8_t* p) {
    const uint16_t* q = reinterpret_cast<const uint16_t*>(p);
    return (uint32_t)q[0] | ((uint32_t)q[1] << 16);
}
__device__ __forceinline__ uint32_t ld16(const uint8_t* p) { return *reinterpret_cast<const uint16_t*>(p); }

// One 32-value block of a weight row: byte l of u (unsigned) maps to ws[l/16] * byte + c[l/16].
// Offsets of the signed kinds are folded into c (c = -off * ws, exact: off is a power of 2),
// the mins of Q2_K / Q4_K / Q5_K are c = -min.
struct WBlock {
    uint32_t u[8];
    float ws[2], c[2];
};

// get_scale_min_k4: 6-bit scale and min of block j (0..7) of a Q4_K / Q5_K superblock
__device__ __forceinline__ void scale_min_k4(int j, uint32_t s0, uint32_t s1, uint32_t s2, int& sc, int& m) {
    const uint32_t s[3] = {s0, s1, s2};
    auto byte = [&](int i) { return (int)((s[i >> 2] >> (8 * (i & 3))) & 0xFF); };
    if (j < 4) {
        sc = byte(j) & 63;
        m = byte(j + 4) & 63;
    } else {
        sc = (byte(j + 4) & 0xF) | ((byte(j - 4) >> 6) << 4);
        m = (byte(j + 4) >> 4) | ((byte(j) >> 6) << 4);
    }
}

// Raw loads and decode of block `blk` (0..K/32-1) of one weight row, per GGML layout:
//   Q2_K  scales[16] qs[64] d dmin              84 B / 256, q = 2 bits, per-16 4-bit scale & min
//   Q3_K  hmask[32] qs[64] scales[12] d         110 B, q = 2 bits + hmask bit - 4, per-16 6-bit scale - 32
//   Q4_K  d dmin scales[12] qs[128]             144 B, q = nibble, per-32 6-bit scale & min
//   Q5_K  d dmin scales[12] qh[32] qs[128]      176 B, q = nibble + qh bit << 4
//   Q6_K  ql[128] qh[64] scales[16] d           210 B, q = nibble + 2 bits << 4 - 32, per-16 int8 scale
//   Q8_0  d qs[32]                              34 B / 32, q = int8
// (dequant32, prefill_kernels.cu:57-144; dequantizeRow, cpu_kquants.cpp:227-280)
template <int KIND>
__device__ __forceinline__ void load_wblock(const uint8_t* row, int blk, WBlock& o) {
    const int sb = blk >> 3, j = blk & 7;
    if constexpr (KIND == kKqQ2K) {
        const uint8_t* b = row + (size_t)sb * 84;
        const int h = j >> 2, s = j & 3;
#pragma unroll
        for (int w = 0; w < 8; ++w) o.u[w] = (ld32(b + 16 + 32 * h + 4 * w) >> (2 * s)) & 0x03030303u;
        const uint32_t scw = ld32(b + 8 * h + 4 * (s >> 1)) >> (16 * (s & 1));
        const uint32_t dd = ld32(b + 80);
        const float d = half_bits(dd & 0xFFFF), dmin = half_bits(dd >> 16);
#pragma unroll
        for (int c = 0; c < 2; ++c) {
            const int sc = (scw >> (8 * c)) & 0xFF;
            o.ws[c] = d * (float)(sc & 0xF);
            o.c[c] = -(dmin * (float)(sc >> 4));
        }
    } else if constexpr (KIND == kKqQ3K) {
        const uint8_t* b = row + (size_t)sb * 110;
        const int h = j >> 2, s = j & 3;
#pragma unroll
        for (int w = 0; w < 8; ++w) {
            const uint32_t lo = (ld16x2(b + 32 + 32 * h + 4 * w) >> (2 * s)) & 0x03030303u;
            const uint32_t hb = (ld16x2(b + 4 * w) >> (4 * h + s)) & 0x01010101u;
            o.u[w] = lo | (hb << 2);  // q + 4, 0..7
        }
        const uint32_t s0 = ld16x2(b + 96), s1 = ld16x2(b + 100), s2 = ld16x2(b + 104);
        const uint32_t sw[3] = {s0, s1, s2};
        auto byte = [&](int i) { return (int)((sw[i >> 2] >> (8 * (i & 3))) & 0xFF); };
        const float d = half_bits(ld16(b + 108));
#pragma unroll
        for (int c = 0; c < 2; ++c) {
            const int g = 8 * h + 2 * s + c;
            const int lo = g < 8 ? (byte(g) & 0xF) : (byte(g - 8) >> 4);
            const int hi = (byte(8 + (g & 3)) >> (2 * (g >> 2))) & 3;
            o.ws[c] = d * (float)((lo | (hi << 4)) - 32);
            o.c[c] = -4.0f * o.ws[c];
        }
    } else if constexpr (KIND == kKqQ4K || KIND == kKqQ5K) {
        constexpr bool Q5 = KIND == kKqQ5K;
        const uint8_t* b = row + (size_t)sb * (Q5 ? 176 : 144);
        const int jj = j >> 1, hi = j & 1;
        const uint8_t* qs = b + (Q5 ? 48 : 16) + 32 * jj;
#pragma unroll
        for (int w = 0; w < 8; ++w) {
            uint32_t v = (ld32(qs + 4 * w) >> (4 * hi)) & 0x0F0F0F0Fu;
            if constexpr (Q5) v |= ((ld32(b + 16 + 4 * w) >> j) & 0x01010101u) << 4;
            o.u[w] = v;
        }
        int sc, m;
        scale_min_k4(j, ld32(b + 4), ld32(b + 8), ld32(b + 12), sc, m);
        const uint32_t dd = ld32(b);
        o.ws[0] = o.ws[1] = half_bits(dd & 0xFFFF) * (float)sc;
        o.c[0] = o.c[1] = -(half_bits(dd >> 16) * (float)m);
    } else if constexpr (KIND == kKqQ6K) {
        const uint8_t* b = row + (size_t)sb * 210;
        const int h = j >> 2, p = j & 3;
#pragma unroll
        for (int w = 0; w < 8; ++w) {
            const uint32_t ql = ld16x2(b + 64 * h + 32 * (p & 1) + 4 * w);
            const uint32_t lo = (p < 2 ? ql : ql >> 4) & 0x0F0F0F0Fu;
            const uint32_t hb = (ld16x2(b + 128 + 32 * h + 4 * w) >> (2 * p)) & 0x03030303u;
            o.u[w] = lo | (hb << 4);  // q + 32, 0..63
        }
        const uint32_t scp = ld16(b + 192 + 8 * h + 2 * p);
        const float d = half_bits(ld16(b + 208));
#pragma unroll
        for (int c = 0; c < 2; ++c) {
            o.ws[c] = d * (float)(int8_t)((scp >> (8 * c)) & 0xFF);
            o.c[c] = -32.0f * o.ws[c];
        }
    } else {  // Q8_0
        const uint8_t* b = row + (size_t)blk * 34;
#pragma unroll
        for (int w = 0; w < 8; ++w) o.u[w] = ld16x2(b + 2 + 4 * w) ^ 0x80808080u;  // q + 128
        o.ws[0] = o.ws[1] = half_bits(ld16(b));
        o.c[0] = o.c[1] = -128.0f * o.ws[0];
    }
}

// byte i of w as a float (v_cvt_f32_ubyte{0..3})
__device__ __forceinline__ float ubyte(uint32_t w, int i) { return (float)((w >> (8 * i)) & 0xFF); }

// 32 decoded values -> 64 bytes of row r of an fp16 tile at chunks 4*half .. 4*half+3,
// each 16-byte chunk c stored at slot c ^ (r & 7) (conflict-free 16-byte MFMA operand reads)
__device__ __forceinline__ void store_tile32(unsigned char* tile, int r, int half, const uint32_t (&u)[8],
                                             const float (&ws)[2], const float (&c)[2]) {
#pragma unroll
    for (int ch = 0; ch < 4; ++ch) {
        h8v v;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            const int l = 8 * ch + e;  // value index in the block
            v[e] = (_Float16)__builtin_fmaf(ws[l >> 4], ubyte(u[l >> 2], l & 3), c[l >> 4]);
        }
        const int slot = (4 * half + ch) ^ (r & 7);
        *reinterpret_cast<h8v*>(tile + r * kGRowB + slot * 16) = v;
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

template <int KIND>
__global__ __launch_bounds__(kGThreads, 2) void kq_gemm_kernel(KqGemmParams p) {
    __shared__ __align__(16) unsigned char sw0[kGBN * kGRowB];
    __shared__ __align__(16) unsigned char sw1[kGBN * kGRowB];
    __shared__ __align__(16) unsigned char sx0[kGBT * kGRowB];
    __shared__ __align__(16) unsigned char sx1[kGBT * kGRowB];

    // workgroup -> (row block, token block): the token blocks of one row block get ids
    // that are equal mod 8, so with round-robin placement over the 8 XCDs they share an
    // XCD and its L2 copy of the weight rows
    const int nrb = (p.N + kGBN - 1) / kGBN, ntb = (p.T + kGBT - 1) / kGBT;
    const int id = blockIdx.x;
    const int rb = (id % 8) + 8 * (id / (8 * ntb));
    const int tb = (id / 8) % ntb;
    if (rb >= nrb) return;  // padding of the last group of 8 row blocks
    const int n0 = rb * kGBN, t0 = tb * kGBT;

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wn = wave & 1, wt = wave >> 1;

    // staging role: weight row n0 + lr, block half lh of the stage; token t0 + lr, half lh
    const int lr = tid >> 1, lh = tid & 1;
    const size_t row_bytes = p.row_bytes;
    const bool w_ok = n0 + lr < p.N;
    const bool x_ok = t0 + lr < p.T;
    const uint8_t* wrow = p.W + (size_t)(w_ok ? n0 + lr : 0) * row_bytes;
    const int8_t* xrow = p.xq + (size_t)(x_ok ? t0 + lr : 0) * p.K;
    const float* xdrow = p.xd + (size_t)(x_ok ? t0 + lr : 0) * (p.K / 32);

    WBlock wb;
    uint4 xa, xb;
    float xs;
    auto load_stage = [&](int k0) __attribute__((always_inline)) {
        const int blk = k0 / 32 + lh;
        load_wblock<KIND>(wrow, blk, wb);
        xa = *reinterpret_cast<const uint4*>(xrow + 32 * blk);
        xb = *reinterpret_cast<const uint4*>(xrow + 32 * blk + 16);
        xs = xdrow[blk];
    };
    auto store_stage = [&](unsigned char* sw, unsigned char* sx) __attribute__((always_inline)) {
        if (!w_ok) {
            wb.ws[0] = wb.ws[1] = wb.c[0] = wb.c[1] = 0.0f;
        }
        store_tile32(sw, lr, lh, wb.u, wb.ws, wb.c);
        // activations: q = byte ^ 0x80 - 128, value = fp16(xd * q) from fma(xd, q + 128, -128 xd)
        const uint32_t xu[8] = {xa.x ^ 0x80808080u, xa.y ^ 0x80808080u, xa.z ^ 0x80808080u, xa.w ^ 0x80808080u,
                                xb.x ^ 0x80808080u, xb.y ^ 0x80808080u, xb.z ^ 0x80808080u, xb.w ^ 0x80808080u};
        const float s = x_ok ? xs : 0.0f;
        const float xsv[2] = {s, s}, xc[2] = {-128.0f * s, -128.0f * s};
        store_tile32(sx, lr, lh, xu, xsv, xc);
    };

    f16v acc[2][2];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;

    auto compute = [&](const unsigned char* sw, const unsigned char* sx) __attribute__((always_inline)) {
#pragma unroll
        for (int kk = 0; kk < kGBK / 16; ++kk) {
            const int ch = 2 * kk + (lane >> 5);  // this lane's 8 K values of the 16
            h8v a[2], b[2];
#pragma unroll
            for (int i = 0; i < 2; ++i) {
                const int r = wn * 64 + 32 * i + (lane & 31);
                a[i] = *reinterpret_cast<const h8v*>(sw + r * kGRowB + ((ch ^ (r & 7)) * 16));
            }
#pragma unroll
            for (int j = 0; j < 2; ++j) {
                const int r = wt * 64 + 32 * j + (lane & 31);
                b[j] = *reinterpret_cast<const h8v*>(sx + r * kGRowB + ((ch ^ (r & 7)) * 16));
            }
#pragma unroll
            for (int i = 0; i < 2; ++i)
#pragma unroll
                for (int j = 0; j < 2; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a[i], b[j], acc[i][j], 0, 0, 0);
        }
    };

    const int nst = p.K / kGBK;
    load_stage(0);
    store_stage(sw0, sx0);
    __syncthreads();
    for (int st = 0; st < nst; st += 2) {
        if (st + 1 < nst) load_stage((st + 1) * kGBK);
        compute(sw0, sx0);
        if (st + 1 < nst) store_stage(sw1, sx1);
        __syncthreads();
        if (st + 1 >= nst) break;
        if (st + 2 < nst) load_stage((st + 2) * kGBK);
        compute(sw1, sx1);
        if (st + 2 < nst) store_stage(sw0, sx0);
        __syncthreads();
    }

    // acc[i][j][r]: weight row n0 + wn*64 + 32i + 8(r/4) + 4(lane/32) + r%4,
    // token t0 + wt*64 + 32j + lane%32
#pragma unroll
    for (int j = 0; j < 2; ++j) {
        const int t = t0 + wt * 64 + 32 * j + (lane & 31);
        if (t >= p.T) continue;
        uint16_t* yrow = p.Y + (size_t)t * p.ldy;
        const uint16_t* rrow = p.res ? p.res + (size_t)t * p.ldy : nullptr;
#pragma unroll
        for (int i = 0; i < 2; ++i)
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int n = n0 + wn * 64 + 32 * i + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
                if (n < p.N) yrow[n] = epilogue(acc[i][j][r], p.bias, rrow, n);
            }
    }
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

}  // namespace

int launch_kq_gemm(int kind, const KqGemmParams& p, hipStream_t stream) {
    const int nrb = (p.N + kGBN - 1) / kGBN, ntb = (p.T + kGBT - 1) / kGBT;
    const dim3 grid(((nrb + 7) / 8) * 8 * ntb);
    switch (kind) {
        case kKqQ2K: hipLaunchKernelGGL(kq_gemm_kernel<kKqQ2K>, grid, dim3(kGThreads), 0, stream, p); break;
        case kKqQ3K: hipLaunchKernelGGL(kq_gemm_kernel<kKqQ3K>, grid, dim3(kGThreads), 0, stream, p); break;
        case kKqQ4K: hipLaunchKernelGGL(kq_gemm_kernel<kKqQ4K>, grid, dim3(kGThreads), 0, stream, p); break;
        case kKqQ5K: hipLaunchKernelGGL(kq_gemm_kernel<kKqQ5K>, grid, dim3(kGThreads), 0, stream, p); break;
        case kKqQ6K: hipLaunchKernelGGL(kq_gemm_kernel<kKqQ6K>, grid, dim3(kGThreads), 0, stream, p); break;
        case kKqQ80: hipLaunchKernelGGL(kq_gemm_kernel<kKqQ80>, grid, dim3(kGThreads), 0, stream, p); break;
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
