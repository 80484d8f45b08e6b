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
// Data flow of one wave per 32-position tile:
//   HBM --(coalesced 16 B loads, one tile ahead in registers)--> LDS (padded rows)
//   S^T[32 x 16] = K[32 x D] . Q^T[D x 16]     v_mfma_f32_16x16x32_f16, K from LDS
//   online softmax on S^T in registers: every lane owns one query head (l % 16)
//   O^T[D x 16] += V^T[D x 32] . P^T[32 x 16]   P stays in the registers the
//                                               S^T MFMA produced it in; V^T read
//                                               column-wise from LDS
// The four waves of a workgroup take interleaved tiles of the split and are
// merged through LDS; splits are merged by fa_merge_kernel (log-sum-exp).
#include "fa_common.hpp"
#include "fa_internal.hpp"

namespace fa {
namespace {

constexpr int kWaves = 4;
constexpr int kThreads = kWaves * 64;
constexpr int kTile = 32;

template <int D, bool Q8>
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
    static constexpr int COMB_LDS = kWaves * 16 * (D + 2) * 4;
    static constexpr int LDS = (kWaves * WAVE_LDS > COMB_LDS ? kWaves * WAVE_LDS : COMB_LDS);
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

// Dequantize 16 int8 values with one fp16 scale into two 16-byte fp16 chunks.
__device__ __forceinline__ void dequant16(u4 raw, float sc, u4& lo, u4& hi) {
    const int8_t* c = reinterpret_cast<const int8_t*>(&raw);
    h8 a, b;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        a[j] = (_Float16)((float)c[j] * sc);
        b[j] = (_Float16)((float)c[8 + j] * sc);
    }
    lo = *reinterpret_cast<u4*>(&a);
    hi = *reinterpret_cast<u4*>(&b);
}

template <int D, bool PAGED, bool Q8>
__global__ __launch_bounds__(kThreads) void fa_decode_kernel(DecodeParams p) {
    using Gm = Geo<D, Q8>;
    __shared__ __align__(16) unsigned char smem[Gm::LDS];

    const int split = blockIdx.x;
    const int kvh = blockIdx.y / p.ngb, gb = blockIdx.y % p.ngb;
    const int b = blockIdx.z;
    const int S = context_len(p, b, PAGED);
    const int chunk = p.single ? (S > 0 ? ((S + kSpan - 1) / kSpan) * kSpan : kSpan) : split_chunk(S);
    const int nsp = p.single ? 1 : split_count(S);
    if (split >= nsp) return;  // inactive split; the merge ignores it
    const int start = split * chunk;
    const int end = min(S, start + chunk);  // positions [start, end)

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int col = lane & 15, kb = lane >> 4;
    const int g = gb * 16 + col;
    const bool gvalid = g < p.G;
    const int head = kvh * p.G + g;

    // Q^T as the B operand of S^T = K Q^T: lane (col = head, kb) holds q[d = s*32 + kb*8 .. +8].
    h8 qf[Gm::KSTEPS];
    {
        const uint16_t* qrow = p.q + ((size_t)b * p.Hq + (gvalid ? head : 0)) * D;
#pragma unroll
        for (int s = 0; s < Gm::KSTEPS; ++s) {
            u4 raw = gvalid ? *reinterpret_cast<const u4*>(qrow + s * 32 + kb * 8) : u4{0, 0, 0, 0};
            qf[s] = *reinterpret_cast<h8*>(&raw);
        }
    }

    unsigned char* kl = smem + wave * Gm::WAVE_LDS;
    unsigned char* vl = kl + kTile * Gm::LROW;
    const char* kbase = static_cast<const char*>(p.k) + (size_t)kvh * (Q8 ? D : D * 2);
    const char* vbase = static_cast<const char*>(p.v) + (size_t)kvh * (Q8 ? D : D * 2);
    const size_t rowb = (size_t)p.kv_dim * (Q8 ? 1 : 2);

    float m_run = kNegBig, l_run = 0.0f;
    f4 o[Gm::DTILES];
#pragma unroll
    for (int i = 0; i < Gm::DTILES; ++i) o[i] = f4{0.f, 0.f, 0.f, 0.f};

    const int ntiles = (end - start + kTile - 1) / kTile;
    u4 kr[Gm::NLD], vr[Gm::NLD];
    float ksc[Gm::NLD], vsc[Gm::NLD];
    const int lrow = lane / Gm::CPR, lchunk = lane % Gm::CPR;

    auto load_tile = [&](int t) {
        const int base = start + t * kTile;
#pragma unroll
        for (int r = 0; r < Gm::NLD; ++r) {
            const int pos = base + r * Gm::RPI + lrow;
            if (pos < end) {
                const size_t ri = row_index<PAGED>(p, b, pos);
                kr[r] = ld_nt(reinterpret_cast<const u4*>(kbase + ri * rowb) + lchunk);
                vr[r] = ld_nt(reinterpret_cast<const u4*>(vbase + ri * rowb) + lchunk);
                if (Q8) {
                    const size_t si = (ri * p.kv_dim + (size_t)kvh * D + lchunk * 16) / 32;
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

    int t = wave;
    if (t < ntiles) load_tile(t);
    for (; t < ntiles; t += kWaves) {
        // registers -> wave-private LDS tile
#pragma unroll
        for (int r = 0; r < Gm::NLD; ++r) {
            const int row = r * Gm::RPI + lrow;
            if (Q8) {
                u4 lo, hi;
                dequant16(kr[r], ksc[r], lo, hi);
                *reinterpret_cast<u4*>(kl + row * Gm::LROW + lchunk * 32) = lo;
                *reinterpret_cast<u4*>(kl + row * Gm::LROW + lchunk * 32 + 16) = hi;
                dequant16(vr[r], vsc[r], lo, hi);
                *reinterpret_cast<u4*>(vl + row * Gm::LROW + lchunk * 32) = lo;
                *reinterpret_cast<u4*>(vl + row * Gm::LROW + lchunk * 32 + 16) = hi;
            } else {
                *reinterpret_cast<u4*>(kl + row * Gm::LROW + lchunk * 16) = kr[r];
                *reinterpret_cast<u4*>(vl + row * Gm::LROW + lchunk * 16) = vr[r];
            }
        }
        // LDS operations of one wave complete in order: the reads below see these writes.
        __builtin_amdgcn_wave_barrier();
        if (t + kWaves < ntiles) load_tile(t + kWaves);  // next tile in flight during the math

        // S^T = K Q^T over two 16-row m-tiles
        f4 sacc[2] = {f4{0.f, 0.f, 0.f, 0.f}, f4{0.f, 0.f, 0.f, 0.f}};
#pragma unroll
        for (int mt = 0; mt < 2; ++mt) {
#pragma unroll
            for (int s = 0; s < Gm::KSTEPS; ++s) {
                const h8 a = *reinterpret_cast<const h8*>(kl + (mt * 16 + col) * Gm::LROW + (s * 32 + kb * 8) * 2);
                sacc[mt] = mfma16x16x32(a, qf[s], sacc[mt]);
            }
        }

        // online softmax (log2 domain); lane column = query head, rows = positions
        const int tbase = start + t * kTile;
        float sc[8];
        float mx = kNegBig;
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const int mt = j >> 2, i = j & 3;
            float x = sacc[mt][i] * p.scale2;
            if (__builtin_isnan(x)) x = kNegBig;
            const bool valid = tbase + mt * 16 + kb * 4 + i < end;
            sc[j] = valid ? x : -__builtin_inff();
            mx = fmaxf(mx, sc[j]);
        }
        mx = wave_max_xor(mx, 16);
        mx = wave_max_xor(mx, 32);
        const float m_new = fmaxf(m_run, mx);
        const float da = m_run - m_new;
        const float alpha = da < kCut2 ? 0.0f : exp2_fast(da);
        h8 pf;
        float psum = 0.0f;
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const float df = sc[j] - m_new;  // -inf for masked rows
            const float e = df < kCut2 ? 0.0f : exp2_fast(df);
            const _Float16 eh = (_Float16)e;
            pf[j] = eh;
            psum += (float)eh;
        }
        l_run = l_run * alpha + psum;
        m_run = m_new;

        // O^T += V^T P^T; k index j of lane block kb <-> tile row (j<4 ? kb*4+j : 16+kb*4+j-4)
#pragma unroll
        for (int dt = 0; dt < Gm::DTILES; ++dt) {
            h8 va;
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                const int row = (j < 4) ? (kb * 4 + j) : (16 + kb * 4 + (j - 4));
                va[j] = *reinterpret_cast<const _Float16*>(vl + row * Gm::LROW + (dt * 16 + col) * 2);
            }
            o[dt] = mfma16x16x32(va, pf, o[dt] * alpha);
        }
        __builtin_amdgcn_wave_barrier();
    }

    // ---- combine the four waves of the workgroup through LDS ----
    l_run = wave_sum_xor(l_run, 16);
    l_run = wave_sum_xor(l_run, 32);
    __syncthreads();  // all waves done with their tiles; LDS is reused
    float* cm = reinterpret_cast<float*>(smem);           // [kWaves][16]
    float* cl = cm + kWaves * 16;                          // [kWaves][16]
    float* co = cl + kWaves * 16;                          // [kWaves][16][D]
    if (kb == 0) {
        cm[wave * 16 + col] = m_run;
        cl[wave * 16 + col] = l_run;
    }
#pragma unroll
    for (int dt = 0; dt < Gm::DTILES; ++dt)
#pragma unroll
        for (int i = 0; i < 4; ++i) co[(wave * 16 + col) * D + dt * 16 + kb * 4 + i] = o[dt][i];
    __syncthreads();

    const int gcount = min(16, p.G - gb * 16);
    for (int idx = tid; idx < gcount * D; idx += kThreads) {
        const int gg = idx / D, d = idx % D;
        float M = cm[gg];
#pragma unroll
        for (int w = 1; w < kWaves; ++w) M = fmaxf(M, cm[w * 16 + gg]);
        float L = 0.0f, O = 0.0f;
#pragma unroll
        for (int w = 0; w < kWaves; ++w) {
            const float df = cm[w * 16 + gg] - M;
            const float wt = df < kCut2 ? 0.0f : exp2_fast(df);
            L += wt * cl[w * 16 + gg];
            O += wt * co[(w * 16 + gg) * D + d];
        }
        const int hh = kvh * p.G + gb * 16 + gg;
        const size_t row = (size_t)b * p.Hq + hh;
        if (nsp == 1) {
            const float r = L > 1e-12f ? O / L : 0.0f;
            reinterpret_cast<_Float16*>(p.out)[row * D + d] = out_half(r);
        } else {
            const size_t slot = row * p.nsplit_grid + split;
            p.part_o[slot * D + d] = O;
            if (d == 0) {
                p.part_ml[slot * 2] = M;
                p.part_ml[slot * 2 + 1] = L;
            }
        }
    }
}

// Log-sum-exp merge of the split partials of one query head (one workgroup per
// (sequence, head)): M = max m_s, w_s = exp(m_s - M) (0 below -50),
// out = sum w_s o_s / sum w_s l_s  (attention_kernels.cu:207-235).
template <int D, bool PAGED>
__global__ __launch_bounds__(kThreads) void fa_merge_kernel(DecodeParams p) {
    constexpr int NP = kThreads / D;  // split partitions summed per output element
    __shared__ float s_w[kNsplitCap];
    __shared__ float s_red[kWaves];
    __shared__ float s_acc[NP][D];
    const int row = blockIdx.x;       // b * Hq + head
    const int b = row / p.Hq;
    const int S = context_len(p, b, PAGED);
    const int nsp = split_count(S);
    if (p.single || nsp <= 1) return;  // the decode kernel wrote the output
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const float* ml = p.part_ml + (size_t)row * p.nsplit_grid * 2;
    const float* po = p.part_o + (size_t)row * p.nsplit_grid * D;

    float m = kNegBig;
    for (int s = tid; s < nsp; s += kThreads) m = fmaxf(m, ml[2 * s]);
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) m = wave_max_xor(m, off);
    if (lane == 0) s_red[wave] = m;
    __syncthreads();
    float M = s_red[0];
#pragma unroll
    for (int w = 1; w < kWaves; ++w) M = fmaxf(M, s_red[w]);
    __syncthreads();
    float l = 0.0f;
    for (int s = tid; s < nsp; s += kThreads) {
        const float df = ml[2 * s] - M;
        const float w = df < kCut2 ? 0.0f : exp2_fast(df);
        s_w[s] = w;
        l += w * ml[2 * s + 1];
    }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) l = wave_sum_xor(l, off);
    if (lane == 0) s_red[wave] = l;
    __syncthreads();
    float L = 0.0f;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) L += s_red[w];

    const int d = tid % D, part = tid / D;
    float acc = 0.0f;
    for (int s = part; s < nsp; s += NP) acc += s_w[s] * po[(size_t)s * D + d];
    s_acc[part][d] = acc;
    __syncthreads();
    if (part == 0) {
        float a = 0.0f;
#pragma unroll
        for (int q = 0; q < NP; ++q) a += s_acc[q][d];
        const float r = L > 1e-12f ? a / L : 0.0f;
        reinterpret_cast<_Float16*>(p.out)[(size_t)row * D + d] = out_half(r);
    }
}

template <int D, bool PAGED, bool Q8>
int launch_t(const DecodeParams& p, int batch, hipStream_t stream) {
    const dim3 grid(p.single ? 1 : p.nsplit_grid, p.Hkv * p.ngb, batch);
    hipLaunchKernelGGL((fa_decode_kernel<D, PAGED, Q8>), grid, dim3(kThreads), 0, stream, p);
    if (hipGetLastError() != hipSuccess) return -1;
    if (!p.single) {
        hipLaunchKernelGGL((fa_merge_kernel<D, PAGED>), dim3(batch * p.Hq), dim3(kThreads), 0, stream, p);
        if (hipGetLastError() != hipSuccess) return -1;
    }
    return 0;
}

}  // namespace

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
