// Causal chunked-prefill attention on gfx950 MFMA.
//
// Semantics: launchPrefillAttention (attention_kernels.h:36-50, .cu:513-684):
// query t of the chunk sits at position p0 + t (p0 = *d_pos0) and attends to
// cache positions [0, p0 + t]; NaN score -> -1e30, exp cut off below -50 from
// the running max, fp32 accumulation, output NaN -> 0, clamp, RNE fp16. Row t
// equals decode attention with S = p0 + t + 1 up to the order of fp32 additions.
//
// Work decomposition: rows r = t * G + g of one kv head (all query heads of the
// GQA group for every token share its K/V). A workgroup owns 128 rows (4 waves
// x 32) and streams the kv head's K/V in 32-position tiles through LDS, shared
// by the four waves:
//   K tile row-major            -> A operand of S^T = K Q^T   (ds_read_b128)
//   V tile transposed, with the positions of one lane block stored together
//                               -> A operand of O^T += V^T P^T (ds_read_b128)
// Each wave keeps Q^T, O^T and the softmax state of its 32 rows in registers;
// every K/V fragment read from LDS feeds two MFMAs (two 16-row tiles).
#include "fa_common.hpp"
#include "fa_internal.hpp"

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

template <int D, bool Q8>
int launch_pf(const PrefillParams& p, hipStream_t stream) {
    const int R = p.T * p.G;
    const dim3 grid((R + kPfRowsWG - 1) / kPfRowsWG, p.Hkv);
    hipLaunchKernelGGL((fa_prefill_kernel<D, Q8>), grid, dim3(kPfThreads), 0, stream, p);
    return hipGetLastError() == hipSuccess ? 0 : -1;
}

}  // namespace

int launch_prefill(const PrefillParams& p, int head_dim, bool q8, hipStream_t stream) {
    if (head_dim == 128) return q8 ? launch_pf<128, true>(p, stream) : launch_pf<128, false>(p, stream);
    if (head_dim == 64) return q8 ? launch_pf<64, true>(p, stream) : launch_pf<64, false>(p, stream);
    return -2;
}

}  // namespace fa
