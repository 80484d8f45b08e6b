// KV append for gfx950: RoPE on q and k at the token's position, rotated k and
// raw v stored into the layer cache (contiguous or paged), and the int8 cache
// variant.
//
// Rotation (cpu_ops.cpp:26-43, cuda_math_kernels.cu:363-404):
//   x0' = x0*c - x1*s, x1' = x0*s + x1*c in fp32, NaN -> 0, clamp +-65504, RNE fp16;
//   neox pairs (i, i + d/2), otherwise (2i, 2i + 1).
// (c, s) come from the host-built table (friday_attn_rope_table_*) and the products
// are not contracted into FMAs, so the stored bits equal the reference CPU path's.
#include "fa_common.hpp"
#include "fa_internal.hpp"

namespace fa {
namespace {

// One thread per (token, head, 16-byte chunk): 128-bit loads and stores of 8 fp16 values.
// Heads [0, Hq) are query heads, [Hq, Hq + Hkv) key heads (their thread also moves the
// matching v chunks). NeoX pairs (i, i + D/2): a thread takes the chunk of elements
// [8c, 8c + 8) and its partner chunk [D/2 + 8c, ...), 8 pairs; interleaved pairs: the
// chunk [8c, 8c + 8), 4 pairs (2i, 2i + 1).
template <bool PAGED>
__global__ __launch_bounds__(256) void fa_rope_store_kernel(RopeParams p) {
    const int t = blockIdx.y;
    const int hd2 = p.D >> 1;
    const int cpp = p.neox ? hd2 / 8 : p.D / 8;  // threads per head
    const int idx = blockIdx.x * 256 + threadIdx.x;
    if (idx >= (p.Hq + p.Hkv) * cpp) return;
    const int h = idx / cpp, c = idx - h * cpp;
    const int kv_dim = p.Hkv * p.D;
    const bool is_k = h >= p.Hq;
    _Float16* x = is_k ? reinterpret_cast<_Float16*>(p.k) + (size_t)t * kv_dim + (h - p.Hq) * p.D
                       : reinterpret_cast<_Float16*>(p.q) + (size_t)t * p.Hq * p.D + h * p.D;
    // element offsets of the chunk (and, NeoX, its partner chunk)
    const int e0 = 8 * c, e1 = p.neox ? hd2 + 8 * c : 8 * c;
    // the loads whose addresses do not depend on the position go out before it is read, so
    // their latency overlaps the position's round trip; they are non-temporal (each value is
    // read once: T = 512 at 40q/8kv d128 measured 5.5 against 6.3 us with the default policy)
    const h8 a = __builtin_nontemporal_load(reinterpret_cast<const h8*>(x + e0));
    const h8 bv = __builtin_nontemporal_load(reinterpret_cast<const h8*>(x + e1));
    const bool store_kv = is_k && p.k_dst;
    const _Float16* vs = reinterpret_cast<const _Float16*>(p.v) + (size_t)t * kv_dim + (h - p.Hq) * p.D;
    h8 v0 = h8{0, 0, 0, 0, 0, 0, 0, 0}, v1 = v0;
    if (store_kv) {
        v0 = __builtin_nontemporal_load(reinterpret_cast<const h8*>(vs + e0));
        if (p.neox) v1 = __builtin_nontemporal_load(reinterpret_cast<const h8*>(vs + e1));
    }
    const int pos = PAGED ? p.seq_lens[t] - 1 : (p.d_pos ? *p.d_pos : p.pos) + t;
    if (pos < 0 || pos >= p.max_ctx) return;
    const float2* cs = reinterpret_cast<const float2*>(p.table) + (size_t)pos * hd2;
    // every table entry of this thread is loaded before any q / k value is touched: with the
    // loads inside the rotation loop the compiler converted the first chunk (waiting for it)
    // before issuing them, so their round trip followed the chunk's instead of overlapping it
    // (NeoX: the 8 entries of elements e0 .. e0 + 7; interleaved: the 4 entries e0/2 ..
    // e0/2 + 3 of its 4 pairs, in ct[0..3], the last two loads repeating the first two)
    float2 ct[8];
    const int c0 = p.neox ? e0 : (e0 >> 1);
#pragma unroll
    for (int j = 0; j < 8; j += 2) {
        const f4 c2 = *reinterpret_cast<const f4*>(cs + c0 + (p.neox ? j : (j & 2)));
        ct[j] = float2{c2[0], c2[1]};
        ct[j + 1] = float2{c2[2], c2[3]};
    }
    // the chunk values are first needed here, after the table loads went out (the memory
    // clobber keeps those loads above this point; the chunk registers stay untouched until it)
    asm volatile("" ::"v"(a), "v"(bv) : "memory");
    h8 ra, rb;
    if (p.neox) {
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            _Float16 r0, r1;
            rope_rotate((float)a[j], (float)bv[j], ct[j].x, ct[j].y, r0, r1);
            ra[j] = r0;
            rb[j] = r1;
        }
    } else {
#pragma unroll
        for (int j = 0; j < 8; j += 2) {
            _Float16 r0, r1;
            rope_rotate((float)a[j], (float)a[j + 1], ct[j >> 1].x, ct[j >> 1].y, r0, r1);
            ra[j] = r0;
            ra[j + 1] = r1;
        }
        rb = ra;
    }
    *reinterpret_cast<h8*>(x + e0) = ra;
    if (p.neox) *reinterpret_cast<h8*>(x + e1) = rb;
    if (store_kv) {
        size_t row;
        if (PAGED) {
            const int phys = p.block_table[(size_t)t * p.bt_stride + (pos >> 4)];
            row = (size_t)phys * kPageTokens + (pos & 15);
        } else {
            row = (size_t)pos;
        }
        const size_t off = row * kv_dim + (size_t)(h - p.Hq) * p.D;
        _Float16* kd = reinterpret_cast<_Float16*>(p.k_dst) + off;
        _Float16* vd = reinterpret_cast<_Float16*>(p.v_dst) + off;
        *reinterpret_cast<h8*>(kd + e0) = ra;
        *reinterpret_cast<h8*>(vd + e0) = v0;
        if (p.neox) {
            *reinterpret_cast<h8*>(kd + e1) = rb;
            *reinterpret_cast<h8*>(vd + e1) = v1;
        }
    }
}

// int8 append (cuda_math_kernels.cu:409-432): 32 lanes per 32-value block,
// K blocks first, then V. dh = fp16(amax / 127); q = clamp(rne(x * (1/dh)), +-127).
__global__ __launch_bounds__(256) void fa_store_kv_q8_kernel(Q8StoreParams p) {
    const int lane = threadIdx.x & 31;
    const int blk = blockIdx.x * 8 + (threadIdx.x >> 5);
    const int nblk = p.kv_dim / 32;
    const int t = blockIdx.y;
    const bool is_v = blk >= nblk;
    const int bb = is_v ? blk - nblk : blk;
    // the value is loaded before the position is read (its address does not depend on it),
    // so the two round trips overlap
    asm volatile("" ::"s"(p.k), "s"(p.v), "s"(p.d_pos), "s"(p.pos));  // one batch of argument loads
    // straight-line: lanes past the last block read block 0 of k (a valid address; unused)
    const bool in_row = blk < 2 * nblk;
    const uint16_t* src = (in_row && is_v ? p.v : p.k) + (size_t)t * p.kv_dim;
    const _Float16 xh = reinterpret_cast<const _Float16*>(src)[(in_row ? bb : 0) * 32 + lane];
    const int pos = (p.d_pos ? *p.d_pos : p.pos) + t;
    const bool active = blk < 2 * nblk && pos >= 0 && pos < p.max_ctx;
    float x = active ? (float)xh : 0.0f;
    if (__builtin_isnan(x)) x = 0.0f;
    float amax = fabsf(x);
#pragma unroll
    for (int off = 16; off > 0; off >>= 1) amax = fmaxf(amax, __shfl_xor(amax, off, 32));
    if (!active) return;
    const _Float16 dh = (_Float16)(amax / 127.0f);
    const float d = (float)dh;
    const float inv = d > 0.0f ? 1.0f / d : 0.0f;
    int q = (int)rintf(x * inv);
    q = max(-127, min(127, q));
    int8_t* dst = (is_v ? p.v_dst : p.k_dst) + (size_t)pos * p.kv_dim;
    dst[bb * 32 + lane] = (int8_t)q;
    if (lane == 0) reinterpret_cast<_Float16*>(is_v ? p.vs_dst : p.ks_dst)[(size_t)pos * nblk + bb] = dh;
}

}  // namespace

int launch_rope_store(const RopeParams& p, bool paged, hipStream_t stream) {
    const int threads = (p.Hq + p.Hkv) * (p.neox ? p.D / 16 : p.D / 8);
    const dim3 grid((threads + 255) / 256, p.T);
    if (paged)
        hipLaunchKernelGGL(fa_rope_store_kernel<true>, grid, dim3(256), 0, stream, p);
    else
        hipLaunchKernelGGL(fa_rope_store_kernel<false>, grid, dim3(256), 0, stream, p);
    return hipGetLastError() == hipSuccess ? 0 : -1;
}

int launch_store_kv_q8(const Q8StoreParams& p, hipStream_t stream) {
    const int nblk2 = 2 * (p.kv_dim / 32);
    const dim3 grid((nblk2 + 7) / 8, p.T);
    hipLaunchKernelGGL(fa_store_kv_q8_kernel, grid, dim3(256), 0, stream, p);
    return hipGetLastError() == hipSuccess ? 0 : -1;
}

}  // namespace fa
