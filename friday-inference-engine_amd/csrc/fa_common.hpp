// Shared device helpers for the gfx950 KV-cache kernels: fp16 vector types,
// the 16x16x32 f16 MFMA wrapper and wave64 reductions.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace fa {

typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef _Float16 h4 __attribute__((ext_vector_type(4)));
typedef _Float16 h2 __attribute__((ext_vector_type(2)));
typedef float f4 __attribute__((ext_vector_type(4)));
typedef uint32_t u4 __attribute__((ext_vector_type(4)));

constexpr float kLog2e = 1.4426950408889634f;
// exp cut-off of the reference (diff < -50 -> weight 0), in log2 units.
constexpr float kCut2 = -50.0f * kLog2e;
constexpr float kNegBig = -1e30f;  // score of a NaN dot product (attention_kernels.cu:69)

// D = A(16x32) * B(32x16) + C on gfx950. Lane l holds row/column l%16 of A/B
// and 8 consecutive k values of block l/16; C/D: column l%16, rows 4*(l/16)+i.
__device__ __forceinline__ f4 mfma16x16x32(h8 a, h8 b, f4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}

// D = A(16x16) * B(16x16) + C: lane l holds row/column l%16 of A/B and 4
// consecutive k values of block l/16; C/D as above.
__device__ __forceinline__ f4 mfma16x16x16(h4 a, h4 b, f4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x16f16(a, b, c, 0, 0, 0);
}

// bf16 operands travel in the same 16-bit registers as fp16 ones (h8 holds the raw
// bits); mma16<true> hands them to the bf16 MFMA (8 bits of significand, fp32 range),
// mma16<false> to the fp16 one. Both accumulate in fp32.
typedef __bf16 b8 __attribute__((ext_vector_type(8)));
template <bool BF>
__device__ __forceinline__ f4 mma16(h8 a, h8 b, f4 c) {
    if constexpr (BF)
        return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(b8, a), __builtin_bit_cast(b8, b), c, 0, 0, 0);
    else
        return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}

// float -> the 16-bit operand type, round to nearest even (bits in a _Float16 slot)
template <bool BF>
__device__ __forceinline__ _Float16 to_p(float x) {
    if constexpr (BF)
        return __builtin_bit_cast(_Float16, (__bf16)x);
    else
        return (_Float16)x;
}

// eight bf16 ones (0x3F80) in fp16 slots
__device__ __forceinline__ h8 bf16_splat_one() {
    const _Float16 one = __builtin_bit_cast(_Float16, (unsigned short)0x3F80);
    return h8{one, one, one, one, one, one, one, one};
}

__device__ __forceinline__ float exp2_fast(float x) { return __builtin_amdgcn_exp2f(x); }

// ds_read_b64_tr_b16: within each group of 16 lanes, lane i receives in slot k
// element (i % 4) of the four fp16 values addressed by lane 4k + i/4 of its group.
__device__ __forceinline__ h4 lds_read_tr16(const unsigned char* p) {
    typedef short s4 __attribute__((ext_vector_type(4)));
    const s4 r = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
        (__attribute__((address_space(3))) s4*)(__attribute__((address_space(3))) const void*)p);
    return *reinterpret_cast<const h4*>(&r);
}

// A operand of O^T = V^T P^T from a row-major fp16 V tile (row stride `ldr` bytes)
// for MFMA k-slots j = 0..3 -> tile rows kb*4 + j and j = 4..7 -> rows 16 + kb*4 + j-4,
// column (output dim) = lane % 16 of the 16-wide d tile. `p` must point at row
// kb*4 + (lane%16)/4, column d0 + 4*(lane % 4) of the lane's group kb = lane / 16.
__device__ __forceinline__ h8 read_vt(const unsigned char* p, int ldr) {
    const h4 lo = lds_read_tr16(p);
    const h4 hi = lds_read_tr16(p + 16 * ldr);
    return h8{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
}

// One RoPE rotation (cpu_ops.cpp:37-40, cuda_math_kernels.cu:387-392):
// x0' = x0*c - x1*s, x1' = x0*s + x1*c with every product rounded on its own
// (no FMA contraction), then NaN -> 0, clamp to +-65504, RNE fp16.
__device__ __forceinline__ float rot_clamp(float r) {
    if (__builtin_isnan(r)) return 0.0f;
    return fminf(fmaxf(r, -65504.0f), 65504.0f);
}
__device__ __forceinline__ void rope_rotate(float a, float b, float c, float s, _Float16& r0, _Float16& r1) {
#pragma clang fp contract(off)
    const float ac = a * c, bs = b * s, as = a * s, bc = b * c;
    r0 = (_Float16)rot_clamp(ac - bs);
    r1 = (_Float16)rot_clamp(as + bc);
}

// Reference output rule: NaN -> 0, clamp to +-65504, round to nearest even fp16.
__device__ __forceinline__ _Float16 out_half(float r) {
    if (__builtin_isnan(r)) r = 0.0f;
    r = fminf(fmaxf(r, -65504.0f), 65504.0f);
    return (_Float16)r;
}

// Output element: the fp16 rule above, or for bf16 outputs NaN -> 0 and round to
// nearest even bf16 (no clamp: bf16 has the fp32 range)
template <bool BF>
__device__ __forceinline__ _Float16 out_elem(float r) {
    if constexpr (BF) {
        if (__builtin_isnan(r)) r = 0.0f;
        return __builtin_bit_cast(_Float16, (__bf16)r);
    } else {
        return out_half(r);
    }
}

__device__ __forceinline__ float wave_max_xor(float v, int mask) { return fmaxf(v, __shfl_xor(v, mask, 64)); }

// max of v over the lanes l, l^16, l^32, l^48 (the four lane blocks of an MFMA
// column) with the gfx950 VALU lane swaps, no LDS round trip
// v_max_f32 as the hardware does it: a quiet NaN operand yields the other operand. (fmaxf
// on values that come out of a lane swap first quiets each operand with a v_max of itself.)
__device__ __forceinline__ float max_raw(float a, float b) {
    float r;
    asm("v_max_f32 %0, %1, %2" : "=v"(r) : "v"(a), "v"(b));
    return r;
}
__device__ __forceinline__ float col_max4(float v) {
    const auto a = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    v = max_raw(__uint_as_float(a[0]), __uint_as_float(a[1]));
    const auto b = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return max_raw(__uint_as_float(b[0]), __uint_as_float(b[1]));
}
__device__ __forceinline__ float wave_sum_xor(float v, int mask) { return v + __shfl_xor(v, mask, 64); }

// sum of v over the lanes l, l^16, l^32, l^48, the same bits in all four lanes
__device__ __forceinline__ float col_sum4(float v) {
    const auto a = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    v = __uint_as_float(a[0]) + __uint_as_float(a[1]);
    const auto b = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return __uint_as_float(b[0]) + __uint_as_float(b[1]);
}

// Agent-scope coherent access (global_store/load ... sc1): the store is written
// through to the device coherence point and the load bypasses a possibly stale
// XCD-local L2 line, so data handed between workgroups of one launch needs no
// cache-wide buffer_wbl2 / buffer_inv fence.
__device__ __forceinline__ void st_agent(float* p, float v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float ld_agent(const float* p) {
    return __hip_atomic_load(const_cast<float*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
// Agent-coherent buffer loads (cache policy sc1): they see data that other
// workgroups of the same launch wrote through to memory, without a cache-wide
// invalidate, and unlike volatile accesses they pipeline like ordinary loads.
typedef int i4v __attribute__((ext_vector_type(4)));
typedef int i2v __attribute__((ext_vector_type(2)));
constexpr int kCpolSc1 = 16;
__device__ __forceinline__ __amdgpu_buffer_rsrc_t coherent_rsrc(const void* base, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes, 0x00020000);
}
__device__ __forceinline__ f4 ld_coherent4(__amdgpu_buffer_rsrc_t r, uint32_t byte_off) {
    const i4v x = __builtin_amdgcn_raw_buffer_load_b128(r, (int)byte_off, 0, kCpolSc1);
    return *reinterpret_cast<const f4*>(&x);
}
__device__ __forceinline__ float2 ld_coherent2(__amdgpu_buffer_rsrc_t r, uint32_t byte_off) {
    const i2v x = __builtin_amdgcn_raw_buffer_load_b64(r, (int)byte_off, 0, kCpolSc1);
    return *reinterpret_cast<const float2*>(&x);
}

// The same accesses with the cache policy as a parameter: kCpolSc1 (agent-coherent, as
// above) or kCpolSc0 (loads miss the CU's L1 and are served by the XCD's L2, coherent with
// plain stores of other CUs of the same XCD; stores with policy 0 are written to that L2).
constexpr int kCpolSc0 = 1;
template <int CP>
__device__ __forceinline__ f4 ld_pol4(__amdgpu_buffer_rsrc_t r, uint32_t byte_off) {
    const i4v x = __builtin_amdgcn_raw_buffer_load_b128(r, (int)byte_off, 0, CP);
    return *reinterpret_cast<const f4*>(&x);
}
template <int CP>
__device__ __forceinline__ float2 ld_pol2(__amdgpu_buffer_rsrc_t r, uint32_t byte_off) {
    const i2v x = __builtin_amdgcn_raw_buffer_load_b64(r, (int)byte_off, 0, CP);
    return *reinterpret_cast<const float2*>(&x);
}
template <int CP>
__device__ __forceinline__ uint32_t ld_pol1(__amdgpu_buffer_rsrc_t r, uint32_t byte_off) {
    return (uint32_t)__builtin_amdgcn_raw_buffer_load_b32(r, (int)byte_off, 0, CP);
}
template <int CP>
__device__ __forceinline__ void st_pol4(__amdgpu_buffer_rsrc_t r, uint32_t byte_off, f4 v) {
    __builtin_amdgcn_raw_buffer_store_b128(*reinterpret_cast<const i4v*>(&v), r, (int)byte_off, 0, CP);
}
template <int CP>
__device__ __forceinline__ void st_pol2(__amdgpu_buffer_rsrc_t r, uint32_t byte_off, float2 v) {
    __builtin_amdgcn_raw_buffer_store_b64(*reinterpret_cast<const i2v*>(&v), r, (int)byte_off, 0, CP);
}
template <int CP>
__device__ __forceinline__ void st_pol1(__amdgpu_buffer_rsrc_t r, uint32_t byte_off, uint32_t v) {
    __builtin_amdgcn_raw_buffer_store_b32((int)v, r, (int)byte_off, 0, CP);
}

// Buffer descriptor from wave-uniform values, built from SGPRs (readfirstlane): without it
// the compiler may treat the descriptor as divergent and wrap every load in a waterfall loop.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t uniform_rsrc(const void* base, uint32_t bytes) {
    const uint64_t a = reinterpret_cast<uint64_t>(base);
    const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)a), hi = __builtin_amdgcn_readfirstlane((uint32_t)(a >> 32));
    const void* ptr = reinterpret_cast<const void*>(((uint64_t)hi << 32) | lo);
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(ptr), (short)0, (int)__builtin_amdgcn_readfirstlane(bytes),
                                             0x00020000);
}

// Buffer loads; offsets at or past the descriptor's byte count read as zero. 16 bytes with
// the nontemporal cache policy (nt: K/V rows, read once), and one fp16 value as its bits
// with the default policy (int8 block scales: one cache line holds every kv head's scales of
// a position, read by all their workgroups; nt there measured 1 % slower).
constexpr int kCpolNt = 2;
__device__ __forceinline__ u4 ld_buf_nt(__amdgpu_buffer_rsrc_t r, uint32_t byte_off) {
    const i4v x = __builtin_amdgcn_raw_buffer_load_b128(r, (int)byte_off, 0, kCpolNt);
    return *reinterpret_cast<const u4*>(&x);
}
__device__ __forceinline__ short ld_buf_f16(__amdgpu_buffer_rsrc_t r, uint32_t byte_off) {
    return __builtin_amdgcn_raw_buffer_load_b16(r, (int)byte_off, 0, 0);
}
// Copies of loaded registers, made at this point of the program into registers other than
// the source (early clobber). A pipeline stage that is copied out and then reloaded in
// place keeps its loop-carried registers: left to itself, the compiler may load the refill
// into fresh registers and move it back at the end of the loop iteration, which waits for
// the refill right after issuing it. The fp16 form also keeps the compiler from repacking
// or converting the loaded bits before this point.
__device__ __forceinline__ uint32_t copy_here(uint32_t x) {
    uint32_t y;
    asm volatile("v_mov_b32 %0, %1" : "=&v"(y) : "v"(x));
    return y;
}
__device__ __forceinline__ u4 copy_here(u4 x) {
    return u4{copy_here(x[0]), copy_here(x[1]), copy_here(x[2]), copy_here(x[3])};
}
__device__ __forceinline__ _Float16 f16_bits_here(short x) {
    return __builtin_bit_cast(_Float16, (short)copy_here((uint32_t)(uint16_t)x));
}

__device__ __forceinline__ void st_coherent4(__amdgpu_buffer_rsrc_t r, uint32_t byte_off, f4 v) {
    __builtin_amdgcn_raw_buffer_store_b128(*reinterpret_cast<const i4v*>(&v), r, (int)byte_off, 0, kCpolSc1);
}
__device__ __forceinline__ void st_coherent2(__amdgpu_buffer_rsrc_t r, uint32_t byte_off, float2 v) {
    __builtin_amdgcn_raw_buffer_store_b64(*reinterpret_cast<const i2v*>(&v), r, (int)byte_off, 0, kCpolSc1);
}

// Materialises a wave-uniform value in SGPRs at this point of the program (so its load
// is issued here, together with the others pinned next to it).
template <typename T>
__device__ __forceinline__ void pin_sgpr(const T& x) {
    asm volatile("" ::"s"(x));
}

// s_waitcnt vmcnt(0): every vector memory operation of this wave has completed.
// The memory clobber keeps the compiler from moving memory accesses across it.
__device__ __forceinline__ void wait_vmem() { asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); }

template <typename T>
__device__ __forceinline__ T ld_nt(const T* p) {
    return __builtin_nontemporal_load(p);
}

// Dequantize 16 int8 values with one fp16 scale into two 16-byte fp16 chunks. Each code
// q becomes the fp16 number 1664 + q by splicing (q ^ 0x80) under the exponent byte
// 0x66 (v_perm), minus 1664 (exact), times the scale: one fp16 rounding of the exact
// product, the same bits as rounding the fp32 product q * scale to fp16.
__device__ __forceinline__ void dequant16(u4 raw, _Float16 sc, u4& lo, u4& hi) {
    const h2 s2 = h2{sc, sc};
    const h2 bias = h2{(_Float16)1664.0f, (_Float16)1664.0f};
    uint32_t o[8];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const uint32_t u = raw[i] ^ 0x80808080u;
        const uint32_t d0 = __builtin_amdgcn_perm(0x66666666u, u, 0x04010400u);  // bytes u0 66 u1 66
        const uint32_t d1 = __builtin_amdgcn_perm(0x66666666u, u, 0x04030402u);  // bytes u2 66 u3 66
        const h2 x0 = (__builtin_bit_cast(h2, d0) - bias) * s2;
        const h2 x1 = (__builtin_bit_cast(h2, d1) - bias) * s2;
        o[2 * i] = __builtin_bit_cast(uint32_t, x0);
        o[2 * i + 1] = __builtin_bit_cast(uint32_t, x1);
    }
    lo = u4{o[0], o[1], o[2], o[3]};
    hi = u4{o[4], o[5], o[6], o[7]};
}

}  // namespace fa
