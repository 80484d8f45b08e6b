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

__device__ __forceinline__ float exp2_fast(float x) { return __builtin_amdgcn_exp2f(x); }

// Reference output rule: NaN -> 0, clamp to +-65504, round to nearest even fp16.
__device__ __forceinline__ _Float16 out_half(float r) {
    if (__builtin_isnan(r)) r = 0.0f;
    r = fminf(fmaxf(r, -65504.0f), 65504.0f);
    return (_Float16)r;
}

__device__ __forceinline__ float wave_max_xor(float v, int mask) { return fmaxf(v, __shfl_xor(v, mask, 64)); }
__device__ __forceinline__ float wave_sum_xor(float v, int mask) { return v + __shfl_xor(v, mask, 64); }

template <typename T>
__device__ __forceinline__ T ld_nt(const T* p) {
    return __builtin_nontemporal_load(p);
}

}  // namespace fa
