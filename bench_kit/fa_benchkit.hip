// Benchmark helpers of bench.py (not part of the product ABI): device-side synthetic data
// and a plain streaming copy used to calibrate the HBM byte counters.
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace {

__device__ __forceinline__ uint32_t mix32(uint32_t x) {
    x ^= x >> 16;
    x *= 0x7feb352dU;
    x ^= x >> 15;
    x *= 0x846ca68bU;
    x ^= x >> 16;
    return x;
}

// Approximately N(0, scale^2) fp16 values from a counter hash (sum of 4 uniforms).
__global__ void fill_normal_f16(_Float16* dst, size_t n, uint32_t seed, float scale) {
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x) {
        const uint32_t base = mix32((uint32_t)i * 4u + seed * 0x9e3779b9u);
        float s = 0.0f;
#pragma unroll
        for (int j = 0; j < 4; ++j) s += (float)(mix32(base + j) >> 8) * (1.0f / 16777216.0f);
        dst[i] = (_Float16)((s - 2.0f) * 1.7320508f * scale);
    }
}

// The same values rounded to bf16 (round to nearest even), stored as raw bits.
__global__ void fill_normal_bf16(uint16_t* dst, size_t n, uint32_t seed, float scale) {
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x) {
        const uint32_t base = mix32((uint32_t)i * 4u + seed * 0x9e3779b9u);
        float s = 0.0f;
#pragma unroll
        for (int j = 0; j < 4; ++j) s += (float)(mix32(base + j) >> 8) * (1.0f / 16777216.0f);
        dst[i] = __builtin_bit_cast(uint16_t, (__bf16)((s - 2.0f) * 1.7320508f * scale));
    }
}

__global__ void copy_u4(const uint4* __restrict__ src, uint4* __restrict__ dst, size_t n) {
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x)
        dst[i] = src[i];
}

}  // namespace

extern "C" {

int fabk_fill_normal_f16(void* dst, size_t n, uint32_t seed, float scale, void* stream) {
    hipLaunchKernelGGL(fill_normal_f16, dim3(4096), dim3(256), 0, static_cast<hipStream_t>(stream),
                       static_cast<_Float16*>(dst), n, seed, scale);
    return hipGetLastError() == hipSuccess ? 0 : -1;
}

int fabk_fill_normal_bf16(void* dst, size_t n, uint32_t seed, float scale, void* stream) {
    hipLaunchKernelGGL(fill_normal_bf16, dim3(4096), dim3(256), 0, static_cast<hipStream_t>(stream),
                       static_cast<uint16_t*>(dst), n, seed, scale);
    return hipGetLastError() == hipSuccess ? 0 : -1;
}

// Copies nbytes (multiple of 16) with one 16-byte load and store per element.
int fabk_copy(const void* src, void* dst, size_t nbytes, void* stream) {
    hipLaunchKernelGGL(copy_u4, dim3(8192), dim3(256), 0, static_cast<hipStream_t>(stream),
                       static_cast<const uint4*>(src), static_cast<uint4*>(dst), nbytes / 16);
    return hipGetLastError() == hipSuccess ? 0 : -1;
}

}  // extern "C"
