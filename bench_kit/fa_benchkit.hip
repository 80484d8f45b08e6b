// Benchmark helpers of bench.py (not part of the product ABI): device-side synthetic data,
// a plain streaming copy used to calibrate the HBM byte counters, and read-pattern probes
// (the K/V access patterns of the decode kernel without its arithmetic) that bound what a
// decode launch can stream.
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

// Read-pattern probe over one layer's K and V caches of S rows x ROWB bytes: 256
// workgroups; workgroup group g of NG = ROWB / SLICE reads the SLICE-byte column g of the
// rows of its split (S / (256 / NG) rows), K and V, with W waves that keep NST tiles of
// 4 x 1 KiB loads per tensor in flight each (non-temporal 16-byte buffer loads, as the
// decode kernel). SM: the groups of one split are dealt to one XCD (split-major ids).
// The loaded bits are folded into one word that is stored only if it equals a magic value.
constexpr int kProbeS = 32768;
__device__ __forceinline__ __amdgpu_buffer_rsrc_t probe_rsrc(const void* base, uint32_t bytes) {
    const uint64_t a = reinterpret_cast<uint64_t>(base);
    const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)a), hi = __builtin_amdgcn_readfirstlane((uint32_t)(a >> 32));
    return __builtin_amdgcn_make_buffer_rsrc(reinterpret_cast<void*>(((uint64_t)hi << 32) | lo), (short)0,
                                             (int)__builtin_amdgcn_readfirstlane(bytes), 0x00020000);
}
typedef int i4v __attribute__((ext_vector_type(4)));
__device__ __forceinline__ i4v probe_ld(__amdgpu_buffer_rsrc_t r, uint32_t off) {
    return __builtin_amdgcn_raw_buffer_load_b128(r, (int)off, 0, 2);
}
template <int ROWB, int SLICE, int W, int NST, bool SM>
__global__ __launch_bounds__(W * 64) void read_probe(const char* K, const char* V, int* out) {
    constexpr int NG = ROWB / SLICE, NSPL = 256 / NG;
    constexpr uint32_t NROWS = kProbeS / NSPL;
    const int lin = blockIdx.x;
    int g, split;
    if (SM && NG > 1) {
        const int r = lin >> 3;
        g = r % NG;
        split = (lin & 7) + 8 * (r / NG);
    } else {
        g = lin % NG;
        split = lin / NG;
    }
    const uint32_t row0 = split * NROWS;
    constexpr int LPR = SLICE >= 1024 ? 64 : SLICE / 16;       // lanes per row and load
    constexpr int RPL = 64 / LPR;                               // rows per load
    constexpr int LDR = SLICE > 1024 ? SLICE / 1024 : 1;        // loads per row
    constexpr uint32_t TR = SLICE >= 1024 ? 4 / LDR : 4 * RPL;  // rows per tile
    constexpr uint32_t NT = NROWS / TR;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int lrow = lane / LPR, lch = lane % LPR;
    const __amdgpu_buffer_rsrc_t rk = probe_rsrc(K + (size_t)row0 * ROWB + g * SLICE, NROWS * ROWB);
    const __amdgpu_buffer_rsrc_t rv = probe_rsrc(V + (size_t)row0 * ROWB + g * SLICE, NROWS * ROWB);
    auto off = [&](uint32_t t, int r) -> uint32_t {
        if (t >= NT) return 0x7fffffffu;  // past the descriptor: zeros, no access
        if (SLICE >= 1024) return (t * TR + r / LDR) * ROWB + (r % LDR) * 1024 + lane * 16;
        return (t * TR + r * RPL + lrow) * ROWB + lch * 16;
    };
    i4v acc = {0, 0, 0, 0};
    i4v bk[NST][4], bv[NST][4];
#pragma unroll
    for (int s = 0; s < NST; ++s) {
#pragma unroll
        for (int r = 0; r < 4; ++r) bk[s][r] = probe_ld(rk, off(wave + s * W, r));
#pragma unroll
        for (int r = 0; r < 4; ++r) bv[s][r] = probe_ld(rv, off(wave + s * W, r));
    }
    for (uint32_t t0 = wave; t0 < NT; t0 += NST * W) {
#pragma unroll
        for (int s = 0; s < NST; ++s) {
#pragma unroll
            for (int r = 0; r < 4; ++r) acc ^= bk[s][r] ^ bv[s][r];
            const uint32_t t = t0 + (s + NST) * W;
#pragma unroll
            for (int r = 0; r < 4; ++r) bk[s][r] = probe_ld(rk, off(t, r));
#pragma unroll
            for (int r = 0; r < 4; ++r) bv[s][r] = probe_ld(rv, off(t, r));
        }
    }
    const int x = acc[0] ^ acc[1] ^ acc[2] ^ acc[3];
    if (x == 0x12345678) out[lin] = x;
}
__global__ void empty_kernel(int*) {}

struct ProbeVariant {
    const char* name;
    int rowb;
    void (*fn)(const char*, const char*, int*);
    int threads;
};
#define FABK_PROBE(ROWB, SLICE, W, NST, SM, NAME) \
    {NAME, ROWB, read_probe<ROWB, SLICE, W, NST, SM>, W * 64}
const ProbeVariant kProbes[] = {
    FABK_PROBE(2048, 256, 4, 1, false, "fp16 rows, 256 B kv-head slices, 4 waves x 1 tile (the decode pattern)"),
    FABK_PROBE(2048, 256, 4, 1, true, "fp16 rows, 256 B slices, split-major placement"),
    FABK_PROBE(2048, 256, 4, 2, false, "fp16 rows, 256 B slices, 4 waves x 2 tiles"),
    FABK_PROBE(2048, 256, 8, 1, false, "fp16 rows, 256 B slices, 8 waves x 1 tile"),
    FABK_PROBE(2048, 512, 8, 1, false, "fp16 rows, 512 B slices (kv-head pairs), 8 waves x 1 tile"),
    FABK_PROBE(2048, 2048, 4, 1, false, "fp16 rows, whole 2 KiB rows, 4 waves x 1 tile"),
    FABK_PROBE(2048, 2048, 8, 1, false, "fp16 rows, whole 2 KiB rows, 8 waves x 1 tile"),
    FABK_PROBE(1024, 128, 8, 1, true, "int8 rows, 128 B slices, split-major, 8 waves x 1 tile (the int8 pattern)"),
    FABK_PROBE(1024, 128, 4, 2, true, "int8 rows, 128 B slices, split-major, 4 waves x 2 tiles"),
    FABK_PROBE(1024, 256, 8, 1, true, "int8 rows, 256 B slices (kv-head pairs), 8 waves x 1 tile"),
    FABK_PROBE(1024, 1024, 8, 1, false, "int8 rows, whole 1 KiB rows, 8 waves x 1 tile"),
};
#undef FABK_PROBE

}  // namespace

extern "C" {

// Read probes: the number of variants; a variant's name and cache row bytes; one launch of
// variant v over the layer at K / V (kProbeS rows each). Variant -1 is an empty kernel of
// 256 workgroups (the launch floor).
int fabk_probe_count(void) { return (int)(sizeof(kProbes) / sizeof(kProbes[0])); }
const char* fabk_probe_name(int v) { return v >= 0 && v < fabk_probe_count() ? kProbes[v].name : "empty kernel"; }
int fabk_probe_row_bytes(int v) { return v >= 0 && v < fabk_probe_count() ? kProbes[v].rowb : 0; }
int fabk_probe_launch(int v, const void* K, const void* V, void* out, void* stream) {
    const hipStream_t s = static_cast<hipStream_t>(stream);
    if (v < 0) {
        hipLaunchKernelGGL(empty_kernel, dim3(256), dim3(256), 0, s, static_cast<int*>(out));
    } else if (v < fabk_probe_count()) {
        hipLaunchKernelGGL(kProbes[v].fn, dim3(256), dim3(kProbes[v].threads), 0, s, static_cast<const char*>(K),
                           static_cast<const char*>(V), static_cast<int*>(out));
    } else {
        return -1;
    }
    return hipGetLastError() == hipSuccess ? 0 : -1;
}

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
