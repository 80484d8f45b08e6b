// extern "C" wrapper over the reference's own CPU path, compiled from the
// reference sources where they lie (cpu_ops.cpp, cpu_kquants.cpp,
// cpu_threadpool.cpp). TEST INFRASTRUCTURE ONLY: built into oracle/_ref/ by
// oracle/Makefile (target "ref") and used to pin the C restatement in
// fa_oracle.c and as bench.py's cpu_baseline ("kind": "reference").
#include <cstdint>
#include <memory>

#include "cpu_kquants.h"
#include "cpu_ops.h"
#include "cpu_threadpool.h"

namespace {
std::unique_ptr<friday_cpu::ThreadPool> g_pool;
int g_threads = -1;
friday_cpu::ThreadPool& pool(int threads) {
    if (!g_pool || g_threads != threads) {
        g_pool.reset(new friday_cpu::ThreadPool(threads));
        g_threads = threads;
    }
    return *g_pool;
}
}  // namespace

extern "C" {

float ref_half_to_float(uint16_t h) { return friday_cpu::halfToFloat(h); }
uint16_t ref_float_to_half(float f) { return friday_cpu::floatToHalf(f); }
void ref_round_to_half(float* x, int n) { friday_cpu::roundToHalf(x, n); }

// cpu_ops.cpp:26-43 (q/k are fp32 arrays rotated in place and rounded to fp16 precision)
void ref_rope(float* q, float* k, int head_dim, int nq, int nk, int pos, float freq_base, int neox,
              const float* freq_factors) {
    friday_cpu::rope(q, k, head_dim, nq, nk, pos, freq_base, neox != 0, freq_factors);
}

// cpu_ops.cpp:45-83 over a [seq][nkv*hd] fp32 cache, `threads` pool threads (incl. caller)
void ref_decode_attention(const float* q, const float* k_cache, const float* v_cache, float* out, int seq,
                          int num_heads, int num_kv_heads, int head_dim, int threads) {
    friday_cpu::decodeAttention(q, k_cache, v_cache, out, seq, num_heads, num_kv_heads, head_dim, pool(threads));
}

int ref_pool_size(int threads) { return pool(threads).size(); }

// cpu_kquants.cpp:75-139: x [K] fp32 -> q [K] int8, d [K/32]
void ref_quantize_activation(const float* x, int K, int8_t* q, float* d) {
    friday_cpu::Q8Activation a;
    friday_cpu::quantizeActivation(x, K, a);
    for (int i = 0; i < K; ++i) q[i] = a.q[i];
    for (int i = 0; i < K / 32; ++i) d[i] = a.d[i];
}

// cpu_kquants.cpp:227-280 for a GGUF dtype name ("Q2_K" ...); 0 if unsupported
int ref_dequantize_row(const char* dtype, const uint8_t* row, float* out, int dim) {
    return friday_cpu::dequantizeRow(dtype, row, out, dim) ? 1 : 0;
}

// cpu_kquants.cpp:437-455: y[r] = gemvRowsScalar row r against x quantised by quantizeActivation
void ref_gemv_rows_scalar(const char* dtype, const uint8_t* W, const float* x, int K, float* y, int r0, int r1) {
    friday_cpu::KQuant t;
    if (!friday_cpu::kquantFromDtype(dtype, &t)) return;
    friday_cpu::Q8Activation a;
    friday_cpu::quantizeActivation(x, K, a);
    friday_cpu::gemvRowsScalar(t, W, a, y, r0, r1);
}

// cpu_kquants.cpp:688-: the default (AVX2 when the host has it) row GEMV, timed as the CPU baseline
void ref_gemv_rows(const char* dtype, const uint8_t* W, const float* x, int K, float* y, int r0, int r1) {
    friday_cpu::KQuant t;
    if (!friday_cpu::kquantFromDtype(dtype, &t)) return;
    friday_cpu::Q8Activation a;
    friday_cpu::quantizeActivation(x, K, a);
    friday_cpu::gemvRows(t, W, a, y, r0, r1);
}

}  // extern "C"
