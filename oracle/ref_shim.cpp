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

}  // extern "C"
