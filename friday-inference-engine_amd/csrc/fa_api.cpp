// C-ABI layer of libfriday_attn: argument validation (before any HIP call),
// status codes instead of the reference's exceptions/abort, and the host-side
// RoPE table. Entry points are declared and documented in include/friday_attn.h.
#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstdlib>
#include <atomic>
#include <mutex>
#include <string>
#include <vector>

#include "../../include/friday_attn.h"
#include "fa_internal.hpp"

namespace {

thread_local std::string g_err;

int fail(int code, const char* fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    std::vsnprintf(buf, sizeof(buf), fmt, ap);
    va_end(ap);
    g_err = buf;
    return code;
}

int ok() {
    g_err.clear();
    return FA_OK;
}

int launch_status(int rc, const char* what) {
    if (rc == -2) return fail(FA_ERR_UNSUPPORTED, "%s: unsupported configuration", what);
    if (rc != 0) {
        const hipError_t e = hipGetLastError();
        return fail(FA_ERR_LAUNCH, "%s: launch failed: %s", what, hipGetErrorString(e));
    }
    return ok();
}

bool head_dim_ok(int d) { return d == 64 || d == 128; }

// The append moves 16-byte chunks: every tensor it touches must be 16-byte aligned (null is fine).
bool aligned16(const void* a, const void* b, const void* c, const void* d, const void* e) {
    return ((reinterpret_cast<uintptr_t>(a) | reinterpret_cast<uintptr_t>(b) | reinterpret_cast<uintptr_t>(c) |
             reinterpret_cast<uintptr_t>(d) | reinterpret_cast<uintptr_t>(e)) & 15) == 0;
}

// Shape rules of the reference launchers (attention_kernels.cu:416-419, 450-454).
int check_heads(const char* what, int Hq, int Hkv, int d) {
    if (!head_dim_ok(d)) return fail(FA_ERR_UNSUPPORTED, "%s: head_dim must be 64 or 128 (got %d)", what, d);
    if (Hkv <= 0 || Hq <= 0 || Hq % Hkv != 0)
        return fail(FA_ERR_INVALID, "%s: invalid shape (num_heads %d, num_kv_heads %d)", what, Hq, Hkv);
    return FA_OK;
}

// One RoPE angle pair, written with the formula of friday_cpu::rope (cpu_ops.cpp:29-32).
void rope_fill(float* table, int max_ctx, int head_dim, float freq_base, const float* ff) {
    const int hd2 = head_dim / 2;
    for (int i = 0; i < hd2; ++i) {
        const float den = std::pow(freq_base, (2.0f * (float)i) / (float)head_dim);
        for (int p = 0; p < max_ctx; ++p) {
            float theta = (float)p / den;
            if (ff) theta /= ff[i];
            float* e = table + ((size_t)p * hd2 + i) * 2;
            e[0] = std::cos(theta);
            e[1] = std::sin(theta);
        }
    }
}

int env_int(const char* name, int dflt, int lo, int hi) {
    const char* e = std::getenv(name);
    if (!e || !*e) return dflt;
    const int v = std::atoi(e);
    return v < lo ? lo : (v > hi ? hi : v);
}

// Workspace: arrival counter slots [B*Hq], 256 bytes each, at offset 0 (the fused
// merge uses B*Hkv*ceil(G/16) <= B*Hq of them, each an arrival count and the base it had
// when the last launch completed; they must stay at a fixed place whatever the split
// count of a call), then part_o [B*Hq][ns][d] fp32 and
// part_ml [B*Hq][ns][2].
size_t counters_bytes(int batch, int Hq) { return (size_t)batch * Hq * fa::kCounterStride * sizeof(int); }

size_t split_ws_bytes(int batch, int Hq, int max_seq, int d) {
    const size_t ns = (size_t)fa::split_bound(max_seq, fa::min_chunk(), fa::max_splits());
    // counter slots, then the partials (o, then m and l), then one flag word per split
    return counters_bytes(batch, Hq) + (size_t)batch * Hq * ns * ((size_t)d + 3) * sizeof(float);
}

// counter_region > 0: the partials start at that fixed offset instead of right after this
// call's counter slots (a workspace shared by calls with different head counts).
void set_workspace(fa::DecodeParams& p, void* ws, int batch, int d, bool fused, size_t counter_region = 0) {
    char* base = static_cast<char*>(ws);
    p.counters = fused ? reinterpret_cast<int*>(base) : nullptr;
    p.part_o = reinterpret_cast<float*>(base + (counter_region ? counter_region : counters_bytes(batch, p.Hq)));
    p.part_ml = p.part_o + (size_t)batch * p.Hq * p.nsplit_grid * d;
    p.flags = reinterpret_cast<unsigned*>(p.part_ml + (size_t)batch * p.Hq * p.nsplit_grid * 2);
}

}  // namespace

namespace fa {
// Split partition: about S / min_chunk splits of >= min_chunk positions, at most
// max_splits (a multiple of 128 and <= 256 respectively).
int min_chunk() {
    static const int v = env_int("FRIDAY_ATTN_MIN_CHUNK", 128, 1, 1 << 20) / kSpan * kSpan;
    return v < kSpan ? kSpan : v;
}
int max_splits() {
    static const int v = env_int("FRIDAY_ATTN_MAX_SPLITS", kMaxSplitsLimit, 1, kMaxSplitsLimit);
    return v;
}
// Decode placement and merge form: the environment's choice, read once, until
// friday_attn_set_decode_form overrides it for the process.
std::atomic<int> g_local_merge{-1}, g_split_major{-1}, g_kv_pair{-1};
int q8_deep_default() {
    static const int v = env_int("FRIDAY_ATTN_Q8_DEEP", 0, 0, 1);
    return v;
}
int kv_pair_for(bool paged, int Hkv, int ngb) {
    static const int v = env_int("FRIDAY_ATTN_KV_PAIR", 0, 0, 1);
    const int o = g_kv_pair.load(std::memory_order_relaxed);
    const int want = o >= 0 ? o : v;
    return want && !paged && ngb == 1 && Hkv % 2 == 0 ? 2 : 1;
}
int local_merge_default() {
    static const int v = env_int("FRIDAY_ATTN_LOCAL_MERGE", 0, 0, 1);
    const int o = g_local_merge.load(std::memory_order_relaxed);
    return o >= 0 ? o : v;
}
int split_major_default() {
    static const int v = env_int("FRIDAY_ATTN_SPLIT_MAJOR", 0, 0, 1);
    const int o = g_split_major.load(std::memory_order_relaxed);
    return o >= 0 ? o : v;
}
// Compute units of the current device (256 on an MI355X), asked once per device.
int device_cus() {
    static std::atomic<int> cus[64];
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
    int n = cus[dev].load(std::memory_order_relaxed);
    if (n <= 0) {
        if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) n = 256;
        cus[dev].store(n, std::memory_order_relaxed);
    }
    return n;
}
// Splits per (kv head, head block) so that one sequence keeps about `target`
// workgroups streaming: one per CU of the device (FRIDAY_ATTN_TARGET_WGS overrides it).
// The partition stays a function of S, the head layout and the device, never of the batch.
int splits_for(int Hkv, int ngb) {
    static const int target_env = env_int("FRIDAY_ATTN_TARGET_WGS", 0, 0, 1 << 16);
    const int target = target_env > 0 ? target_env : device_cus();
    const int groups = Hkv * ngb;
    int ns = target / (groups > 0 ? groups : 1);
    ns = ns < 1 ? 1 : ns;
    return ns < max_splits() ? ns : max_splits();
}
}  // namespace fa

extern "C" {

const char* friday_attn_last_error(void) { return g_err.c_str(); }

int friday_attn_version(void) { return 100; }

// ---------------- RoPE table ----------------

size_t friday_attn_rope_table_bytes(int max_ctx, int head_dim) {
    if (max_ctx <= 0 || head_dim <= 0 || head_dim % 2) return 0;
    return (size_t)max_ctx * (head_dim / 2) * 2 * sizeof(float);
}

int friday_attn_rope_table_fill_host(float* table, int max_ctx, int head_dim, float freq_base,
                                     const float* freq_factors_host) {
    if (!table || max_ctx <= 0 || !head_dim_ok(head_dim) || !(freq_base > 0.0f))
        return fail(FA_ERR_INVALID, "rope_table_fill_host: invalid arguments");
    rope_fill(table, max_ctx, head_dim, freq_base, freq_factors_host);
    return ok();
}

int friday_attn_rope_table_upload(float* d_table, int max_ctx, int head_dim, float freq_base,
                                  const float* freq_factors_host, void* stream) {
    if (!d_table || max_ctx <= 0 || !head_dim_ok(head_dim) || !(freq_base > 0.0f))
        return fail(FA_ERR_INVALID, "rope_table_upload: invalid arguments");
    std::vector<float> host((size_t)max_ctx * head_dim);
    rope_fill(host.data(), max_ctx, head_dim, freq_base, freq_factors_host);
    hipStream_t s = static_cast<hipStream_t>(stream);
    if (hipMemcpyAsync(d_table, host.data(), host.size() * sizeof(float), hipMemcpyHostToDevice, s) != hipSuccess ||
        hipStreamSynchronize(s) != hipSuccess)
        return fail(FA_ERR_LAUNCH, "rope_table_upload: copy failed: %s", hipGetErrorString(hipGetLastError()));
    return ok();
}

// ---------------- append ----------------

int friday_attn_rope_store_kv(uint16_t* q, uint16_t* k, const uint16_t* v, uint16_t* k_layer, uint16_t* v_layer,
                              const int* d_pos, int pos, int T, int head_dim, int num_q_heads, int num_kv_heads,
                              int max_ctx, const float* rope_table, int neox, void* stream) {
    const char* w = "rope_store_kv";
    if (int rc = check_heads(w, num_q_heads, num_kv_heads, head_dim)) return rc;
    if (T <= 0 || max_ctx <= 0 || !q || !k || !rope_table) return fail(FA_ERR_INVALID, "%s: invalid arguments", w);
    if ((k_layer == nullptr) != (v_layer == nullptr) || (k_layer && !v))
        return fail(FA_ERR_INVALID, "%s: k_layer, v_layer and v must be given together", w);
    if (!d_pos && (pos < 0 || pos + T > max_ctx))
        return fail(FA_ERR_INVALID, "%s: positions [%d, %d) exceed max_ctx %d", w, pos, pos + T, max_ctx);
    if (!aligned16(q, k, v, k_layer, v_layer)) return fail(FA_ERR_INVALID, "%s: q, k, v and caches must be 16-byte aligned", w);
    fa::RopeParams p{};
    p.q = q; p.k = k; p.v = v; p.k_dst = k_layer; p.v_dst = v_layer; p.table = rope_table;
    p.d_pos = d_pos; p.pos = pos; p.T = T; p.D = head_dim; p.Hq = num_q_heads; p.Hkv = num_kv_heads;
    p.max_ctx = max_ctx; p.neox = neox ? 1 : 0;
    return launch_status(fa::launch_rope_store(p, false, static_cast<hipStream_t>(stream)), w);
}

int friday_attn_store_kv_q8(const uint16_t* k, const uint16_t* v, int8_t* k_layer, uint16_t* k_scale,
                            int8_t* v_layer, uint16_t* v_scale, const int* d_pos, int pos, int T, int kv_dim,
                            int max_ctx, void* stream) {
    const char* w = "store_kv_q8";
    if (!k || !v || !k_layer || !k_scale || !v_layer || !v_scale || T <= 0 || max_ctx <= 0)
        return fail(FA_ERR_INVALID, "%s: invalid arguments", w);
    if (kv_dim <= 0 || kv_dim % 32) return fail(FA_ERR_INVALID, "%s: kv_dim must be a multiple of 32", w);
    if (!d_pos && (pos < 0 || pos + T > max_ctx))
        return fail(FA_ERR_INVALID, "%s: positions [%d, %d) exceed max_ctx %d", w, pos, pos + T, max_ctx);
    fa::Q8StoreParams p{};
    p.k = k; p.v = v; p.k_dst = k_layer; p.ks_dst = k_scale; p.v_dst = v_layer; p.vs_dst = v_scale;
    p.d_pos = d_pos; p.pos = pos; p.T = T; p.kv_dim = kv_dim; p.max_ctx = max_ctx;
    return launch_status(fa::launch_store_kv_q8(p, static_cast<hipStream_t>(stream)), w);
}

// ---------------- decode ----------------

static int decode_common(const char* w, const uint16_t* q, const void* k, const void* v, uint16_t* out, int seq_len,
                         const int* d_pos, int max_seq, int Hq, int Hkv, int d, void* ws, size_t ws_bytes,
                         bool single, bool fused, const uint16_t* ks, const uint16_t* vs, void* stream) {
    if (int rc = check_heads(w, Hq, Hkv, d)) return rc;
    if (!q || !k || !v || !out) return fail(FA_ERR_INVALID, "%s: null tensor", w);
    if (max_seq <= 0) return fail(FA_ERR_INVALID, "%s: invalid max_seq_len %d", w, max_seq);
    if (!d_pos && (seq_len <= 0 || seq_len > max_seq))
        return fail(FA_ERR_INVALID, "%s: seq_len %d outside [1, %d]", w, seq_len, max_seq);
    const bool q8 = ks && vs;
    if ((ks == nullptr) != (vs == nullptr)) return fail(FA_ERR_INVALID, "%s: give both k_scale and v_scale", w);
    if (!aligned16(q, k, v, nullptr, nullptr) || reinterpret_cast<uintptr_t>(out) % 8)
        return fail(FA_ERR_INVALID, "%s: q and the caches must be 16-byte aligned, out 8-byte aligned", w);
    const int G = Hq / Hkv;
    fa::DecodeParams p{};
    p.q = q; p.k = k; p.v = v; p.k_scale = ks; p.v_scale = vs; p.d_pos = d_pos;
    p.seq_len = d_pos ? 0 : seq_len;
    p.max_seq = max_seq;
    p.out = out; p.Hq = Hq; p.Hkv = Hkv; p.G = G; p.ngb = (G + 15) / 16; p.kv_dim = Hkv * d;
    p.single = single ? 1 : 0;
    p.min_chunk = fa::min_chunk();
    p.kpw = fa::kv_pair_for(false, Hkv, p.ngb);
    p.max_splits = fa::splits_for(Hkv / p.kpw, p.ngb);
    p.scale2 = (1.0f / std::sqrt((float)d)) * 1.4426950408889634f;
    if (!single) {
        // host length: the grid only needs the splits of seq_len
        const int grid_len = d_pos ? max_seq : seq_len;
        p.nsplit_grid = fa::split_bound(grid_len, p.min_chunk, p.max_splits);
        const size_t need = split_ws_bytes(1, Hq, grid_len, d);
        if (need >= (size_t(1) << 31))  // partials are addressed with 32-bit buffer offsets
            return fail(FA_ERR_UNSUPPORTED, "%s: split workspace beyond 2 GiB (%zu bytes)", w, need);
        if (!ws || ws_bytes < need)
            return fail(FA_ERR_WORKSPACE, "%s: workspace of %zu bytes needed (got %zu)", w, need, ws_bytes);
        set_workspace(p, ws, 1, d, fused);
    } else {
        p.nsplit_grid = 1;
    }
    return launch_status(fa::launch_decode(p, d, 1, false, q8, static_cast<hipStream_t>(stream)), w);
}

int friday_attn_decode_attention(const uint16_t* q, const uint16_t* k_cache, const uint16_t* v_cache, uint16_t* out,
                                 int seq_len, int num_heads, int num_kv_heads, int head_dim, void* stream) {
    return decode_common("decode_attention", q, k_cache, v_cache, out, seq_len, nullptr, seq_len > 0 ? seq_len : 1,
                         num_heads, num_kv_heads, head_dim, nullptr, 0, true, false, nullptr, nullptr, stream);
}

int friday_attn_decode_attention_dev_pos(const uint16_t* q, const uint16_t* k_cache, const uint16_t* v_cache,
                                         uint16_t* out, const int* d_pos, int max_seq_len, int num_heads,
                                         int num_kv_heads, int head_dim, void* stream) {
    if (!d_pos) return fail(FA_ERR_INVALID, "decode_attention_dev_pos: d_pos is null");
    return decode_common("decode_attention_dev_pos", q, k_cache, v_cache, out, 0, d_pos, max_seq_len, num_heads,
                         num_kv_heads, head_dim, nullptr, 0, true, false, nullptr, nullptr, stream);
}

int friday_attn_decode_fits_shared_memory(int max_seq_len) { return max_seq_len > 0 ? 1 : 0; }

size_t friday_attn_split_workspace_bytes(int num_heads, int max_seq_len) {
    if (num_heads <= 0 || max_seq_len <= 0) return 0;
    return split_ws_bytes(1, num_heads, max_seq_len, 128);
}

int friday_attn_decode_attention_split(const uint16_t* q, const void* k_cache, const void* v_cache, uint16_t* out,
                                       int seq_len, const int* d_pos, int max_seq_len, int num_heads,
                                       int num_kv_heads, int head_dim, void* workspace, size_t workspace_bytes,
                                       void* stream, const uint16_t* k_scale, const uint16_t* v_scale) {
    return decode_common("decode_attention_split", q, k_cache, v_cache, out, seq_len, d_pos, max_seq_len, num_heads,
                         num_kv_heads, head_dim, workspace, workspace_bytes, false, false, k_scale, v_scale, stream);
}

int friday_attn_decode_workspace_init(void* workspace, size_t workspace_bytes, void* stream) {
    if (!workspace || workspace_bytes == 0 || workspace_bytes % 4)
        return fail(FA_ERR_INVALID, "decode_workspace_init: invalid workspace");
    return launch_status(fa::launch_zero_fill(workspace, workspace_bytes, static_cast<hipStream_t>(stream)),
                         "decode_workspace_init");
}

int friday_attn_set_decode_form(int local_merge, int split_major, int kv_pair) {
    if (local_merge < -1 || local_merge > 1 || split_major < -1 || split_major > 1 || kv_pair < -1 || kv_pair > 1)
        return fail(FA_ERR_INVALID, "set_decode_form: values must be -1, 0 or 1");
    fa::g_local_merge.store(local_merge, std::memory_order_relaxed);
    fa::g_split_major.store(split_major, std::memory_order_relaxed);
    fa::g_kv_pair.store(kv_pair, std::memory_order_relaxed);
    // the local form's placement check runs now (the null stream, synchronised), so that
    // launches recorded into graphs later can use the form
    if (local_merge == 1) fa::local_placement_ok(nullptr);
    return ok();
}

int friday_attn_decode_workspace_status(const void* workspace, size_t workspace_bytes, void* stream) {
    const char* w = "decode_workspace_status";
    if (!workspace || workspace_bytes < (fa::kStatusWord + 1) * sizeof(unsigned))
        return fail(FA_ERR_INVALID, "%s: invalid workspace", w);
    unsigned word = 0;
    hipStream_t s = static_cast<hipStream_t>(stream);
    if (hipMemcpyAsync(&word, static_cast<const unsigned*>(workspace) + fa::kStatusWord, sizeof(word),
                       hipMemcpyDeviceToHost, s) != hipSuccess ||
        hipStreamSynchronize(s) != hipSuccess)
        return fail(FA_ERR_LAUNCH, "%s: copy failed: %s", w, hipGetErrorString(hipGetLastError()));
    if (word & fa::kStatusMergeTimeout)
        return fail(FA_ERR_TIMEOUT,
                    "%s: a fused merge gave up waiting for its splits; outputs since the last "
                    "friday_attn_decode_workspace_init are not valid: initialise the workspace again", w);
    return ok();
}

int friday_attn_decode_attention_fused(const uint16_t* q, const void* k_cache, const void* v_cache, uint16_t* out,
                                       int seq_len, const int* d_pos, int max_seq_len, int num_heads,
                                       int num_kv_heads, int head_dim, void* workspace, size_t workspace_bytes,
                                       void* stream, const uint16_t* k_scale, const uint16_t* v_scale) {
    return decode_common("decode_attention_fused", q, k_cache, v_cache, out, seq_len, d_pos, max_seq_len, num_heads,
                         num_kv_heads, head_dim, workspace, workspace_bytes, false, true, k_scale, v_scale, stream);
}

namespace {
// Shared by the fp16 and int8 one-launch steps.
int decode_step_common(const char* w, uint16_t* q, const uint16_t* k, const uint16_t* v, const void* k_layer,
                       const void* v_layer, const uint16_t* k_scale, const uint16_t* v_scale, uint16_t* out,
                       const int* d_pos, int pos, int max_ctx, int num_heads, int num_kv_heads, int head_dim,
                       const float* rope_table, int neox, void* workspace, size_t workspace_bytes, void* stream,
                       int8_t* out_q = nullptr, float* out_d = nullptr, size_t counter_region = 0) {
    if (int rc = check_heads(w, num_heads, num_kv_heads, head_dim)) return rc;
    if (!q || !k || !v || !k_layer || !v_layer || !out || !rope_table || max_ctx <= 0)
        return fail(FA_ERR_INVALID, "%s: invalid arguments", w);
    if (!d_pos && (pos < 0 || pos >= max_ctx))
        return fail(FA_ERR_INVALID, "%s: position %d outside [0, %d)", w, pos, max_ctx);
    // q, the new k / v rows and the cache rows move as 16-byte chunks, out as 8-byte ones
    if (!aligned16(q, k, v, k_layer, v_layer) || reinterpret_cast<uintptr_t>(out) % 8)
        return fail(FA_ERR_INVALID, "%s: q, k, v and the caches must be 16-byte aligned, out 8-byte aligned", w);
    const bool q8 = k_scale != nullptr;
    const int G = num_heads / num_kv_heads;
    fa::DecodeParams p{};
    p.q = q; p.k = k_layer; p.v = v_layer; p.d_pos = d_pos; p.seq_len = d_pos ? 0 : pos + 1; p.max_seq = max_ctx;
    p.k_scale = k_scale; p.v_scale = v_scale;
    p.out = out; p.Hq = num_heads; p.Hkv = num_kv_heads; p.G = G; p.ngb = (G + 15) / 16;
    p.out_q = out_q; p.out_d = out_d;
    p.kv_dim = num_kv_heads * head_dim;
    p.min_chunk = fa::min_chunk();
    p.kpw = fa::kv_pair_for(false, num_kv_heads, p.ngb);
    p.max_splits = fa::splits_for(num_kv_heads / p.kpw, p.ngb);
    p.scale2 = (1.0f / std::sqrt((float)head_dim)) * 1.4426950408889634f;
    p.rope_table = rope_table; p.k_new = k; p.v_new = v; p.neox = neox ? 1 : 0;
    const int grid_len = d_pos ? max_ctx : pos + 1;
    p.nsplit_grid = fa::split_bound(grid_len, p.min_chunk, p.max_splits);
    size_t need = split_ws_bytes(1, num_heads, grid_len, head_dim);
    if (counter_region) {
        if (counters_bytes(1, num_heads) > counter_region)
            return fail(FA_ERR_WORKSPACE, "%s: %d heads exceed the counter region", w, num_heads);
        need += counter_region - counters_bytes(1, num_heads);
    }
    if (need >= (size_t(1) << 31))  // partials are addressed with 32-bit buffer offsets
        return fail(FA_ERR_UNSUPPORTED, "%s: split workspace beyond 2 GiB (%zu bytes)", w, need);
    if (!workspace || workspace_bytes < need)
        return fail(FA_ERR_WORKSPACE, "%s: workspace of %zu bytes needed (got %zu)", w, need, workspace_bytes);
    set_workspace(p, workspace, 1, head_dim, true, counter_region);
    return launch_status(fa::launch_decode(p, head_dim, 1, false, q8, static_cast<hipStream_t>(stream)), w);
}
}  // namespace

int friday_attn_decode_step(uint16_t* q, const uint16_t* k, const uint16_t* v, uint16_t* k_layer, uint16_t* v_layer,
                            uint16_t* out, const int* d_pos, int pos, int max_ctx, int num_heads, int num_kv_heads,
                            int head_dim, const float* rope_table, int neox, void* workspace, size_t workspace_bytes,
                            void* stream) {
    return decode_step_common("decode_step", q, k, v, k_layer, v_layer, nullptr, nullptr, out, d_pos, pos, max_ctx,
                              num_heads, num_kv_heads, head_dim, rope_table, neox, workspace, workspace_bytes, stream);
}

namespace {
// Device scratch of friday_attn_decode_step_noalloc: the arrival counters and split
// partials that a caller's workspace holds otherwise. The counters have a fixed region of
// 1 MiB (one 256-byte slot per query head, up to 4096 heads) and the partials the 3 MiB
// after it, whatever the head count of a call, so calls of models with different head
// counts can share the scratch (each call leaves its counters equal to their bases). Every
// GPU the library runs on holds its own copy until the process ends.
constexpr size_t kScratchBytes = size_t(4) << 20;
constexpr size_t kScratchCounterBytes = size_t(1) << 20;
__device__ __align__(256) unsigned char scratch[kScratchBytes];

// The device address of the current device's scratch (the host-side name `scratch` is not
// one), looked up once per device with that device current and kept. Nothing is launched:
// the array is zero when the code object is loaded (counter and base start equal, and every
// completed call advances both by the same amount), so the first call may be made under
// stream capture or on any stream. A failed lookup is not kept; the next call tries again.
std::mutex g_scratch_mu;
void* g_scratch_ptr[64] = {};

void* scratch_ptr(hipError_t* err) {
    int dev = 0;
    if ((*err = hipGetDevice(&dev)) != hipSuccess) return nullptr;
    if (dev < 0 || dev >= 64) return *err = hipErrorInvalidDevice, nullptr;
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (!g_scratch_ptr[dev]) {
        void* ptr = nullptr;
        if ((*err = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch))) != hipSuccess) return nullptr;
        g_scratch_ptr[dev] = ptr;
    }
    return g_scratch_ptr[dev];
}
}  // namespace

int friday_attn_decode_step_noalloc(uint16_t* q, const uint16_t* k, const uint16_t* v, uint16_t* k_layer,
                                    uint16_t* v_layer, uint16_t* out, const int* d_pos, int pos, int max_ctx,
                                    int num_heads, int num_kv_heads, int head_dim, const float* rope_table, int neox,
                                    void* stream) {
    const char* w = "decode_step_noalloc";
    if (int rc = check_heads(w, num_heads, num_kv_heads, head_dim)) return rc;
    if (!q || !k || !v || !k_layer || !v_layer || !out || !rope_table || max_ctx <= 0)
        return fail(FA_ERR_INVALID, "%s: invalid arguments", w);
    if (!d_pos && (pos < 0 || pos >= max_ctx))
        return fail(FA_ERR_INVALID, "%s: position %d outside [0, %d)", w, pos, max_ctx);
    const size_t need = kScratchCounterBytes + (split_ws_bytes(1, num_heads, d_pos ? max_ctx : pos + 1, head_dim) -
                                                counters_bytes(1, num_heads));
    if (counters_bytes(1, num_heads) > kScratchCounterBytes || need > kScratchBytes)
        return fail(FA_ERR_WORKSPACE, "%s: needs %zu bytes of scratch, more than the %zu held per GPU", w, need,
                    kScratchBytes);
    if (!aligned16(q, k, v, k_layer, v_layer) || reinterpret_cast<uintptr_t>(out) % 8)
        return fail(FA_ERR_INVALID, "%s: q, k, v and the caches must be 16-byte aligned, out 8-byte aligned", w);
    hipError_t err = hipSuccess;
    void* ws = scratch_ptr(&err);
    if (!ws) return fail(FA_ERR_LAUNCH, "%s: device scratch unavailable: %s", w, hipGetErrorString(err));
    return decode_step_common(w, q, k, v, k_layer, v_layer, nullptr, nullptr, out, d_pos, pos, max_ctx, num_heads,
                              num_kv_heads, head_dim, rope_table, neox, ws, kScratchBytes, stream, nullptr, nullptr,
                              kScratchCounterBytes);
}

int friday_attn_decode_step_q8(uint16_t* q, const uint16_t* k, const uint16_t* v, int8_t* k_layer,
                               uint16_t* k_scale, int8_t* v_layer, uint16_t* v_scale, uint16_t* out,
                               const int* d_pos, int pos, int max_ctx, int num_heads, int num_kv_heads,
                               int head_dim, const float* rope_table, int neox, void* workspace,
                               size_t workspace_bytes, void* stream) {
    if (!k_scale || !v_scale) return fail(FA_ERR_INVALID, "decode_step_q8: scales required");
    return decode_step_common("decode_step_q8", q, k, v, k_layer, v_layer, k_scale, v_scale, out, d_pos, pos,
                              max_ctx, num_heads, num_kv_heads, head_dim, rope_table, neox, workspace,
                              workspace_bytes, stream);
}

int friday_attn_decode_step_quant(uint16_t* q, const uint16_t* k, const uint16_t* v, uint16_t* k_layer,
                                  uint16_t* v_layer, uint16_t* out, int8_t* out_q, float* out_d, const int* d_pos,
                                  int pos, int max_ctx, int num_heads, int num_kv_heads, int head_dim,
                                  const float* rope_table, int neox, void* workspace, size_t workspace_bytes,
                                  void* stream) {
    const char* w = "decode_step_quant";
    if (!out_q || !out_d) return fail(FA_ERR_INVALID, "%s: out_q and out_d required", w);
    if (reinterpret_cast<uintptr_t>(out_q) % 4 || reinterpret_cast<uintptr_t>(out_d) % 4)
        return fail(FA_ERR_INVALID, "%s: out_q / out_d must be 4-byte aligned", w);
    return decode_step_common(w, q, k, v, k_layer, v_layer, nullptr, nullptr, out, d_pos, pos, max_ctx, num_heads,
                              num_kv_heads, head_dim, rope_table, neox, workspace, workspace_bytes, stream, out_q,
                              out_d);
}

// ---------------- prefill ----------------

int friday_attn_prefill_supported(int num_heads, int num_kv_heads, int head_dim) {
    return head_dim_ok(head_dim) && num_kv_heads > 0 && num_heads > 0 && num_heads % num_kv_heads == 0 ? 1 : 0;
}

int friday_attn_prefill_attention(const uint16_t* q, const void* k_cache, const void* v_cache, uint16_t* out, int T,
                                  const int* d_pos0, int num_heads, int num_kv_heads, int head_dim, void* stream,
                                  const uint16_t* k_scale, const uint16_t* v_scale) {
    const char* w = "prefill_attention";
    if (T <= 0) return ok();  // the reference launcher returns early (attention_kernels.cu:656)
    if (int rc = check_heads(w, num_heads, num_kv_heads, head_dim)) return rc;
    if (!q || !k_cache || !v_cache || !out || !d_pos0) return fail(FA_ERR_INVALID, "%s: null argument", w);
    if ((k_scale == nullptr) != (v_scale == nullptr)) return fail(FA_ERR_INVALID, "%s: give both scales", w);
    fa::PrefillParams p{};
    p.q = q; p.k = k_cache; p.v = v_cache; p.k_scale = k_scale; p.v_scale = v_scale; p.out = out;
    p.d_pos0 = d_pos0; p.T = T; p.Hq = num_heads; p.Hkv = num_kv_heads; p.G = num_heads / num_kv_heads;
    p.scale2 = (1.0f / std::sqrt((float)head_dim)) * 1.4426950408889634f;
    return launch_status(fa::launch_prefill(p, head_dim, k_scale != nullptr, static_cast<hipStream_t>(stream)), w);
}

int friday_attn_prefill_attention_bf16(const uint16_t* q, const uint16_t* k_cache, const uint16_t* v_cache,
                                       uint16_t* out, int T, const int* d_pos0, int num_heads, int num_kv_heads,
                                       int head_dim, void* stream) {
    const char* w = "prefill_attention_bf16";
    if (T <= 0) return ok();
    if (int rc = check_heads(w, num_heads, num_kv_heads, head_dim)) return rc;
    if (!q || !k_cache || !v_cache || !out || !d_pos0) return fail(FA_ERR_INVALID, "%s: null argument", w);
    fa::PrefillParams p{};
    p.q = q; p.k = k_cache; p.v = v_cache; p.out = out;
    p.d_pos0 = d_pos0; p.T = T; p.Hq = num_heads; p.Hkv = num_kv_heads; p.G = num_heads / num_kv_heads;
    p.scale2 = (1.0f / std::sqrt((float)head_dim)) * 1.4426950408889634f;
    return launch_status(fa::launch_prefill_bf16(p, head_dim, static_cast<hipStream_t>(stream)), w);
}

// ---------------- paged ----------------

static int paged_decode_common(const char* w, uint16_t* q, const uint16_t* k_new, const uint16_t* v_new,
                               uint16_t* k_pool, uint16_t* v_pool, uint16_t* out, const int32_t* block_table,
                               int block_table_stride, const int32_t* seq_lens, int batch, int max_seq_len,
                               int num_heads, int num_kv_heads, int head_dim, const float* rope_table, int neox,
                               void* workspace, size_t workspace_bytes, void* stream) {
    if (int rc = check_heads(w, num_heads, num_kv_heads, head_dim)) return rc;
    if (batch <= 0 || max_seq_len <= 0 || !q || !k_pool || !v_pool || !out || !block_table || !seq_lens)
        return fail(FA_ERR_INVALID, "%s: invalid arguments", w);
    if (block_table_stride <= 0 || (long long)block_table_stride * FA_PAGE_TOKENS < max_seq_len)
        return fail(FA_ERR_INVALID, "%s: block_table_stride %d cannot address max_seq_len %d", w,
                    block_table_stride, max_seq_len);
    if (!aligned16(q, k_new, v_new, k_pool, v_pool) || reinterpret_cast<uintptr_t>(out) % 8)
        return fail(FA_ERR_INVALID, "%s: q, k, v and the pools must be 16-byte aligned, out 8-byte aligned", w);
    const int G = num_heads / num_kv_heads;
    fa::DecodeParams p{};
    p.q = q; p.k = k_pool; p.v = v_pool; p.block_table = block_table; p.bt_stride = block_table_stride;
    p.seq_lens = seq_lens; p.max_seq = max_seq_len; p.out = out;
    p.Hq = num_heads; p.Hkv = num_kv_heads; p.G = G; p.ngb = (G + 15) / 16; p.kv_dim = num_kv_heads * head_dim;
    p.scale2 = (1.0f / std::sqrt((float)head_dim)) * 1.4426950408889634f;
    p.rope_table = rope_table; p.k_new = k_new; p.v_new = v_new; p.neox = neox ? 1 : 0;
    p.min_chunk = fa::min_chunk();
    p.kpw = 1;
    p.max_splits = fa::splits_for(num_kv_heads, p.ngb);
    p.nsplit_grid = fa::split_bound(max_seq_len, p.min_chunk, p.max_splits);
    const size_t need = split_ws_bytes(batch, num_heads, max_seq_len, head_dim);
    if (need >= (size_t(1) << 31))  // partials are addressed with 32-bit buffer offsets
        return fail(FA_ERR_UNSUPPORTED, "%s: split workspace beyond 2 GiB (%zu bytes)", w, need);
    if (!workspace || workspace_bytes < need)
        return fail(FA_ERR_WORKSPACE, "%s: workspace of %zu bytes needed (got %zu)", w, need, workspace_bytes);
    set_workspace(p, workspace, batch, head_dim, true);
    return launch_status(fa::launch_decode(p, head_dim, batch, true, false, static_cast<hipStream_t>(stream)), w);
}

size_t friday_attn_paged_workspace_bytes(int batch, int num_heads, int max_seq_len) {
    if (batch <= 0 || num_heads <= 0 || max_seq_len <= 0) return 0;
    return split_ws_bytes(batch, num_heads, max_seq_len, 128);
}

int friday_attn_paged_rope_store_kv(uint16_t* q, uint16_t* k, const uint16_t* v, uint16_t* k_pool, uint16_t* v_pool,
                                    const int32_t* block_table, int block_table_stride, const int32_t* seq_lens,
                                    int batch, int head_dim, int num_q_heads, int num_kv_heads, int max_ctx,
                                    const float* rope_table, int neox, void* stream) {
    const char* w = "paged_rope_store_kv";
    if (int rc = check_heads(w, num_q_heads, num_kv_heads, head_dim)) return rc;
    if (batch <= 0 || max_ctx <= 0 || !q || !k || !v || !k_pool || !v_pool || !block_table || !seq_lens ||
        !rope_table || block_table_stride <= 0 || (long long)block_table_stride * FA_PAGE_TOKENS < max_ctx)
        return fail(FA_ERR_INVALID, "%s: invalid arguments", w);
    if (!aligned16(q, k, v, k_pool, v_pool)) return fail(FA_ERR_INVALID, "%s: q, k, v and pools must be 16-byte aligned", w);
    fa::RopeParams p{};
    p.q = q; p.k = k; p.v = v; p.k_dst = k_pool; p.v_dst = v_pool; p.table = rope_table;
    p.block_table = block_table; p.bt_stride = block_table_stride; p.seq_lens = seq_lens;
    p.T = batch; p.D = head_dim; p.Hq = num_q_heads; p.Hkv = num_kv_heads; p.max_ctx = max_ctx;
    p.neox = neox ? 1 : 0;
    return launch_status(fa::launch_rope_store(p, true, static_cast<hipStream_t>(stream)), w);
}

int friday_attn_paged_decode_step(uint16_t* q, const uint16_t* k, const uint16_t* v, uint16_t* k_pool,
                                  uint16_t* v_pool, uint16_t* out, const int32_t* block_table,
                                  int block_table_stride, const int32_t* seq_lens, int batch, int max_seq_len,
                                  int num_heads, int num_kv_heads, int head_dim, const float* rope_table, int neox,
                                  void* workspace, size_t workspace_bytes, void* stream) {
    const char* w = "paged_decode_step";
    if (!k || !v || !rope_table) return fail(FA_ERR_INVALID, "%s: invalid arguments", w);
    return paged_decode_common(w, q, k, v, k_pool, v_pool, out, block_table, block_table_stride, seq_lens, batch,
                               max_seq_len, num_heads, num_kv_heads, head_dim, rope_table, neox, workspace,
                               workspace_bytes, stream);
}

int friday_attn_paged_decode_attention(const uint16_t* q, const uint16_t* k_pool, const uint16_t* v_pool,
                                       uint16_t* out, const int32_t* block_table, int block_table_stride,
                                       const int32_t* seq_lens, int batch, int max_seq_len, int num_heads,
                                       int num_kv_heads, int head_dim, void* workspace, size_t workspace_bytes,
                                       void* stream) {
    return paged_decode_common("paged_decode_attention", const_cast<uint16_t*>(q), nullptr, nullptr,
                               const_cast<uint16_t*>(k_pool), const_cast<uint16_t*>(v_pool), out, block_table,
                               block_table_stride, seq_lens, batch, max_seq_len, num_heads, num_kv_heads, head_dim,
                               nullptr, 0, workspace, workspace_bytes, stream);
}

// ---------------- prefill projection GEMM ----------------

static bool kq_kind_ok(int kind) { return kind >= FA_KQ_Q2_K && kind <= FA_KQ_Q8_0; }

size_t friday_q8_row_bytes(int kind, int K) {
    if (!kq_kind_ok(kind) || K <= 0) return 0;
    static const int sb_bytes[7] = {0, 84, 110, 144, 176, 210, 0};
    if (kind == FA_KQ_Q8_0) return K % 32 ? 0 : (size_t)(K / 32) * 34;
    return K % 256 ? 0 : (size_t)(K / 256) * sb_bytes[kind];
}

int friday_quantize_q8_rows(const uint16_t* x, int rows, int K, int8_t* xq, float* xd, void* stream) {
    const char* w = "quantize_q8_rows";
    if (rows <= 0) return ok();
    if (K <= 0 || K % 32) return fail(FA_ERR_INVALID, "%s: K must be a positive multiple of 32 (got %d)", w, K);
    if (!x || !xq || !xd) return fail(FA_ERR_INVALID, "%s: null argument", w);
    if (rows > 65535) return fail(FA_ERR_UNSUPPORTED, "%s: at most 65535 rows per call (got %d)", w, rows);
    return launch_status(fa::launch_quantize_q8_rows(x, rows, K, xq, xd, static_cast<hipStream_t>(stream)), w);
}

int friday_gemm_q8_supported(int kind, int K) { return kq_kind_ok(kind) && K > 0 && K % 256 == 0 ? 1 : 0; }

namespace {
// K-split workspaces of friday_gemm_q8, one per (device, stream): launches on one stream
// run in order, so they can share it. A workspace grows only outside stream capture; the
// buffers it outgrows stay allocated until the process ends, because a captured graph
// may still hold them.
struct GemmWs {
    int dev;
    void* stream;
    void* ptr;
    size_t bytes;
};
std::mutex g_ws_mu;
std::vector<GemmWs> g_ws;
std::vector<void*> g_ws_retired;

// The workspace of (current device, stream) with at least `bytes`, or null when that would
// need an allocation during stream capture. Sets *rc on a HIP error.
void* gemm_workspace(void* stream, size_t bytes, int* rc) {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) return *rc = -1, nullptr;
    std::lock_guard<std::mutex> lk(g_ws_mu);
    GemmWs* e = nullptr;
    for (auto& w : g_ws)
        if (w.dev == dev && w.stream == stream) e = &w;
    if (e && e->bytes >= bytes) return e->ptr;
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    if (hipStreamIsCapturing(static_cast<hipStream_t>(stream), &cs) != hipSuccess) (void)hipGetLastError();
    if (cs != hipStreamCaptureStatusNone) return nullptr;
    const size_t nb = ((bytes + (1u << 20) - 1) >> 20) << 20;
    void* ptr = nullptr;
    if (hipMalloc(&ptr, nb) != hipSuccess) return *rc = -1, nullptr;
    // counters start at zero; ordered before the launch that follows on this stream
    if (hipMemsetAsync(ptr, 0, (size_t)fa::kKqMaxCounters * fa::kCounterStride * 4, static_cast<hipStream_t>(stream)) !=
        hipSuccess)
        return *rc = -1, nullptr;
    if (e) {
        g_ws_retired.push_back(e->ptr);
        e->ptr = ptr;
        e->bytes = nb;
    } else {
        g_ws.push_back(GemmWs{dev, stream, ptr, nb});
    }
    return ptr;
}
}  // namespace

int friday_gemm_q8_reserve(int T, int K, int N, void* stream) {
    const char* w = "gemm_q8_reserve";
    if (T <= 0 || N <= 0 || K <= 0 || K % 256) return fail(FA_ERR_INVALID, "%s: invalid T=%d K=%d N=%d", w, T, K, N);
    const fa::KqPlan sp = fa::kq_gemm_plan(T, K, N);
    int rc = 0;
    if (!gemm_workspace(stream, sp.bytes, &rc))
        return fail(rc ? FA_ERR_LAUNCH : FA_ERR_WORKSPACE, "%s: %s", w,
                    rc ? "workspace allocation failed" : "cannot allocate during stream capture");
    return ok();
}

namespace {
int gemm_common(const char* w, int kind, const void* W, const int8_t* xq, const float* xd, int T, int K, int N,
                uint16_t* Y, int ldy, void* stream, const float* bias, const uint16_t* res, char* ws,
                const fa::KqPlan& sp) {
    fa::KqGemmParams p{};
    p.W = static_cast<const uint8_t*>(W); p.xq = xq; p.xd = xd; p.Y = Y; p.bias = bias; p.res = res;
    p.row_bytes = friday_q8_row_bytes(kind, K);
    p.T = T; p.K = K; p.N = N; p.ldy = ldy;
    // no workspace (stream capture without friday_gemm_q8_reserve): one pass over K, and each
    // workgroup dequantises its activation tile itself (the same values)
    if (ws) {
        if (sp.xh) p.xh = reinterpret_cast<const uint16_t*>(ws + sp.xh_off);
        if (sp.ksplit > 1) {
            p.ksplit = sp.ksplit; p.sps = sp.sps;
            p.counters = reinterpret_cast<int*>(ws);
            p.part = reinterpret_cast<float*>(ws + sp.part_off);
        }
    }
    return launch_status(fa::launch_kq_gemm(kind, p, static_cast<hipStream_t>(stream)), w);
}

int gemm_check(const char* w, int kind, const void* W, const int8_t* xq, const float* xd, int T, int K, int N,
               const uint16_t* Y, int ldy) {
    if (!friday_gemm_q8_supported(kind, K))
        return fail(FA_ERR_UNSUPPORTED, "%s: unsupported type %d or K=%d (K must be a multiple of 256)", w, kind, K);
    if (N <= 0 || ldy < N) return fail(FA_ERR_INVALID, "%s: invalid N=%d / ldy=%d", w, N, ldy);
    if (!W || !xq || !xd || !Y) return fail(FA_ERR_INVALID, "%s: null argument", w);
    if (reinterpret_cast<uintptr_t>(W) % 4 || reinterpret_cast<uintptr_t>(xq) % 16 ||
        reinterpret_cast<uintptr_t>(xd) % 4 || reinterpret_cast<uintptr_t>(Y) % 2)
        return fail(FA_ERR_INVALID, "%s: misaligned W (4 B), xq (16 B), xd or Y", w);
    const long long blocks = (long long)((N + 127) / 128 + 7) / 8 * 8 * ((T + 127) / 128);
    if (blocks > 0x7fffffffLL) return fail(FA_ERR_UNSUPPORTED, "%s: T=%d x N=%d too large for one launch", w, T, N);
    return FA_OK;
}
}  // namespace

int friday_gemm_q8(int kind, const void* W, const int8_t* xq, const float* xd, int T, int K, int N, uint16_t* Y,
                   int ldy, void* stream, const float* bias, const uint16_t* res) {
    const char* w = "gemm_q8";
    if (T <= 0 && friday_gemm_q8_supported(kind, K)) return ok();
    if (int rc = gemm_check(w, kind, W, xq, xd, T > 0 ? T : 1, K, N, Y, ldy)) return rc;
    const fa::KqPlan sp = fa::kq_gemm_plan(T, K, N);
    int rc = 0;
    char* ws = static_cast<char*>(gemm_workspace(stream, sp.bytes, &rc));
    if (rc) return fail(FA_ERR_LAUNCH, "%s: workspace allocation failed", w);
    return gemm_common(w, kind, W, xq, xd, T, K, N, Y, ldy, stream, bias, res, ws, sp);
}

size_t friday_gemm_q8_workspace_bytes(int T, int K, int N) {
    if (T <= 0 || N <= 0 || K <= 0 || K % 256) return 0;
    return fa::kq_gemm_plan(T, K, N).bytes;
}

int friday_gemm_q8_ws(int kind, const void* W, const int8_t* xq, const float* xd, int T, int K, int N, uint16_t* Y,
                      int ldy, void* stream, const float* bias, const uint16_t* res, void* workspace,
                      size_t workspace_bytes) {
    const char* w = "gemm_q8_ws";
    if (T <= 0 && friday_gemm_q8_supported(kind, K)) return ok();
    if (int rc = gemm_check(w, kind, W, xq, xd, T > 0 ? T : 1, K, N, Y, ldy)) return rc;
    const fa::KqPlan sp = fa::kq_gemm_plan(T, K, N);
    if (!workspace || workspace_bytes < sp.bytes || reinterpret_cast<uintptr_t>(workspace) % 256)
        return fail(FA_ERR_WORKSPACE, "%s: 256-byte aligned workspace of %zu bytes needed (got %zu)", w, sp.bytes,
                    workspace_bytes);
    return gemm_common(w, kind, W, xq, xd, T, K, N, Y, ldy, stream, bias, res, static_cast<char*>(workspace), sp);
}

int friday_gemv_q8(int kind, const void* W, const int8_t* xq, const float* xd, int K, int N, uint16_t* y,
                   void* stream, const void* W2, uint16_t* y2, const float* bias, const uint16_t* res) {
    const char* w = "gemv_q8";
    if (!kq_kind_ok(kind)) return fail(FA_ERR_UNSUPPORTED, "%s: unsupported type %d", w, kind);
    if (K <= 0 || K % (kind == FA_KQ_Q8_0 ? 32 : 256))
        return fail(FA_ERR_UNSUPPORTED, "%s: K=%d must be a multiple of %d", w, K, kind == FA_KQ_Q8_0 ? 32 : 256);
    if (N <= 0) return fail(FA_ERR_INVALID, "%s: invalid N=%d", w, N);
    if (!W || !xq || !xd || !y || (W2 && !y2)) return fail(FA_ERR_INVALID, "%s: null argument", w);
    if (reinterpret_cast<uintptr_t>(W) % 4 || reinterpret_cast<uintptr_t>(W2) % 4 ||
        reinterpret_cast<uintptr_t>(xq) % 16 || reinterpret_cast<uintptr_t>(xd) % 4)
        return fail(FA_ERR_INVALID, "%s: misaligned W / W2 (4 B), xq (16 B) or xd", w);
    if ((long long)N * (W2 ? 2 : 1) > 0x7fffffffLL - 3) return fail(FA_ERR_UNSUPPORTED, "%s: N too large", w);
    fa::KqGemvParams p{};
    p.W = static_cast<const uint8_t*>(W); p.W2 = static_cast<const uint8_t*>(W2); p.xq = xq; p.xd = xd;
    p.y = y; p.y2 = y2; p.bias = bias; p.res = res;
    p.row_bytes = friday_q8_row_bytes(kind, K);
    p.K = K; p.N = N;
    return launch_status(fa::launch_kq_gemv(kind, p, static_cast<hipStream_t>(stream)), w);
}

}  // extern "C"
