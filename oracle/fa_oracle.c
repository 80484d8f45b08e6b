/*
 * CPU oracle for the FRIDAY KV-cache path. TEST INFRASTRUCTURE ONLY: loaded by
 * tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg as the
 * checker; the product library never links or calls it.
 *
 * Build: gcc -O2 -ffp-contract=off (see oracle/Makefile). Contraction is off so
 * that a*c - b*s is two rounded products and one rounded difference, as in the
 * reference CPU build (x86-64 baseline, no FMA).
 *
 * Pinning (tests/test_oracle.py):
 *   fp16 helpers   exhaustive vs numpy float16 and vs the reference's own
 *                  cpu_kquants.cpp built into oracle/_ref (when present);
 *   rope/append    bit-exact vs reference cpu_ops.cpp rope via oracle/_ref and
 *                  committed golden vectors made from it; pos 0 identity;
 *   decode         bit-exact vs reference cpu_ops.cpp decodeAttention (oracle/_ref,
 *                  golden vectors); fp64 brute force; closed forms (S=1, equal
 *                  rows, dominant key, NaN rows, GQA head sharing);
 *   split/merge    partition invariance vs the unsplit oracle; 1-split merge
 *                  identity;
 *   prefill        row t equals decode at S = p0+t+1 by construction, causal
 *                  perturbation invariance;
 *   q8 append      closed forms (zero block, amax element maps to +-127,
 *                  dequant error <= dh/2) and brute-force rne;
 *   bf16 prefill   (no reference counterpart) conversions vs torch bfloat16,
 *                  exhaustive / 200k patterns; equals the fp16 prefill up to the
 *                  final rounding on inputs both types hold; fp64 brute force.
 */
#include "fa_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

/* ---- fp16 (cpu_kquants.cpp:17-58 halfToFloat/floatToHalf, :141-163 roundToHalf) ---- */

float or_half_to_float(uint16_t h) {
    const int sign = (h >> 15) & 1;
    const int e = (h >> 10) & 0x1f;
    const int m = h & 0x3ff;
    float v;
    if (e == 0) {
        v = ldexpf((float)m, -24); /* zero or subnormal: m * 2^-24, exact */
    } else if (e == 31) {
        v = m ? NAN : INFINITY;
    } else {
        v = ldexpf((float)(m | 0x400), e - 25);
    }
    if (e == 31 && m) {
        /* keep the payload bits like the bit-level conversion does */
        uint32_t bits = ((uint32_t)sign << 31) | 0x7f800000u | ((uint32_t)m << 13);
        memcpy(&v, &bits, 4);
        return v;
    }
    return sign ? -v : v;
}

uint16_t or_float_to_half(float f) {
    uint32_t x;
    memcpy(&x, &f, 4);
    const uint16_t sign = (uint16_t)((x >> 16) & 0x8000u);
    const uint32_t ax = x & 0x7fffffffu;
    if (ax > 0x7f800000u) return (uint16_t)(sign | 0x7e00u); /* NaN (quiet) */
    if (ax == 0x7f800000u) return (uint16_t)(sign | 0x7c00u);
    /* Scale so that one fp16 ulp at this magnitude becomes 1, round to an
     * integer half-to-even, then rebuild. Works for subnormals (ulp 2^-24). */
    int exp2;
    const float a = fabsf(f);
    if (a == 0.0f) return sign;
    frexpf(a, &exp2); /* a = mant * 2^exp2, mant in [0.5, 1) */
    int e_unb = exp2 - 1; /* a in [2^e_unb, 2^(e_unb+1)) */
    if (e_unb < -14) e_unb = -14; /* subnormal range shares the 2^-24 ulp */
    const int ulp_exp = e_unb - 10;
    double scaled = ldexp((double)a, -ulp_exp); /* exact: a has 24 bits */
    double r = nearbyint(scaled);               /* default mode: ties to even */
    double back = ldexp(r, ulp_exp);
    if (back >= 65520.0) return (uint16_t)(sign | 0x7c00u); /* overflow -> inf */
    /* encode back (exactly representable in fp16 now) */
    if (back < ldexp(1.0, -14)) {
        return (uint16_t)(sign | (uint16_t)ldexp(back, 24));
    }
    int be;
    double bm = frexp(back, &be); /* back = bm * 2^be, bm in [0.5,1) */
    const int hexp = be - 1 + 15;
    const uint16_t mant = (uint16_t)(ldexp(bm, 11) - 1024.0);
    return (uint16_t)(sign | (uint16_t)(hexp << 10) | mant);
}

float or_round_to_half(float v) {
    if (isnan(v)) v = 0.0f;
    else if (v > 65504.0f) v = 65504.0f;
    else if (v < -65504.0f) v = -65504.0f;
    return or_half_to_float(or_float_to_half(v));
}

void or_halves_to_floats(const uint16_t* h, float* f, size_t n) {
    for (size_t i = 0; i < n; ++i) f[i] = or_half_to_float(h[i]);
}

void or_floats_to_halves(const float* f, uint16_t* h, size_t n) {
    for (size_t i = 0; i < n; ++i) h[i] = or_float_to_half(f[i]);
}

/* ---- bf16 (no reference counterpart: the reference caches are fp16). The top 16
 * bits of an fp32; float -> bf16 rounds to nearest even on the dropped 16 bits. ---- */

float or_bf16_to_float(uint16_t b) {
    const uint32_t x = (uint32_t)b << 16;
    float f;
    memcpy(&f, &x, 4);
    return f;
}

uint16_t or_float_to_bf16(float f) {
    uint32_t x;
    memcpy(&x, &f, 4);
    if ((x & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((x >> 16) | 0x0040u); /* NaN stays NaN (quiet) */
    const uint32_t lsb = (x >> 16) & 1u;
    return (uint16_t)((x + 0x7fffu + lsb) >> 16);
}

/* output rule of the bf16 prefill: NaN -> 0, round to nearest even bf16 */
float or_round_to_bf16(float v) {
    if (isnan(v)) v = 0.0f;
    return or_bf16_to_float(or_float_to_bf16(v));
}

/* ---- RoPE (cpu_ops.cpp:26-43) ---- */

void or_rope_table(float* cs, int max_pos, int head_dim, float freq_base, const float* freq_factors) {
    const int hd2 = head_dim / 2;
    for (int i = 0; i < hd2; ++i) {
        const float inv_den = powf(freq_base, (2.0f * (float)i) / (float)head_dim);
        for (int p = 0; p < max_pos; ++p) {
            float theta = (float)p / inv_den;
            if (freq_factors) theta /= freq_factors[i];
            cs[((size_t)p * hd2 + i) * 2 + 0] = cosf(theta);
            cs[((size_t)p * hd2 + i) * 2 + 1] = sinf(theta);
        }
    }
}

static uint16_t rot_store(float r) { return or_float_to_half(or_round_to_half(r)); }

static void rotate_head(uint16_t* x, const float* cs_row, int head_dim, int neox) {
    const int hd2 = head_dim / 2;
    for (int i = 0; i < hd2; ++i) {
        const int o0 = neox ? i : 2 * i;
        const int o1 = neox ? i + hd2 : 2 * i + 1;
        const float c = cs_row[2 * i], s = cs_row[2 * i + 1];
        const float a = or_half_to_float(x[o0]), b = or_half_to_float(x[o1]);
        const float ac = a * c, bs = b * s, as = a * s, bc = b * c;
        x[o0] = rot_store(ac - bs);
        x[o1] = rot_store(as + bc);
    }
}

void or_rope_append(uint16_t* q, uint16_t* k, const uint16_t* v, uint16_t* k_cache, uint16_t* v_cache,
                    const float* cs, int pos0, int T, int Hq, int Hkv, int head_dim, int neox) {
    const int kv_dim = Hkv * head_dim, qd = Hq * head_dim, hd2 = head_dim / 2;
    for (int t = 0; t < T; ++t) {
        const int pos = pos0 + t;
        const float* row = cs + (size_t)pos * hd2 * 2;
        for (int h = 0; h < Hq; ++h) rotate_head(q + (size_t)t * qd + h * head_dim, row, head_dim, neox);
        for (int h = 0; h < Hkv; ++h) rotate_head(k + (size_t)t * kv_dim + h * head_dim, row, head_dim, neox);
        if (k_cache) memcpy(k_cache + (size_t)pos * kv_dim, k + (size_t)t * kv_dim, (size_t)kv_dim * 2);
        if (v_cache) memcpy(v_cache + (size_t)pos * kv_dim, v + (size_t)t * kv_dim, (size_t)kv_dim * 2);
    }
}

/* ---- int8 append (cuda_math_kernels.cu:409-432) ---- */

void or_store_kv_q8(const uint16_t* k, const uint16_t* v, int8_t* k_cache, uint16_t* k_scale, int8_t* v_cache,
                    uint16_t* v_scale, int pos0, int T, int kv_dim) {
    const int nblk = kv_dim / 32;
    for (int t = 0; t < T; ++t) {
        const size_t pos = (size_t)pos0 + t;
        for (int which = 0; which < 2; ++which) {
            const uint16_t* src = (which ? v : k) + (size_t)t * kv_dim;
            int8_t* dst = (which ? v_cache : k_cache) + pos * kv_dim;
            uint16_t* sc = (which ? v_scale : k_scale) + pos * nblk;
            for (int b = 0; b < nblk; ++b) {
                float amax = 0.0f;
                for (int i = 0; i < 32; ++i) {
                    float x = or_half_to_float(src[b * 32 + i]);
                    if (isnan(x)) x = 0.0f;
                    const float ax = fabsf(x);
                    if (ax > amax) amax = ax;
                }
                const uint16_t dh = or_float_to_half(amax / 127.0f);
                const float d = or_half_to_float(dh);
                const float inv = d > 0.0f ? 1.0f / d : 0.0f;
                for (int i = 0; i < 32; ++i) {
                    float x = or_half_to_float(src[b * 32 + i]);
                    if (isnan(x)) x = 0.0f;
                    float qf = nearbyintf(x * inv);
                    int qi = qf > 127.0f ? 127 : (qf < -127.0f ? -127 : (int)qf);
                    dst[b * 32 + i] = (int8_t)qi;
                }
                sc[b] = dh;
            }
        }
    }
}

/* ---- decode attention (cpu_ops.cpp:45-83) ---- */

typedef float (*kv_get_fn)(const void* cache, const uint16_t* scale, size_t idx);

static float get_f16(const void* cache, const uint16_t* scale, size_t idx) {
    (void)scale;
    return or_half_to_float(((const uint16_t*)cache)[idx]);
}
static float get_q8(const void* cache, const uint16_t* scale, size_t idx) {
    return (float)((const int8_t*)cache)[idx] * or_half_to_float(scale[idx / 32]);
}
static float get_bf16(const void* cache, const uint16_t* scale, size_t idx) {
    (void)scale;
    return or_bf16_to_float(((const uint16_t*)cache)[idx]);
}

/* bf16 != 0: q, K, V are bf16 and the output takes the bf16 rule (or_round_to_bf16);
 * otherwise fp16 q and the reference's fp16 output rule (or_round_to_half) */
static void decode_any(const uint16_t* q, const void* kc, const uint16_t* ks, const void* vc, const uint16_t* vs,
                       kv_get_fn get, float* out, int S, int Hq, int Hkv, int hd, int kv_stride, int bf16) {
    const int per_kv = Hq / Hkv;
    const float scale = 1.0f / sqrtf((float)hd);
    float* s = (float*)malloc(sizeof(float) * (S > 0 ? S : 1));
    float* acc = (float*)malloc(sizeof(float) * hd);
    float* qf = (float*)malloc(sizeof(float) * hd);
    for (int h = 0; h < Hq; ++h) {
        const int kvh = h / per_kv;
        for (int d = 0; d < hd; ++d) qf[d] = bf16 ? or_bf16_to_float(q[h * hd + d]) : or_half_to_float(q[h * hd + d]);
        float mx = -1e30f;
        for (int p = 0; p < S; ++p) {
            const size_t base = (size_t)p * kv_stride + (size_t)kvh * hd;
            float dot = 0.0f;
            for (int d = 0; d < hd; ++d) dot += qf[d] * get(kc, ks, base + d);
            dot *= scale;
            if (isnan(dot)) dot = -1e30f;
            s[p] = dot;
            if (dot > mx) mx = dot;
        }
        float sum = 0.0f;
        for (int p = 0; p < S; ++p) {
            const float df = s[p] - mx;
            s[p] = df < -50.0f ? 0.0f : expf(df);
            sum += s[p];
        }
        const float inv = sum > 1e-12f ? 1.0f / sum : 0.0f;
        for (int d = 0; d < hd; ++d) acc[d] = 0.0f;
        for (int p = 0; p < S; ++p) {
            const float w = s[p] * inv;
            const size_t base = (size_t)p * kv_stride + (size_t)kvh * hd;
            for (int d = 0; d < hd; ++d) acc[d] += w * get(vc, vs, base + d);
        }
        for (int d = 0; d < hd; ++d) out[h * hd + d] = bf16 ? or_round_to_bf16(acc[d]) : or_round_to_half(acc[d]);
    }
    free(s);
    free(acc);
    free(qf);
}

static void decode_generic(const uint16_t* q, const void* kc, const uint16_t* ks, const void* vc, const uint16_t* vs,
                           kv_get_fn get, float* out, int S, int Hq, int Hkv, int hd, int kv_stride) {
    decode_any(q, kc, ks, vc, vs, get, out, S, Hq, Hkv, hd, kv_stride, 0);
}

void or_decode_attention(const uint16_t* q, const uint16_t* k_cache, const uint16_t* v_cache, float* out, int S,
                         int Hq, int Hkv, int head_dim, int kv_stride) {
    decode_generic(q, k_cache, NULL, v_cache, NULL, get_f16, out, S, Hq, Hkv, head_dim, kv_stride);
}

void or_decode_attention_q8(const uint16_t* q, const int8_t* k_cache, const uint16_t* k_scale, const int8_t* v_cache,
                            const uint16_t* v_scale, float* out, int S, int Hq, int Hkv, int head_dim) {
    decode_generic(q, k_cache, k_scale, v_cache, v_scale, get_q8, out, S, Hq, Hkv, head_dim, Hkv * head_dim);
}

void or_decode_attention_f64(const uint16_t* q, const uint16_t* k_cache, const uint16_t* v_cache, double* out, int S,
                             int Hq, int Hkv, int hd, int kv_stride) {
    const int per_kv = Hq / Hkv;
    const double scale = 1.0 / sqrt((double)hd);
    double* s = (double*)malloc(sizeof(double) * (S > 0 ? S : 1));
    for (int h = 0; h < Hq; ++h) {
        const int kvh = h / per_kv;
        double mx = -1e30;
        for (int p = 0; p < S; ++p) {
            const size_t base = (size_t)p * kv_stride + (size_t)kvh * hd;
            double dot = 0.0;
            for (int d = 0; d < hd; ++d)
                dot += (double)or_half_to_float(q[h * hd + d]) * (double)or_half_to_float(k_cache[base + d]);
            dot *= scale;
            if (isnan(dot)) dot = -1e30;
            s[p] = dot;
            if (dot > mx) mx = dot;
        }
        double sum = 0.0;
        for (int p = 0; p < S; ++p) {
            const double df = s[p] - mx;
            s[p] = df < -50.0 ? 0.0 : exp(df);
            sum += s[p];
        }
        for (int d = 0; d < hd; ++d) {
            double a = 0.0;
            for (int p = 0; p < S; ++p)
                a += s[p] * (double)or_half_to_float(v_cache[(size_t)p * kv_stride + (size_t)kvh * hd + d]);
            out[h * hd + d] = sum > 1e-12 ? a / sum : 0.0;
        }
    }
    free(s);
}

/* ---- split-K + LSE merge (attention_kernels.cu:207-235 merge, :267-411 partials) ---- */

void or_lse_merge(const float* part_o, const float* part_m, const float* part_l, int nsp, int hd, float* out) {
    float M = -1e30f;
    for (int s = 0; s < nsp; ++s) M = fmaxf(M, part_m[s]);
    for (int d = 0; d < hd; ++d) {
        float L = 0.0f, acc = 0.0f;
        for (int s = 0; s < nsp; ++s) {
            const float diff = part_m[s] - M;
            const float w = diff < -50.0f ? 0.0f : expf(diff);
            L += w * part_l[s];
            acc += w * part_o[(size_t)s * hd + d];
        }
        float r = L > 1e-12f ? acc / L : 0.0f;
        out[d] = or_round_to_half(r);
    }
}

void or_decode_attention_split(const uint16_t* q, const uint16_t* k_cache, const uint16_t* v_cache, float* out, int S,
                               int Hq, int Hkv, int hd, int nsplit) {
    const int kv_dim = Hkv * hd, per_kv = Hq / Hkv;
    const float scale = 1.0f / sqrtf((float)hd);
    const int chunk = (S + nsplit - 1) / nsplit;
    const int nsp = (S + chunk - 1) / chunk;
    float* po = (float*)malloc(sizeof(float) * (size_t)nsp * hd);
    float* pm = (float*)malloc(sizeof(float) * nsp);
    float* pl = (float*)malloc(sizeof(float) * nsp);
    float* e = (float*)malloc(sizeof(float) * chunk);
    for (int h = 0; h < Hq; ++h) {
        const int kvh = h / per_kv;
        for (int sp = 0; sp < nsp; ++sp) {
            const int start = sp * chunk, n = (S - start < chunk) ? S - start : chunk;
            float m = -1e30f;
            for (int i = 0; i < n; ++i) {
                const size_t base = (size_t)(start + i) * kv_dim + (size_t)kvh * hd;
                float dot = 0.0f;
                for (int d = 0; d < hd; ++d) dot += or_half_to_float(q[h * hd + d]) * or_half_to_float(k_cache[base + d]);
                float sc = dot * scale;
                if (isnan(sc)) sc = -1e30f;
                e[i] = sc;
                m = fmaxf(m, sc);
            }
            float l = 0.0f;
            for (int i = 0; i < n; ++i) {
                const float df = e[i] - m;
                e[i] = df < -50.0f ? 0.0f : expf(df);
                l += e[i];
            }
            for (int d = 0; d < hd; ++d) {
                float a = 0.0f;
                for (int i = 0; i < n; ++i)
                    a += e[i] * or_half_to_float(v_cache[(size_t)(start + i) * kv_dim + (size_t)kvh * hd + d]);
                po[(size_t)sp * hd + d] = a;
            }
            pm[sp] = m;
            pl[sp] = l;
        }
        or_lse_merge(po, pm, pl, nsp, hd, out + (size_t)h * hd);
    }
    free(po);
    free(pm);
    free(pl);
    free(e);
}

/* ---- prefill (attention_kernels.h:36-45; test_prefill_attention.cu:63-84 equivalence) ---- */

void or_prefill_attention(const uint16_t* q, const uint16_t* k_cache, const uint16_t* v_cache, float* out, int T,
                          int p0, int Hq, int Hkv, int hd) {
    const size_t qd = (size_t)Hq * hd;
    for (int t = 0; t < T; ++t)
        or_decode_attention(q + t * qd, k_cache, v_cache, out + t * qd, p0 + t + 1, Hq, Hkv, hd, Hkv * hd);
}

void or_prefill_attention_q8(const uint16_t* q, const int8_t* k_cache, const uint16_t* k_scale, const int8_t* v_cache,
                             const uint16_t* v_scale, float* out, int T, int p0, int Hq, int Hkv, int hd) {
    const size_t qd = (size_t)Hq * hd;
    for (int t = 0; t < T; ++t)
        or_decode_attention_q8(q + t * qd, k_cache, k_scale, v_cache, v_scale, out + t * qd, p0 + t + 1, Hq, Hkv, hd);
}

/* bf16 q / caches / output: the same causal rows in the same order, bf16 inputs
 * widened exactly, the output rounded by or_round_to_bf16 */
void or_prefill_attention_bf16(const uint16_t* q, const uint16_t* k_cache, const uint16_t* v_cache, float* out, int T,
                               int p0, int Hq, int Hkv, int hd) {
    const size_t qd = (size_t)Hq * hd;
    for (int t = 0; t < T; ++t)
        decode_any(q + t * qd, k_cache, NULL, v_cache, NULL, get_bf16, out + t * qd, p0 + t + 1, Hq, Hkv, hd,
                   Hkv * hd, 1);
}

/* ---- the same prefill rows, blocked for speed (test infrastructure) ----
 *
 * or_prefill_rows_f32 computes rows of or_prefill_attention / _q8 / _bf16 with the very
 * same fp32 operations per output value: the cache values are widened once
 * (or_prefill_widen: the exact fp16 / bf16 value, or the int8 code times its fp16 scale in
 * one fp32 product, as get_q8 forms it), K is stored transposed per kv head so that the dot
 * products of many positions and query heads are formed side by side, and every dot
 * product still accumulates q[d] * k[d] in increasing d from 0.0f, every softmax sum runs
 * over increasing p, and every output column sums w * v over increasing p. Only the
 * loop nesting differs, which changes no rounding (contraction is off). Pinned bit for bit
 * against the row-by-row functions in tests/test_oracle.py. */

/* kt[(h * hd + d) * S + p] and vf[(p * Hkv + h) * hd + d] from a cache of any kind */
void or_prefill_widen(const void* kc, const uint16_t* ks, const void* vc, const uint16_t* vs, int kind, int S,
                      int Hkv, int hd, float* kt, float* vf) {
    kv_get_fn get = kind == 1 ? get_q8 : (kind == 2 ? get_bf16 : get_f16);
    const int kv = Hkv * hd;
    for (int p = 0; p < S; ++p)
        for (int h = 0; h < Hkv; ++h)
            for (int d = 0; d < hd; ++d) {
                const size_t i = (size_t)p * kv + (size_t)h * hd + d;
                kt[((size_t)h * hd + d) * S + p] = get(kc, ks, i);
                vf[i] = get(vc, vs, i);
            }
}

#define OR_PB 256 /* positions per score block */

/* rows t0 .. t0 + T - 1 of a chunk whose row t attends positions [0, p0 + t]; q holds the T
 * rows ([T][Hq * hd], fp16 or bf16 bits), kt / vf come from or_prefill_widen over Smax >=
 * p0 + t0 + T positions; bf16 != 0: bf16 q and the bf16 output rule */
void or_prefill_rows_f32(const uint16_t* q, const float* kt, const float* vf, int Smax, float* out, int T, int p0,
                         int Hq, int Hkv, int hd, int bf16) {
    const int G = Hq / Hkv;
    const float scale = 1.0f / sqrtf((float)hd);
    const int Slast = p0 + T; /* positions the last row attends */
    float* qf = (float*)malloc(sizeof(float) * (size_t)T * G * hd);
    float* s = (float*)malloc(sizeof(float) * (size_t)T * G * (Slast > 0 ? Slast : 1));
    float* acc = (float*)malloc(sizeof(float) * (size_t)T * G * hd);
    for (int h = 0; h < Hkv; ++h) {
        /* the T x G queries of this kv head, widened */
        for (int t = 0; t < T; ++t)
            for (int g = 0; g < G; ++g)
                for (int d = 0; d < hd; ++d) {
                    const uint16_t x = q[(size_t)t * Hq * hd + (size_t)(h * G + g) * hd + d];
                    qf[((size_t)t * G + g) * hd + d] = bf16 ? or_bf16_to_float(x) : or_half_to_float(x);
                }
        /* scores: s[j][p] = sum_d qf[j][d] * k[p][d] in increasing d, for p < the row's length */
        for (int pb = 0; pb < Slast; pb += OR_PB) {
            const int pe = pb + OR_PB < Slast ? pb + OR_PB : Slast;
            for (int j = 0; j < T * G; ++j) {
                float* sj = s + (size_t)j * Slast;
                for (int p = pb; p < pe; ++p) sj[p] = 0.0f;
            }
            for (int d = 0; d < hd; ++d) {
                const float* kr = kt + ((size_t)h * hd + d) * Smax;
                for (int j = 0; j < T * G; ++j) {
                    const int Sj = p0 + j / G + 1;
                    if (pb >= Sj) continue;
                    const int e = pe < Sj ? pe : Sj;
                    const float qd = qf[(size_t)j * hd + d];
                    float* sj = s + (size_t)j * Slast;
                    for (int p = pb; p < e; ++p) sj[p] += qd * kr[p];
                }
            }
        }
        /* softmax per query in increasing p, then acc[d] += w * v[p][d] in increasing p */
        for (int j = 0; j < T * G; ++j) {
            const int Sj = p0 + j / G + 1;
            float* sj = s + (size_t)j * Slast;
            float mx = -1e30f;
            for (int p = 0; p < Sj; ++p) {
                float dot = sj[p] * scale;
                if (isnan(dot)) dot = -1e30f;
                sj[p] = dot;
                if (dot > mx) mx = dot;
            }
            float sum = 0.0f;
            for (int p = 0; p < Sj; ++p) {
                const float df = sj[p] - mx;
                sj[p] = df < -50.0f ? 0.0f : expf(df);
                sum += sj[p];
            }
            const float inv = sum > 1e-12f ? 1.0f / sum : 0.0f;
            for (int p = 0; p < Sj; ++p) sj[p] *= inv;
            float* aj = acc + (size_t)j * hd;
            for (int d = 0; d < hd; ++d) aj[d] = 0.0f;
        }
        for (int p = 0; p < Slast; ++p) {
            const float* vr = vf + ((size_t)p * Hkv + h) * hd;
            for (int j = 0; j < T * G; ++j) {
                if (p >= p0 + j / G + 1) continue;
                const float w = s[(size_t)j * Slast + p];
                float* aj = acc + (size_t)j * hd;
                for (int d = 0; d < hd; ++d) aj[d] += w * vr[d];
            }
        }
        for (int j = 0; j < T * G; ++j) {
            const int t = j / G, g = j % G;
            float* o = out + (size_t)t * Hq * hd + (size_t)(h * G + g) * hd;
            const float* aj = acc + (size_t)j * hd;
            for (int d = 0; d < hd; ++d) o[d] = bf16 ? or_round_to_bf16(aj[d]) : or_round_to_half(aj[d]);
        }
    }
    free(qf);
    free(s);
    free(acc);
}

/* ---- paged addressing (paged_attention.cu:29-41: phys = table[pos/16], row pos%16) ---- */

void or_paged_gather(const uint16_t* pool, const int32_t* block_table, int S, int page, int kv_dim, uint16_t* dst) {
    for (int p = 0; p < S; ++p) {
        const int phys = block_table[p / page];
        memcpy(dst + (size_t)p * kv_dim, pool + ((size_t)phys * page + (p % page)) * kv_dim, (size_t)kv_dim * 2);
    }
}
