/*
 * CPU oracle for the prefill projection GEMM (int8 activations x K-quant
 * weights). TEST INFRASTRUCTURE ONLY: part of libfa_oracle.so, loaded by
 * tests/ and bench.py's cpu_baseline leg; the product library never links it.
 *
 * Restates:
 *   or_quantize_q8_rows   quantize_x_q8_kernel, hpc_k_quants.cu:386-400 (and the
 *                         CPU twin quantizeActivation, cpu_kquants.cpp:75-139):
 *                         per 32 values d = amax / 127 (fp32), inv = d > 0 ? 1/d : 0,
 *                         q = clamp(rne(x * inv), +-127), a NaN product -> 0 (CUDA's
 *                         float -> int conversion; the CPU twin leaves it undefined)
 *   or_dequant_row        dequantizeRow, cpu_kquants.cpp:227-280 (fp32 formulas)
 *   or_kq_block           the integer form of one 32-value block of a weight row,
 *                         dequant32 in prefill_kernels.cu:57-144: integers q, the
 *                         per-16 scale / min of the block
 *   or_gemm_q8            gemm_q8_kernel, prefill_kernels.cu:173-327: per 32-value
 *                         block the exact integer dot product(s), scaled in fp32 and
 *                         accumulated over the blocks in order; then the storeY
 *                         epilogue, prefill_kernels.cu:155-171 (fp16 rounding, + bias
 *                         fp32, + residual fp16, NaN -> 0 and +-65504 clamp at each step)
 *
 * Pinning (tests/test_gemm_oracle.py): quantisation and dequantisation bit-exact
 * against the reference's own cpu_kquants.cpp built into oracle/_ref; the GEMM
 * against the reference's gemvRowsScalar (same integers, other fp32 order) and
 * against an fp64 product of the dequantised operands; the epilogue by its closed
 * forms (NaN inputs, clamping, residual aliasing).
 *
 * Weight kinds use the codes of friday_hpc::Q8Kind (hpc_k_quants.h:39):
 * 1 Q2_K (84 B / 256), 2 Q3_K (110 B), 3 Q4_K (144 B), 4 Q5_K (176 B), 5 Q6_K (210 B),
 * 6 Q8_0 (34 B / 32).
 */
#include "fa_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

enum { KQ2 = 1, KQ3 = 2, KQ4 = 3, KQ5 = 4, KQ6 = 5, KQ80 = 6 };

static float h16(const uint8_t* p) {
    uint16_t h;
    memcpy(&h, p, 2);
    return or_half_to_float(h);
}

size_t or_q8_row_bytes(int kind, int K) {
    switch (kind) {
        case KQ2: return (size_t)(K / 256) * 84;
        case KQ3: return (size_t)(K / 256) * 110;
        case KQ4: return (size_t)(K / 256) * 144;
        case KQ5: return (size_t)(K / 256) * 176;
        case KQ6: return (size_t)(K / 256) * 210;
        case KQ80: return (size_t)(K / 32) * 34;
        default: return 0;
    }
}

void or_quantize_q8_rows(const uint16_t* x, int rows, int K, int8_t* xq, float* xd) {
    for (int r = 0; r < rows; ++r)
        for (int b = 0; b < K / 32; ++b) {
            const uint16_t* p = x + (size_t)r * K + 32 * b;
            float amax = 0.0f;
            for (int i = 0; i < 32; ++i) {
                const float a = fabsf(or_half_to_float(p[i]));
                amax = a > amax ? a : amax; /* fmaxf-style: a NaN never wins */
            }
            const float d = amax / 127.0f;
            const float inv = d > 0.0f ? 1.0f / d : 0.0f;
            for (int i = 0; i < 32; ++i) {
                /* __float2int_rn of a NaN product (inf * 0, NaN input) is 0; C leaves
                 * (int) of NaN undefined, so it is spelled out */
                const float y = or_half_to_float(p[i]) * inv;
                int q = isnan(y) ? 0 : (int)nearbyintf(y);
                q = q < -127 ? -127 : (q > 127 ? 127 : q);
                xq[(size_t)r * K + 32 * b + i] = (int8_t)q;
            }
            xd[(size_t)r * (K / 32) + b] = d;
        }
}

/* get_scale_min_k4 (6-bit scale and min of 32-value block j of a Q4_K / Q5_K superblock) */
static void scale_min_k4(int j, const uint8_t* s, int* sc, int* m) {
    if (j < 4) {
        *sc = s[j] & 63;
        *m = s[j + 4] & 63;
    } else {
        *sc = (s[j + 4] & 0xF) | ((s[j - 4] >> 6) << 4);
        *m = (s[j + 4] >> 4) | ((s[j] >> 6) << 4);
    }
}

/* 6-bit signed sub-scale g (0..15) of a Q3_K superblock (12 packed bytes), minus 32 */
static int q3_scale(const uint8_t* s, int g) {
    const int lo = g < 8 ? (s[g] & 0xF) : (s[g - 8] >> 4);
    const int hi = (s[8 + (g & 3)] >> (2 * (g >> 2))) & 3;
    return (lo | (hi << 4)) - 32;
}

int or_kq_block(int kind, const uint8_t* row, int blk, int32_t* q, float* ws, float* wm) {
    /* value v of the block = ws[v/16] * q[v] - wm[v/16] */
    if (kind == KQ80) {
        const uint8_t* b = row + (size_t)blk * 34;
        for (int l = 0; l < 32; ++l) q[l] = (int8_t)b[2 + l];
        ws[0] = ws[1] = h16(b);
        wm[0] = wm[1] = 0.0f;
        return 0;
    }
    const int sb = blk >> 3, j = blk & 7; /* superblock, 32-value block within it */
    if (kind == KQ2) {
        const uint8_t* b = row + (size_t)sb * 84;
        const int h = j >> 2, s = j & 3;
        const float d = h16(b + 80), dmin = h16(b + 82);
        for (int l = 0; l < 32; ++l) q[l] = (b[16 + 32 * h + l] >> (2 * s)) & 3;
        for (int c = 0; c < 2; ++c) {
            const int sc = b[8 * h + 2 * s + c];
            ws[c] = d * (float)(sc & 0xF);
            wm[c] = dmin * (float)(sc >> 4);
        }
    } else if (kind == KQ3) {
        const uint8_t* b = row + (size_t)sb * 110;
        const int h = j >> 2, s = j & 3;
        const float d = h16(b + 108);
        for (int l = 0; l < 32; ++l) {
            const int lo = (b[32 + 32 * h + l] >> (2 * s)) & 3;
            const int hb = (b[l] >> (4 * h + s)) & 1;
            q[l] = (lo | (hb << 2)) - 4;
        }
        for (int c = 0; c < 2; ++c) {
            ws[c] = d * (float)q3_scale(b + 96, 8 * h + 2 * s + c);
            wm[c] = 0.0f;
        }
    } else if (kind == KQ4 || kind == KQ5) {
        const int q5 = kind == KQ5;
        const uint8_t* b = row + (size_t)sb * (q5 ? 176 : 144);
        const int jj = j >> 1, hi = j & 1;
        const uint8_t* qs = b + (q5 ? 48 : 16) + 32 * jj;
        for (int l = 0; l < 32; ++l) {
            int v = hi ? (qs[l] >> 4) : (qs[l] & 0xF);
            if (q5) v |= ((b[16 + l] >> j) & 1) << 4;
            q[l] = v;
        }
        int sc, m;
        scale_min_k4(j, b + 4, &sc, &m);
        ws[0] = ws[1] = h16(b) * (float)sc;
        wm[0] = wm[1] = h16(b + 2) * (float)m;
    } else if (kind == KQ6) {
        const uint8_t* b = row + (size_t)sb * 210;
        const int h = j >> 2, p = j & 3;
        const float d = h16(b + 208);
        for (int l = 0; l < 32; ++l) {
            const uint8_t qlb = b[64 * h + l + 32 * (p & 1)];
            const int lo = p < 2 ? (qlb & 0xF) : (qlb >> 4);
            const int hb = (b[128 + 32 * h + l] >> (2 * p)) & 3;
            q[l] = (lo | (hb << 4)) - 32;
        }
        for (int c = 0; c < 2; ++c) {
            ws[c] = d * (float)(int8_t)b[192 + 8 * h + 2 * p + c];
            wm[c] = 0.0f;
        }
    } else {
        return -1;
    }
    return 0;
}

void or_dequant_row(int kind, const uint8_t* row, int K, float* out) {
    int32_t q[32];
    float ws[2], wm[2];
    for (int blk = 0; blk < K / 32; ++blk) {
        or_kq_block(kind, row, blk, q, ws, wm);
        /* fp32 with each product rounded (contraction off): (d * sc) * q - dmin * m as
         * cpu_kquants.cpp evaluates it left to right; wm = 0 for the kinds without a
         * min, and x - 0 = x */
        for (int l = 0; l < 32; ++l) out[32 * blk + l] = ws[l >> 4] * (float)q[l] - wm[l >> 4];
    }
}

static float clamp_half_range(float r) {
    if (isnan(r)) return 0.0f;
    return fminf(fmaxf(r, -65504.0f), 65504.0f);
}

/* storeY / storeQ8 (prefill_kernels.cu:155-171, hpc_k_quants.cu:422-437) */
static uint16_t store_y(float acc, const float* bias, const uint16_t* res, int n) {
    uint16_t h = or_float_to_half(acc);
    if (bias) {
        float t = or_half_to_float(h), bb = bias[n];
        if (isnan(t)) t = 0.0f;
        if (isnan(bb)) bb = 0.0f;
        h = or_float_to_half(clamp_half_range(t + bb));
    }
    if (res) {
        float t = or_half_to_float(res[n]), a = or_half_to_float(h);
        if (isnan(t)) t = 0.0f;
        if (isnan(a)) a = 0.0f;
        h = or_float_to_half(clamp_half_range(t + a));
    }
    return h;
}

void or_gemm_q8(int kind, const uint8_t* W, const int8_t* xq, const float* xd, int T, int K, int N,
                const float* bias, const uint16_t* res, int ldy, uint16_t* Y, float* yraw) {
    const size_t rb = or_q8_row_bytes(kind, K);
    const int nblk = K / 32;
    const int has_min = kind == KQ2 || kind == KQ4 || kind == KQ5;
    /* the row's blocks decoded once: q [nblk][32], ws/wm [nblk][2] */
    int32_t* q = (int32_t*)malloc(sizeof(int32_t) * (size_t)K);
    float* ws = (float*)malloc(sizeof(float) * 2 * (size_t)nblk);
    float* wm = (float*)malloc(sizeof(float) * 2 * (size_t)nblk);
    for (int n = 0; n < N; ++n) {
        const uint8_t* row = W + (size_t)n * rb;
        for (int b = 0; b < nblk; ++b) or_kq_block(kind, row, b, q + 32 * b, ws + 2 * b, wm + 2 * b);
        for (int t = 0; t < T; ++t) {
            const int8_t* x = xq + (size_t)t * K;
            float acc = 0.0f;
            for (int b = 0; b < nblk; ++b) {
                int dot[2] = {0, 0}, bsum[2] = {0, 0};
                for (int l = 0; l < 32; ++l) {
                    dot[l >> 4] += q[32 * b + l] * x[32 * b + l];
                    bsum[l >> 4] += x[32 * b + l];
                }
                const float dx = xd[(size_t)t * nblk + b];
                /* integer value of the block against its scales: one fp32 product
                 * per 16 values (both halves share ws for the per-32 kinds) */
                acc = fmaf(dx * ws[2 * b], (float)dot[0], acc);
                acc = fmaf(dx * ws[2 * b + 1], (float)dot[1], acc);
                if (has_min) {
                    acc = fmaf(-wm[2 * b], dx * (float)bsum[0], acc);
                    acc = fmaf(-wm[2 * b + 1], dx * (float)bsum[1], acc);
                }
            }
            if (yraw) yraw[(size_t)t * N + n] = acc;
            if (Y) Y[(size_t)t * ldy + n] = store_y(acc, bias, res ? res + (size_t)t * ldy : NULL, n);
        }
    }
    free(q);
    free(ws);
    free(wm);
}
