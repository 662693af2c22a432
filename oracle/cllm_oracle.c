/*
 * cllm_oracle.c -- CPU restatement of cllm_inference's quantized linear-layer path.
 *
 * TEST INFRASTRUCTURE ONLY: the oracle the HIP path is tested against, never the product. See
 * cllm_oracle.h for the reference line each function follows.
 *
 * Arithmetic contract. The reference is built with clang -O3 and default FP contraction, so
 * every "acc += a * b * c" in its vec_dot kernels becomes fma(a * b, c, acc) and every
 * "acc -= a * b * c" becomes fma(-(a * b), c, acc). This file is compiled with
 * -ffp-contract=off and writes those fmaf() calls out explicitly, so its fp32 bits do not
 * depend on the compiler that builds it.
 *
 * How each part is pinned (tests/test_oracle.py):
 *   - dequantize: known-answer blocks restated from the reference's tests
 *     (tests/quant_test.cpp:58-218 cover Q4_0, Q5_0, Q8_0, Q4_K, Q5_K, Q6_K), plus an
 *     element-by-element decode written independently in numpy from the byte layouts.
 *   - quantize_row_q8_0: bit-exact against vectors produced by the reference compiled from
 *     its own sources (tests/golden), and against closed forms: amax = 127 gives d = 1 and
 *     q = rint(x) with ties to even; an all-zero block gives d = 0, q = 0, bsum = 0.
 *   - vec_dot / matmul_quant: bit-exact against the compiled reference on the golden
 *     vectors; against exact integer dots when d = 1, dmin = 0 and every sub-block scale is
 *     1; and against the fp64 evaluation within 1e-5 relative.
 *   - matmul_quant_batch: bit-identical to per-row matmul_quant, and y(bias) - y == bias.
 *   - oracle_matmul_quant_f64 is checked against a brute-force numpy dequantize-and-dot.
 */
#include "cllm_oracle.h"

#include <math.h>
#include <pthread.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

static __thread char g_err[256];

static int fail(int code, const char* msg) {
    snprintf(g_err, sizeof g_err, "%s", msg);
    return code;
}

const char* oracle_last_error(void) { return g_err; }

/* ---- fp16 decode (include/cllm/core/quant.hpp:31-56) ---------------------------------- */
float oracle_half_to_float(uint16_t h) {
    uint32_t sign = (uint32_t)(h >> 15) & 1u;
    uint32_t e = (uint32_t)(h >> 10) & 0x1Fu;
    uint32_t m = (uint32_t)h & 0x3FFu;
    uint32_t bits;
    if (e == 0) {
        if (m == 0) {
            bits = sign << 31;
        } else {
            /* subnormal: normalise the mantissa */
            int ex = 113; /* 127 - 15 + 1 */
            while ((m & 0x400u) == 0) {
                m <<= 1;
                --ex;
            }
            bits = (sign << 31) | ((uint32_t)ex << 23) | ((m & 0x3FFu) << 13);
        }
    } else if (e == 31) {
        bits = (sign << 31) | 0x7F800000u | (m << 13);
    } else {
        bits = (sign << 31) | ((e + 112u) << 23) | (m << 13);
    }
    float f;
    memcpy(&f, &bits, 4);
    return f;
}

static inline float ld_f16(const uint8_t* p) {
    return oracle_half_to_float((uint16_t)(p[0] | (p[1] << 8)));
}

/* ---- sizes (src/core/quant.cpp:340-369) -------------------------------------------------- */
int oracle_block_size(uint32_t t) {
    switch (t) {
        case ORACLE_F32: case ORACLE_F16: return 1;
        case ORACLE_Q4_0: case ORACLE_Q4_1: case ORACLE_Q5_0: case ORACLE_Q5_1:
        case ORACLE_Q8_0: case ORACLE_Q8_1: return 32;
        case ORACLE_Q2_K: case ORACLE_Q3_K: case ORACLE_Q4_K: case ORACLE_Q5_K:
        case ORACLE_Q6_K: return 256;
        default: return 1;
    }
}

size_t oracle_type_size(uint32_t t) {
    switch (t) {
        case ORACLE_F32: return 4;
        case ORACLE_F16: return 2;
        case ORACLE_Q4_0: return 18;
        case ORACLE_Q4_1: return 20;
        case ORACLE_Q5_0: return 22;
        case ORACLE_Q5_1: return 24;
        case ORACLE_Q8_0: return 34;
        case ORACLE_Q8_1: return 36;
        case ORACLE_Q2_K: return 84;
        case ORACLE_Q3_K: return 110;
        case ORACLE_Q4_K: return 144;
        case ORACLE_Q5_K: return 176;
        case ORACLE_Q6_K: return 210;
        default: return 0;
    }
}

int oracle_has_vec_dot(uint32_t t) {
    return t == ORACLE_Q4_0 || t == ORACLE_Q5_0 || t == ORACLE_Q8_0 || t == ORACLE_Q4_K ||
           t == ORACLE_Q5_K || t == ORACLE_Q6_K;
}

/* 6-bit (scale, min) of sub-block j from the 12 packed bytes (src/core/quant.cpp:72-80). */
static inline void scale_min_k4(int j, const uint8_t* q, int* sc, int* m) {
    if (j < 4) {
        *sc = q[j] & 63;
        *m = q[j + 4] & 63;
    } else {
        *sc = (q[j + 4] & 0x0F) | ((q[j - 4] >> 6) << 4);
        *m = (q[j + 4] >> 4) | ((q[j] >> 6) << 4);
    }
}

/* ---- dequantization: the layout oracle ------------------------------------------------- */
static int known_type(uint32_t t) { return oracle_type_size(t) != 0; }

/* 16 signed 6-bit Q3_K scales (value - 32) from the 12 packed bytes: scale i takes its low
 * four bits from byte i (i < 8, low nibble) or byte i - 8 (i >= 8, high nibble) and its top
 * two bits from byte 8 + i % 4, at bit 2 * (i / 4) (src/core/quant.cpp:259-265). */
static void q3_k_scales(const uint8_t* b, int* out) {
    for (int i = 0; i < 16; ++i) {
        const int grp = i / 4, ii = i % 4;
        const int lo = grp < 2 ? (b[4 * grp + ii] & 0x0F) : (b[4 * (grp - 2) + ii] >> 4);
        const int hi = (b[8 + ii] >> (2 * grp)) & 3;
        out[i] = (lo | (hi << 4)) - 32;
    }
}

int oracle_dequantize(const void* src, float* dst, uint32_t t, int64_t n) {
    const uint8_t* s = (const uint8_t*)src;
    const int bs = oracle_block_size(t);
    if (!known_type(t)) return fail(ORACLE_ERR_TYPE, "unsupported ggml type for dequantize");
    if (n % bs != 0) return fail(ORACLE_ERR_SHAPE, "dequantize: n not a multiple of the block size");
    const int64_t nb = n / bs;
    for (int64_t b = 0; b < nb; ++b) {
        float* o = dst + b * bs;
        switch (t) {
            case ORACLE_F32: /* quant.cpp:29-31 */
                memcpy(o, s, 4);
                s += 4;
                break;
            case ORACLE_F16: /* quant.cpp:34-37 */
                o[0] = ld_f16(s);
                s += 2;
                break;
            case ORACLE_Q8_1: { /* [d f16][s f16][qs i8 x32], value = d*q (quant.cpp:203-214) */
                const float d = ld_f16(s);
                for (int j = 0; j < 32; ++j) o[j] = d * (float)(int8_t)s[4 + j];
                s += 36;
                break;
            }
            case ORACLE_Q4_1: { /* [d][m][16 B], value = d*q + m (quant.cpp:164-177) */
                const float d = ld_f16(s), m = ld_f16(s + 2);
                for (int j = 0; j < 16; ++j) {
                    o[j] = d * (float)(s[4 + j] & 0x0F) + m;
                    o[j + 16] = d * (float)(s[4 + j] >> 4) + m;
                }
                s += 20;
                break;
            }
            case ORACLE_Q5_1: { /* [d][m][qh u32 LE][qs 16 B] (quant.cpp:182-200) */
                const float d = ld_f16(s), m = ld_f16(s + 2);
                const uint32_t qh = (uint32_t)s[4] | ((uint32_t)s[5] << 8) |
                                    ((uint32_t)s[6] << 16) | ((uint32_t)s[7] << 24);
                for (int j = 0; j < 16; ++j) {
                    const int q0 = (s[8 + j] & 0x0F) | (int)(((qh >> j) & 1u) << 4);
                    const int q1 = (s[8 + j] >> 4) | (int)(((qh >> (j + 16)) & 1u) << 4);
                    o[j] = d * (float)q0 + m;
                    o[j + 16] = d * (float)q1 + m;
                }
                s += 24;
                break;
            }
            case ORACLE_Q2_K: { /* [scales 16][qs 64][d][dmin] (quant.cpp:218-248) */
                const uint8_t* sc = s;
                const float d = ld_f16(s + 80), dmin = ld_f16(s + 82);
                /* 32-element group u = 4 h + j of half h: qs[32 h + l] >> 2 j, scale bytes
                 * 8 h + 2 j (elements 0-15) and 8 h + 2 j + 1 (16-31) */
                for (int u = 0; u < 8; ++u) {
                    const int h = u / 4, j = u % 4;
                    for (int half16 = 0; half16 < 2; ++half16) {
                        const uint8_t scb = sc[8 * h + 2 * j + half16];
                        const float dl = d * (float)(scb & 0x0F), ml = dmin * (float)(scb >> 4);
                        for (int l = 0; l < 16; ++l) {
                            const int q = (s[16 + 32 * h + 16 * half16 + l] >> (2 * j)) & 3;
                            o[32 * u + 16 * half16 + l] = dl * (float)q - ml;
                        }
                    }
                }
                s += 84;
                break;
            }
            case ORACLE_Q3_K: { /* [hmask 32][qs 64][scales 12][d] (quant.cpp:252-298) */
                int scv[16];
                q3_k_scales(s + 96, scv);
                const float d = ld_f16(s + 108);
                for (int u = 0; u < 8; ++u) {
                    const int h = u / 4, j = u % 4;
                    const int mbit = 1 << (4 * h + j);
                    for (int half16 = 0; half16 < 2; ++half16) {
                        const float dl = d * (float)scv[8 * h + 2 * j + half16];
                        for (int l = 0; l < 16; ++l) {
                            const int e = 16 * half16 + l;
                            const int q = ((s[32 + 32 * h + e] >> (2 * j)) & 3) - ((s[e] & mbit) ? 0 : 4);
                            o[32 * u + e] = dl * (float)q;
                        }
                    }
                }
                s += 110;
                break;
            }
            case ORACLE_Q8_0: { /* [d f16][qs i8 x32], value = d*q */
                const float d = ld_f16(s);
                for (int j = 0; j < 32; ++j) o[j] = d * (float)(int8_t)s[2 + j];
                s += 34;
                break;
            }
            case ORACLE_Q4_0: { /* [d][16 B]: byte j low nibble -> elem j, high -> elem j+16 */
                const float d = ld_f16(s);
                for (int j = 0; j < 16; ++j) {
                    o[j] = d * (float)((s[2 + j] & 0x0F) - 8);
                    o[j + 16] = d * (float)((s[2 + j] >> 4) - 8);
                }
                s += 18;
                break;
            }
            case ORACLE_Q5_0: { /* [d][qh u32 LE][qs 16 B], bit j of qh = bit 4 of elem j */
                const float d = ld_f16(s);
                const uint32_t qh = (uint32_t)s[2] | ((uint32_t)s[3] << 8) |
                                    ((uint32_t)s[4] << 16) | ((uint32_t)s[5] << 24);
                for (int j = 0; j < 16; ++j) {
                    const int q0 = (s[6 + j] & 0x0F) | (int)(((qh >> j) & 1u) << 4);
                    const int q1 = (s[6 + j] >> 4) | (int)(((qh >> (j + 16)) & 1u) << 4);
                    o[j] = d * (float)(q0 - 16);
                    o[j + 16] = d * (float)(q1 - 16);
                }
                s += 22;
                break;
            }
            case ORACLE_Q4_K: { /* [d][dmin][scales 12][qs 128] */
                const float d = ld_f16(s), dmin = ld_f16(s + 2);
                const uint8_t* sc12 = s + 4;
                const uint8_t* q = s + 16;
                for (int c = 0; c < 4; ++c) {
                    int sc, m;
                    scale_min_k4(2 * c, sc12, &sc, &m);
                    const float d1 = d * (float)sc, m1 = dmin * (float)m;
                    scale_min_k4(2 * c + 1, sc12, &sc, &m);
                    const float d2 = d * (float)sc, m2 = dmin * (float)m;
                    for (int l = 0; l < 32; ++l) {
                        o[64 * c + l] = d1 * (float)(q[32 * c + l] & 0x0F) - m1;
                        o[64 * c + 32 + l] = d2 * (float)(q[32 * c + l] >> 4) - m2;
                    }
                }
                s += 144;
                break;
            }
            case ORACLE_Q5_K: { /* [d][dmin][scales 12][qh 32][qs 128] */
                const float d = ld_f16(s), dmin = ld_f16(s + 2);
                const uint8_t* sc12 = s + 4;
                const uint8_t* qh = s + 16;
                const uint8_t* q = s + 48;
                for (int k = 0; k < 8; ++k) {
                    int sc, m;
                    scale_min_k4(k, sc12, &sc, &m);
                    const float dk = d * (float)sc, mk = dmin * (float)m;
                    for (int l = 0; l < 32; ++l) {
                        const uint8_t byte = q[32 * (k / 2) + l];
                        const int lo = (k & 1) ? (byte >> 4) : (byte & 0x0F);
                        const int v = lo | (((qh[l] >> k) & 1) << 4);
                        o[32 * k + l] = dk * (float)v - mk;
                    }
                }
                s += 176;
                break;
            }
            case ORACLE_Q6_K: { /* [ql 128][qh 64][sc i8 x16][d] */
                const uint8_t* ql = s;
                const uint8_t* qh = s + 128;
                const int8_t* sc = (const int8_t*)(s + 192);
                const float d = ld_f16(s + 208);
                for (int g = 0; g < 2; ++g) {
                    for (int l = 0; l < 32; ++l) {
                        const int is = l / 16;
                        const uint8_t a = ql[64 * g + l], b = ql[64 * g + 32 + l], h = qh[32 * g + l];
                        const int q1 = (a & 0x0F) | (((h >> 0) & 3) << 4);
                        const int q2 = (b & 0x0F) | (((h >> 2) & 3) << 4);
                        const int q3 = (a >> 4) | (((h >> 4) & 3) << 4);
                        const int q4 = (b >> 4) | (((h >> 6) & 3) << 4);
                        o[128 * g + l] = d * (float)sc[8 * g + is + 0] * (float)(q1 - 32);
                        o[128 * g + l + 32] = d * (float)sc[8 * g + is + 2] * (float)(q2 - 32);
                        o[128 * g + l + 64] = d * (float)sc[8 * g + is + 4] * (float)(q3 - 32);
                        o[128 * g + l + 96] = d * (float)sc[8 * g + is + 6] * (float)(q4 - 32);
                    }
                }
                s += 210;
                break;
            }
        }
    }
    return ORACLE_OK;
}

/* ---- dequantize_block (src/core/quant.cpp:371-389) ----------------------------------------
 * ceil(n / bs) whole blocks are decoded and the first n elements kept: the reference's deq_*
 * loops read a partial last block whole and guard every store with "< n". */
int oracle_dequantize_block(const void* src, float* dst, uint32_t t, int64_t n) {
    if (!known_type(t)) return fail(ORACLE_ERR_TYPE, "unsupported ggml type for dequantize");
    if (n <= 0) return ORACLE_OK;
    const int64_t bs = oracle_block_size(t), nfull = (n + bs - 1) / bs * bs;
    if (nfull == n) return oracle_dequantize(src, dst, t, n);
    float* tmp = (float*)malloc((size_t)nfull * sizeof(float));
    if (!tmp) return fail(ORACLE_ERR_SYS, "out of memory");
    const int rc = oracle_dequantize(src, tmp, t, nfull);
    if (rc == ORACLE_OK) memcpy(dst, tmp, (size_t)n * sizeof(float));
    free(tmp);
    return rc;
}

/* ---- float_to_half (include/cllm/core/quant.hpp:58-87) ------------------------------------
 * Normal results keep the top ten mantissa bits (no rounding); results below the normal range
 * are rounded to nearest, ties to even; |f| below 2^-25 gives a signed zero, overflow an
 * infinity, NaN the quiet NaN 0x7E00 (with the sign). */
uint16_t oracle_float_to_half(float f) {
    uint32_t x;
    memcpy(&x, &f, 4);
    const uint32_t sign = (x >> 16) & 0x8000u;
    const uint32_t be = (x >> 23) & 0xFFu;
    uint32_t m = x & 0x7FFFFFu;
    const int32_t e = (int32_t)be - 127 + 15;
    if (be == 0xFFu) return (uint16_t)(sign | (m ? 0x7E00u : 0x7C00u));
    if (e >= 31) return (uint16_t)(sign | 0x7C00u);
    if (e >= 1) return (uint16_t)(sign | ((uint32_t)e << 10) | (m >> 13));
    if (e < -10) return (uint16_t)sign;
    m |= 0x800000u;
    const uint32_t sh = (uint32_t)(14 - e);
    const uint32_t bias = (1u << (sh - 1)) - 1u, odd = (m >> sh) & 1u;
    return (uint16_t)(sign | ((m + bias + odd) >> sh));
}

/* ---- dequantize_block_f16 (src/core/quant.cpp:398-407) --------------------------------------
 * F16 blocks are copied as they are; every other type is dequantized to float, then each value
 * goes through float_to_half. */
int oracle_dequantize_block_f16(const void* src, uint16_t* dst, uint32_t t, int64_t n) {
    if (n <= 0) return known_type(t) ? ORACLE_OK : fail(ORACLE_ERR_TYPE, "unsupported ggml type for dequantize");
    if (t == ORACLE_F16) {
        memcpy(dst, src, (size_t)n * 2);
        return ORACLE_OK;
    }
    float* tmp = (float*)malloc((size_t)n * sizeof(float));
    if (!tmp) return fail(ORACLE_ERR_SYS, "out of memory");
    const int rc = oracle_dequantize_block(src, tmp, t, n);
    if (rc == ORACLE_OK)
        for (int64_t i = 0; i < n; ++i) dst[i] = oracle_float_to_half(tmp[i]);
    free(tmp);
    return rc;
}

/* ---- fp32 -> Q8_0 (src/core/quant.cpp:420-452) ------------------------------------------ */
int oracle_quantize_row_q8_0(const float* x, int64_t n, int8_t* qs, float* scales,
                             int32_t* bsums) {
    if (n % 32 != 0) return fail(ORACLE_ERR_SHAPE, "quantize_row_q8_0: n not divisible by 32");
    for (int64_t b = 0; b < n / 32; ++b) {
        const float* xb = x + b * 32;
        float amax = 0.0f;
        for (int j = 0; j < 32; ++j) {
            const float a = fabsf(xb[j]);
            if (a > amax) amax = a;
        }
        const float d = amax / 127.0f;
        const float id = (d != 0.0f) ? 1.0f / d : 0.0f;
        scales[b] = d;
        int32_t sum = 0;
        for (int j = 0; j < 32; ++j) {
            const float v = xb[j] * id;
            int q = (int)nearbyintf(v);
            if (q > 127) q = 127;
            if (q < -128) q = -128;
            qs[b * 32 + j] = (int8_t)q;
            sum += q;
        }
        bsums[b] = sum;
    }
    return ORACLE_OK;
}

/* ---- vec_dot kernels (AVX2 accumulation order) ----------------------------------------- */

static int32_t dot32(const int8_t* a, const int8_t* b) {
    int32_t s = 0;
    for (int j = 0; j < 32; ++j) s += (int32_t)a[j] * (int32_t)b[j];
    return s;
}

/* src/core/quant.cpp:534-547 */
static float vd_q8_0(const uint8_t* w, const int8_t* qs, const float* sc, int64_t n) {
    float acc = 0.0f;
    for (int64_t b = 0; b < n / 32; ++b, w += 34) {
        const float d = ld_f16(w);
        const int32_t dot = dot32((const int8_t*)(w + 2), qs + b * 32);
        acc = fmaf(d * sc[b], (float)dot, acc);
    }
    return acc;
}

/* src/core/quant.cpp:757-777 */
static float vd_q4_0(const uint8_t* w, const int8_t* qs, const float* sc, const int32_t* bsum,
                     int64_t n) {
    float acc = 0.0f;
    for (int64_t b = 0; b < n / 32; ++b, w += 18) {
        const float d = ld_f16(w);
        const int8_t* x = qs + b * 32;
        int32_t dot = 0;
        for (int j = 0; j < 16; ++j) {
            dot += (int32_t)(w[2 + j] & 0x0F) * x[j];
            dot += (int32_t)(w[2 + j] >> 4) * x[j + 16];
        }
        const float inner = fmaf(-8.0f, (float)bsum[b], (float)dot);
        acc = fmaf(d * sc[b], inner, acc);
    }
    return acc;
}

/* src/core/quant.cpp:863-893 */
static float vd_q5_0(const uint8_t* w, const int8_t* qs, const float* sc, const int32_t* bsum,
                     int64_t n) {
    float acc = 0.0f;
    for (int64_t b = 0; b < n / 32; ++b, w += 22) {
        const float d = ld_f16(w);
        const uint32_t qh = (uint32_t)w[2] | ((uint32_t)w[3] << 8) | ((uint32_t)w[4] << 16) |
                            ((uint32_t)w[5] << 24);
        const int8_t* x = qs + b * 32;
        int32_t dot = 0;
        for (int j = 0; j < 16; ++j) {
            const int q0 = (w[6 + j] & 0x0F) | (int)(((qh >> j) & 1u) << 4);
            const int q1 = (w[6 + j] >> 4) | (int)(((qh >> (j + 16)) & 1u) << 4);
            dot += q0 * x[j] + q1 * x[j + 16];
        }
        const float inner = fmaf(-16.0f, (float)bsum[b], (float)dot);
        acc = fmaf(d * sc[b], inner, acc);
    }
    return acc;
}

/* src/core/quant.cpp:549-590 */
static float vd_q4_k(const uint8_t* w, const int8_t* qs, const float* sc, const int32_t* bsum,
                     int64_t n) {
    float acc = 0.0f;
    for (int64_t s = 0; s < n / 256; ++s, w += 144) {
        const float d = ld_f16(w), dmin = ld_f16(w + 2);
        const uint8_t* sc12 = w + 4;
        const uint8_t* q = w + 16;
        for (int c = 0; c < 4; ++c) {
            for (int half = 0; half < 2; ++half) {
                const int k = 2 * c + half;
                int scv, mv;
                scale_min_k4(k, sc12, &scv, &mv);
                const float dk = d * (float)scv, mk = dmin * (float)mv;
                const int64_t b = s * 8 + k;
                const int8_t* x = qs + b * 32;
                int32_t dot = 0;
                for (int l = 0; l < 32; ++l) {
                    const int v = half ? (q[32 * c + l] >> 4) : (q[32 * c + l] & 0x0F);
                    dot += v * x[l];
                }
                acc = fmaf(dk * sc[b], (float)dot, acc);
                acc = fmaf(-(mk * sc[b]), (float)bsum[b], acc);
            }
        }
    }
    return acc;
}

/* src/core/quant.cpp:592-628 */
static float vd_q5_k(const uint8_t* w, const int8_t* qs, const float* sc, const int32_t* bsum,
                     int64_t n) {
    float acc = 0.0f;
    for (int64_t s = 0; s < n / 256; ++s, w += 176) {
        const float d = ld_f16(w), dmin = ld_f16(w + 2);
        const uint8_t* sc12 = w + 4;
        const uint8_t* qh = w + 16;
        const uint8_t* q = w + 48;
        for (int k = 0; k < 8; ++k) {
            int scv, mv;
            scale_min_k4(k, sc12, &scv, &mv);
            const float dk = d * (float)scv, mk = dmin * (float)mv;
            const int64_t b = s * 8 + k;
            const int8_t* x = qs + b * 32;
            int32_t dot = 0;
            for (int l = 0; l < 32; ++l) {
                const uint8_t byte = q[32 * (k / 2) + l];
                const int lo = (k & 1) ? (byte >> 4) : (byte & 0x0F);
                dot += (lo | (((qh[l] >> k) & 1) << 4)) * x[l];
            }
            acc = fmaf(dk * sc[b], (float)dot, acc);
            acc = fmaf(-(mk * sc[b]), (float)bsum[b], acc);
        }
    }
    return acc;
}

/* src/core/quant.cpp:630-687. Two 16-element halves per activation block, one int8 scale
 * each; the bracket sc_a*dot_a + sc_b*dot_b is an exact integer in fp32. */
static float vd_q6_k(const uint8_t* w, const int8_t* qs, const float* sc, int64_t n) {
    float acc = 0.0f;
    for (int64_t s = 0; s < n / 256; ++s, w += 210) {
        const uint8_t* ql = w;
        const uint8_t* qh = w + 128;
        const int8_t* scs = (const int8_t*)(w + 192);
        const float d = ld_f16(w + 208);
        for (int g = 0; g < 2; ++g) {
            for (int i = 0; i < 4; ++i) {
                const int64_t b = s * 8 + 4 * g + i;
                const int8_t* x = qs + b * 32;
                int32_t dot_a = 0, dot_b = 0;
                for (int l = 0; l < 32; ++l) {
                    const uint8_t lb = ql[64 * g + 32 * (i & 1) + l];
                    const int lo = (i < 2) ? (lb & 0x0F) : (lb >> 4);
                    const int hi = (qh[32 * g + l] >> (2 * i)) & 3;
                    const int v = (lo | (hi << 4)) - 32;
                    if (l < 16) dot_a += v * x[l];
                    else dot_b += v * x[l];
                }
                const float sa = (float)scs[8 * g + 2 * i], sb = (float)scs[8 * g + 2 * i + 1];
                const float inner = fmaf(sa, (float)dot_a, sb * (float)dot_b);
                acc = fmaf(d * sc[b], inner, acc);
            }
        }
    }
    return acc;
}

static float vec_dot_dispatch(const uint8_t* w, uint32_t t, const int8_t* qs, const float* sc,
                              const int32_t* bsum, int64_t n) {
    switch (t) {
        case ORACLE_Q4_0: return vd_q4_0(w, qs, sc, bsum, n);
        case ORACLE_Q5_0: return vd_q5_0(w, qs, sc, bsum, n);
        case ORACLE_Q8_0: return vd_q8_0(w, qs, sc, n);
        case ORACLE_Q4_K: return vd_q4_k(w, qs, sc, bsum, n);
        case ORACLE_Q5_K: return vd_q5_k(w, qs, sc, bsum, n);
        case ORACLE_Q6_K: return vd_q6_k(w, qs, sc, n);
        default: return 0.0f;
    }
}

int oracle_vec_dot_row(const void* w_row, uint32_t t, const int8_t* qs, const float* scales,
                       const int32_t* bsums, int64_t n, float* out) {
    if (!oracle_has_vec_dot(t)) return fail(ORACLE_ERR_TYPE, "vec_dot_row: no kernel for this type");
    *out = vec_dot_dispatch((const uint8_t*)w_row, t, qs, scales, bsums, n);
    return ORACLE_OK;
}

/* ---- row-parallel driver (src/core/thread_pool.cpp:44-89 chunking) --------------------- */

typedef struct {
    const uint8_t* w;
    uint32_t type;
    size_t row_bytes;
    int in_dim, out_dim, n_rows;
    const int8_t* qs;
    const float* sc;
    const int32_t* bs;
    const float* bias;
    float* y;
    size_t j0, j1;
    const float* x;  /* fp32 activations (types without vec_dot) */
    float* buf;      /* per-job dequantization chunk (types without vec_dot) */
} job_t;

/* Types without a vec_dot kernel (src/core/quant.cpp:1404-1430): the row is dequantized in
 * chunks of (512 / bs) * bs elements and accumulated in order into acc, which starts at the
 * bias; clang contracts "acc += xp[i] * buf[i]" into one fma per element. */
static void run_rows_float(const job_t* jb) {
    const int bs = oracle_block_size(jb->type);
    const int chunk = (512 / bs) * bs;
    const size_t ts = oracle_type_size(jb->type);
    for (size_t j = jb->j0; j < jb->j1; ++j) {
        const uint8_t* rp = jb->w + j * jb->row_bytes;
        for (int t = 0; t < jb->n_rows; ++t) {
            const float* x = jb->x + (size_t)t * jb->in_dim;
            float acc = jb->bias ? jb->bias[j] : 0.0f;
            for (int off = 0; off < jb->in_dim; off += chunk) {
                const int len = jb->in_dim - off < chunk ? jb->in_dim - off : chunk;
                oracle_dequantize(rp + (size_t)(off / bs) * ts, jb->buf, jb->type, len);
                for (int i = 0; i < len; ++i) acc = fmaf(x[off + i], jb->buf[i], acc);
            }
            jb->y[(size_t)t * jb->out_dim + j] = acc;
        }
    }
}

static void run_rows(const job_t* jb) {
    if (jb->x) {
        run_rows_float(jb);
        return;
    }
    const int nb = jb->in_dim / 32;
    for (size_t j = jb->j0; j < jb->j1; ++j) {
        const uint8_t* rp = jb->w + j * jb->row_bytes;
        for (int t = 0; t < jb->n_rows; ++t) {
            float acc = vec_dot_dispatch(rp, jb->type, jb->qs + (size_t)t * jb->in_dim,
                                         jb->sc + (size_t)t * nb, jb->bs + (size_t)t * nb,
                                         jb->in_dim);
            if (jb->bias) acc += jb->bias[j];
            jb->y[(size_t)t * jb->out_dim + j] = acc;
        }
    }
}

static void* run_rows_thread(void* p) {
    run_rows((const job_t*)p);
    return NULL;
}

static int run_all(job_t base, int n_threads) {
    const size_t total = (size_t)base.out_dim;
    const int chunk_floats = 512;
    if (n_threads <= 1 || base.out_dim < 256) {
        base.j0 = 0;
        base.j1 = total;
        float* buf = base.x ? (float*)malloc(sizeof(float) * chunk_floats) : NULL;
        if (base.x && !buf) return fail(ORACLE_ERR_SYS, "out of memory");
        base.buf = buf;
        run_rows(&base);
        free(buf);
        return ORACLE_OK;
    }
    /* chunk = ceil(total / workers); one task per chunk */
    const size_t chunk = (total + (size_t)n_threads - 1) / (size_t)n_threads;
    const size_t n_chunks = (total + chunk - 1) / chunk;
    job_t* jobs = (job_t*)calloc(n_chunks, sizeof(job_t));
    pthread_t* th = (pthread_t*)calloc(n_chunks, sizeof(pthread_t));
    float* bufs = base.x ? (float*)malloc(sizeof(float) * chunk_floats * n_chunks) : NULL;
    if (!jobs || !th || (base.x && !bufs)) {
        free(jobs);
        free(th);
        free(bufs);
        return fail(ORACLE_ERR_SYS, "out of memory");
    }
    for (size_t c = 0; c < n_chunks; ++c) {
        jobs[c] = base;
        jobs[c].j0 = c * chunk;
        jobs[c].j1 = (c + 1) * chunk < total ? (c + 1) * chunk : total;
        jobs[c].buf = bufs ? bufs + c * chunk_floats : NULL;
        pthread_create(&th[c], NULL, run_rows_thread, &jobs[c]);
    }
    for (size_t c = 0; c < n_chunks; ++c) pthread_join(th[c], NULL);
    free(jobs);
    free(th);
    free(bufs);
    return ORACLE_OK;
}

static int quantize_rows(const float* x, int in_dim, int n_rows, int8_t** qs, float** sc,
                         int32_t** bs) {
    const size_t nb = (size_t)in_dim / 32;
    *qs = (int8_t*)malloc((size_t)n_rows * in_dim);
    *sc = (float*)malloc((size_t)n_rows * nb * sizeof(float));
    *bs = (int32_t*)malloc((size_t)n_rows * nb * sizeof(int32_t));
    if (!*qs || !*sc || !*bs) return fail(ORACLE_ERR_SYS, "out of memory");
    for (int t = 0; t < n_rows; ++t) {
        int rc = oracle_quantize_row_q8_0(x + (size_t)t * in_dim, in_dim, *qs + (size_t)t * in_dim,
                                          *sc + (size_t)t * nb, *bs + (size_t)t * nb);
        if (rc) return rc;
    }
    return ORACLE_OK;
}

static int matmul_impl(const char* who, const float* x, const void* w, uint32_t type,
                       const float* bias, int in_dim, int out_dim, int n_rows, float* y,
                       int n_threads) {
    char msg[128];
    const int bs = oracle_block_size(type);
    if (bs <= 0 || in_dim % bs != 0) {
        snprintf(msg, sizeof msg, "%s: in_dim not divisible by block size", who);
        return fail(ORACLE_ERR_SHAPE, msg);
    }
    if (!oracle_has_vec_dot(type)) {
        /* quant.cpp:1404-1430 (matmul_quant_batch runs it row by row, 1471-1474) */
        if (!known_type(type)) {
            if (out_dim > 0 && in_dim > 0)
                return fail(ORACLE_ERR_TYPE, "unsupported ggml type for dequantize");
            return ORACLE_OK;
        }
        job_t jb;
        memset(&jb, 0, sizeof jb);
        jb.w = (const uint8_t*)w;
        jb.type = type;
        jb.row_bytes = (size_t)(in_dim / bs) * oracle_type_size(type);
        jb.in_dim = in_dim;
        jb.out_dim = out_dim;
        jb.n_rows = n_rows;
        jb.bias = bias;
        jb.y = y;
        jb.x = x;
        return run_all(jb, n_threads);
    }
    int8_t* qs = NULL;
    float* sc = NULL;
    int32_t* bsum = NULL;
    int rc = quantize_rows(x, in_dim, n_rows, &qs, &sc, &bsum);
    if (rc == ORACLE_OK) {
        job_t jb;
        memset(&jb, 0, sizeof jb);
        jb.w = (const uint8_t*)w;
        jb.type = type;
        jb.row_bytes = (size_t)(in_dim / bs) * oracle_type_size(type);
        jb.in_dim = in_dim;
        jb.out_dim = out_dim;
        jb.n_rows = n_rows;
        jb.qs = qs;
        jb.sc = sc;
        jb.bs = bsum;
        jb.bias = bias;
        jb.y = y;
        rc = run_all(jb, n_threads);
    }
    free(qs);
    free(sc);
    free(bsum);
    return rc;
}

int oracle_matmul_quant(const float* x, const void* w, uint32_t type, const float* bias,
                        int in_dim, int out_dim, float* y, int n_threads) {
    return matmul_impl("matmul_quant", x, w, type, bias, in_dim, out_dim, 1, y, n_threads);
}

int oracle_matmul_quant_batch(const float* x, const void* w, uint32_t type, const float* bias,
                              int in_dim, int out_dim, int n_rows, float* y, int n_threads) {
    if (n_rows <= 0) return ORACLE_OK; /* quant.cpp:1436: returns without touching y */
    if (n_rows == 1) return oracle_matmul_quant(x, w, type, bias, in_dim, out_dim, y, n_threads);
    return matmul_impl("matmul_quant_batch", x, w, type, bias, in_dim, out_dim, n_rows, y,
                       n_threads);
}

/* ---- fp64 evaluation of the same per-block terms -------------------------------------- */

/* Per-block weight terms for row rp: ws[b] (multiplies dx*dot) and wm[b] (multiplies
 * dx*bsum), plus the exact integer dots against activation row x. For Q6_K the integer is
 * sc_a*dot_a + sc_b*dot_b and ws = d. */
static void block_terms(const uint8_t* rp, uint32_t t, const int8_t* x, int nb, double* ws,
                        double* wm, int64_t* idot) {
    const int bs = oracle_block_size(t);
    const size_t ts = oracle_type_size(t);
    for (int wb = 0; wb < nb * 32 / bs; ++wb) {
        const uint8_t* blk = rp + (size_t)wb * ts;
        if (t == ORACLE_Q8_0 || t == ORACLE_Q4_0 || t == ORACLE_Q5_0) {
            const int b = wb;
            const double d = ld_f16(blk);
            int64_t dot = 0;
            for (int j = 0; j < 32; ++j) {
                int v;
                if (t == ORACLE_Q8_0) {
                    v = (int8_t)blk[2 + j];
                } else if (t == ORACLE_Q4_0) {
                    v = (j < 16 ? (blk[2 + j] & 0x0F) : (blk[2 + j - 16] >> 4)) - 8;
                } else {
                    const uint32_t qh = (uint32_t)blk[2] | ((uint32_t)blk[3] << 8) |
                                        ((uint32_t)blk[4] << 16) | ((uint32_t)blk[5] << 24);
                    const int lo = j < 16 ? (blk[6 + j] & 0x0F) : (blk[6 + j - 16] >> 4);
                    v = (lo | (int)(((qh >> j) & 1u) << 4)) - 16;
                }
                dot += (int64_t)v * x[b * 32 + j];
            }
            ws[b] = d;
            wm[b] = 0.0;
            idot[b] = dot;
        } else if (t == ORACLE_Q4_K || t == ORACLE_Q5_K) {
            const double d = ld_f16(blk), dmin = ld_f16(blk + 2);
            const uint8_t* sc12 = blk + 4;
            for (int k = 0; k < 8; ++k) {
                const int b = wb * 8 + k;
                int scv, mv;
                scale_min_k4(k, sc12, &scv, &mv);
                int64_t dot = 0;
                for (int l = 0; l < 32; ++l) {
                    int v;
                    if (t == ORACLE_Q4_K) {
                        const uint8_t byte = blk[16 + 32 * (k / 2) + l];
                        v = (k & 1) ? (byte >> 4) : (byte & 0x0F);
                    } else {
                        const uint8_t byte = blk[48 + 32 * (k / 2) + l];
                        v = ((k & 1) ? (byte >> 4) : (byte & 0x0F)) | (((blk[16 + l] >> k) & 1) << 4);
                    }
                    dot += (int64_t)v * x[b * 32 + l];
                }
                ws[b] = d * scv;
                wm[b] = dmin * mv;
                idot[b] = dot;
            }
        } else { /* Q6_K */
            const double d = ld_f16(blk + 208);
            const int8_t* scs = (const int8_t*)(blk + 192);
            for (int g = 0; g < 2; ++g) {
                for (int i = 0; i < 4; ++i) {
                    const int b = wb * 8 + 4 * g + i;
                    int64_t dot_a = 0, dot_b = 0;
                    for (int l = 0; l < 32; ++l) {
                        const uint8_t lb = blk[64 * g + 32 * (i & 1) + l];
                        const int lo = (i < 2) ? (lb & 0x0F) : (lb >> 4);
                        const int hi = (blk[128 + 32 * g + l] >> (2 * i)) & 3;
                        const int v = (lo | (hi << 4)) - 32;
                        if (l < 16) dot_a += (int64_t)v * x[b * 32 + l];
                        else dot_b += (int64_t)v * x[b * 32 + l];
                    }
                    ws[b] = d;
                    wm[b] = 0.0;
                    idot[b] = (int64_t)scs[8 * g + 2 * i] * dot_a + (int64_t)scs[8 * g + 2 * i + 1] * dot_b;
                }
            }
        }
    }
}

int oracle_matmul_quant_f64(const float* x, const void* w, uint32_t type, const float* bias,
                            int in_dim, int out_dim, int n_rows, double* y, double* abs_sum) {
    const int bs = oracle_block_size(type);
    if (bs <= 0 || in_dim % bs != 0) return fail(ORACLE_ERR_SHAPE, "matmul_quant: in_dim not divisible by block size");
    if (!known_type(type)) return fail(ORACLE_ERR_TYPE, "unsupported ggml type for dequantize");
    if (n_rows <= 0) return ORACLE_OK;
    if (!oracle_has_vec_dot(type)) {
        /* dequantized fp32 weights times fp32 activations, summed exactly in fp64 */
        const size_t rb = (size_t)(in_dim / bs) * oracle_type_size(type);
        float* wrow = (float*)malloc(sizeof(float) * (size_t)in_dim);
        if (!wrow) return fail(ORACLE_ERR_SYS, "out of memory");
        for (int j = 0; j < out_dim; ++j) {
            oracle_dequantize((const uint8_t*)w + (size_t)j * rb, wrow, type, in_dim);
            for (int t = 0; t < n_rows; ++t) {
                const float* xt = x + (size_t)t * in_dim;
                double acc = bias ? (double)bias[j] : 0.0, aab = bias ? fabs((double)bias[j]) : 0.0;
                for (int i = 0; i < in_dim; ++i) {
                    const double p = (double)xt[i] * (double)wrow[i];
                    acc += p;
                    aab += fabs(p);
                }
                y[(size_t)t * out_dim + j] = acc;
                if (abs_sum) abs_sum[(size_t)t * out_dim + j] = aab;
            }
        }
        free(wrow);
        return ORACLE_OK;
    }
    int8_t* qs = NULL;
    float* sc = NULL;
    int32_t* bsum = NULL;
    int rc = quantize_rows(x, in_dim, n_rows, &qs, &sc, &bsum);
    const int nb = in_dim / 32;
    double* ws = (double*)malloc(sizeof(double) * nb);
    double* wm = (double*)malloc(sizeof(double) * nb);
    int64_t* idot = (int64_t*)malloc(sizeof(int64_t) * nb);
    if (rc == ORACLE_OK && (!ws || !wm || !idot)) rc = fail(ORACLE_ERR_SYS, "out of memory");
    const size_t row_bytes = (size_t)(in_dim / bs) * oracle_type_size(type);
    for (int t = 0; rc == ORACLE_OK && t < n_rows; ++t) {
        const int8_t* xq = qs + (size_t)t * in_dim;
        const float* xs = sc + (size_t)t * nb;
        const int32_t* xb = bsum + (size_t)t * nb;
        for (int j = 0; j < out_dim; ++j) {
            block_terms((const uint8_t*)w + (size_t)j * row_bytes, type, xq, nb, ws, wm, idot);
            double acc = 0.0, aab = 0.0;
            for (int b = 0; b < nb; ++b) {
                double main_t = ws[b] * (double)xs[b] * (double)idot[b];
                /* Q4_0/Q5_0 fold their -8/-16 offset into idot (one exact bracket, as
                 * quant.cpp:775 and 891 do), so only the K-quants carry a min term. */
                const double min_t = wm[b] * (double)xs[b] * (double)xb[b];
                acc += main_t - min_t;
                aab += fabs(main_t) + fabs(min_t);
            }
            if (bias) {
                acc += bias[j];
                aab += fabs((double)bias[j]);
            }
            y[(size_t)t * out_dim + j] = acc;
            if (abs_sum) abs_sum[(size_t)t * out_dim + j] = aab;
        }
    }
    free(ws);
    free(wm);
    free(idot);
    free(qs);
    free(sc);
    free(bsum);
    return rc;
}

/* ---- producers of the linear layers' activations (src/core/engine.cpp) ----------------- */

/* rms_norm_ptr (engine.cpp:23-28) on each of `rows` rows: a sequential sum of squares, which
 * clang contracts into one fma per element, then rms = 1 / sqrt(sum / n + eps) and
 * out = (x * rms) * w. */
int oracle_rms_norm(const float* x, const float* w, int n, int rows, float eps, float* out) {
    if (n <= 0 || rows < 0) return fail(ORACLE_ERR_SHAPE, "rms_norm: bad shape");
    for (int r = 0; r < rows; ++r) {
        const float* xr = x + (size_t)r * n;
        float* o = out + (size_t)r * n;
        float sum = 0.0f;
        for (int i = 0; i < n; ++i) sum = fmaf(xr[i], xr[i], sum);
        const float rms = 1.0f / sqrtf(sum / (float)n + eps);
        for (int i = 0; i < n; ++i) o[i] = xr[i] * rms * w[i];
    }
    return ORACLE_OK;
}

/* silu(gate) * up element-wise, silu(v) = v / (1 + exp(-v)) (engine.cpp:38, 511, 596). */
int oracle_swiglu(const float* gate, const float* up, int64_t n, float* out) {
    for (int64_t i = 0; i < n; ++i) out[i] = gate[i] / (1.0f + expf(-gate[i])) * up[i];
    return ORACLE_OK;
}
