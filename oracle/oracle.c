/*
 * oracle.c -- CPU restatement of the dual-precision MoE expert FFN path.
 *
 * TEST INFRASTRUCTURE ONLY (see oracle.h).  Compiled with -ffp-contract=off so
 * that every float expression rounds the way the written C does.
 */
#include "oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

/* ------------------------------------------------------------------ fp16 */

float orc_fp16_to_fp32(uint16_t h) {
    const uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    const uint32_t exp  = (h >> 10) & 0x1f;
    const uint32_t man  = h & 0x3ff;
    uint32_t bits;
    if (exp == 0) {
        if (man == 0) {
            bits = sign;
        } else {                       /* subnormal: value = man * 2^-24 */
            float f = (float)man * 5.9604644775390625e-8f;
            memcpy(&bits, &f, 4);
            bits |= sign;
        }
    } else if (exp == 31) {
        bits = sign | 0x7f800000u | (man << 13);
    } else {
        bits = sign | ((exp + 112) << 23) | (man << 13);
    }
    float out;
    memcpy(&out, &bits, 4);
    return out;
}

/* IEEE binary16 conversion, round to nearest even (the behaviour of F16C
 * vcvtps2ph and of ggml's software fallback). */
uint16_t orc_fp32_to_fp16(float f) {
    uint32_t x;
    memcpy(&x, &f, 4);
    const uint32_t sign = (x >> 16) & 0x8000u;
    const uint32_t ax = x & 0x7fffffffu;
    if (ax >= 0x7f800000u) {                       /* inf / nan */
        return (uint16_t)(sign | 0x7c00u | (ax > 0x7f800000u ? 0x200u : 0));
    }
    if (ax >= 0x477ff000u) {                       /* rounds to >= 65520 -> inf */
        return (uint16_t)(sign | 0x7c00u);
    }
    if (ax < 0x38800000u) {                        /* below min normal half */
        /* value = ax as float; half subnormal unit = 2^-24 */
        float a;
        memcpy(&a, &ax, 4);
        float q = a * 16777216.0f;                 /* exact scaling by 2^24 */
        float r = rintf(q);                        /* RNE in default mode */
        return (uint16_t)(sign | (uint32_t)r);
    }
    /* normal: keep 10 mantissa bits, RNE on the 13 dropped bits */
    uint32_t e = ((ax >> 23) - 112) << 10;
    uint32_t m = (ax >> 13) & 0x3ff;
    uint32_t rest = ax & 0x1fff;
    uint32_t h = e | m;
    if (rest > 0x1000u || (rest == 0x1000u && (m & 1))) h += 1;
    return (uint16_t)(sign | h);
}

/* --------------------------------------------------------------- formats */

#define QK_K 256
typedef struct { uint16_t d, dmin; uint8_t scales[12]; uint8_t qs[128]; } blk_q4_K;      /* 144 B */
typedef struct { uint16_t d; uint8_t qs[64]; uint8_t qh[8]; uint8_t scales[8]; } blk_iq2_s; /* 82 B */
typedef struct { uint16_t d; uint8_t qh[4]; uint8_t qs[16]; } blk_q5_0;                      /* 22 B */
typedef struct { uint16_t d; uint8_t qs[16]; } blk_iq4_nl;                                   /* 18 B */
typedef struct { float d; int8_t qs[QK_K]; int16_t bsums[16]; } blk_q8_K;                    /* 292 B */
typedef struct { uint16_t d; int8_t qs[32]; } blk_q8_0;                                      /* 34 B */
typedef struct { uint16_t d, s; int8_t qs[32]; } blk_q8_1;                                   /* 36 B */

_Static_assert(sizeof(blk_q4_K) == 144, "q4_K");
_Static_assert(sizeof(blk_iq2_s) == 82, "iq2_s");
_Static_assert(sizeof(blk_q5_0) == 22, "q5_0");
_Static_assert(sizeof(blk_iq4_nl) == 18, "iq4_nl");
_Static_assert(sizeof(blk_q8_K) == 292, "q8_K");
_Static_assert(sizeof(blk_q8_0) == 34, "q8_0");
_Static_assert(sizeof(blk_q8_1) == 36, "q8_1");

static const uint16_t iq2s_codes[1024] = {
#include "../llapis_amd/csrc/iq2s_grid.inc"
};

/* the IQ4_NL non-linear levels (ggml-common.h:1110) */
static const int8_t iq4nl_values[16] = {
    -127, -104, -83, -65, -49, -35, -22, -10, 1, 13, 25, 38, 53, 69, 89, 113,
};

/* dequantised IQ2_S codebook byte j of entry k */
static inline int iq2s_grid_byte(int k, int j) {
    static const uint8_t lv[3] = {0x08, 0x19, 0x2b};
    return lv[(iq2s_codes[k] >> (2 * j)) & 3];
}

size_t orc_row_size(int type, int64_t n) {
    switch (type) {
        case ORC_F32:    return (size_t)n * 4;
        case ORC_Q4_K:   return (size_t)(n / QK_K) * sizeof(blk_q4_K);
        case ORC_IQ2_S:  return (size_t)(n / QK_K) * sizeof(blk_iq2_s);
        case ORC_Q5_0:   return (size_t)(n / 32) * sizeof(blk_q5_0);
        case ORC_IQ4_NL: return (size_t)(n / 32) * sizeof(blk_iq4_nl);
        case ORC_Q8_K:   return (size_t)(n / QK_K) * sizeof(blk_q8_K);
        case ORC_Q8_0:   return (size_t)(n / 32) * sizeof(blk_q8_0);
        case ORC_Q8_1:   return (size_t)(n / 32) * sizeof(blk_q8_1);
        default:         abort();
    }
}

/* 6-bit scale / min j of a Q4_K super-block (ggml-quants.c:822-829) */
static inline void q4k_scale_min(int j, const uint8_t * q, int * sc, int * m) {
    if (j < 4) {
        *sc = q[j] & 63;
        *m  = q[j + 4] & 63;
    } else {
        *sc = (q[j + 4] & 0xF) | ((q[j - 4] >> 6) << 4);
        *m  = (q[j + 4] >> 4) | ((q[j] >> 6) << 4);
    }
}

/* ---------------------------------------------------------- dequantise */

void orc_dequantize(int type, const void * vx, float * y, int64_t k) {
    if (type == ORC_Q4_K) {
        const blk_q4_K * x = vx;
        for (int64_t i = 0; i < k / QK_K; ++i) {
            const float d = orc_fp16_to_fp32(x[i].d), mn = orc_fp16_to_fp32(x[i].dmin);
            const uint8_t * q = x[i].qs;
            for (int j = 0; j < 4; ++j) {       /* 64 values per 32 qs bytes */
                int sc, m;
                q4k_scale_min(2 * j, x[i].scales, &sc, &m);
                const float d1 = d * sc, m1 = mn * m;
                q4k_scale_min(2 * j + 1, x[i].scales, &sc, &m);
                const float d2 = d * sc, m2 = mn * m;
                for (int l = 0; l < 32; ++l) *y++ = d1 * (q[l] & 0xF) - m1;
                for (int l = 0; l < 32; ++l) *y++ = d2 * (q[l] >> 4) - m2;
                q += 32;
            }
        }
    } else if (type == ORC_IQ2_S) {
        const blk_iq2_s * x = vx;
        for (int64_t i = 0; i < k / QK_K; ++i) {
            const float d = orc_fp16_to_fp32(x[i].d);
            for (int ib = 0; ib < 8; ++ib) {
                const float db0 = d * (0.5f + (x[i].scales[ib] & 0xf)) * 0.25f;
                const float db1 = d * (0.5f + (x[i].scales[ib] >> 4)) * 0.25f;
                for (int l = 0; l < 4; ++l) {
                    const float dl = l < 2 ? db0 : db1;
                    const int g = x[i].qs[4 * ib + l] | (((x[i].qh[ib] >> (2 * l)) & 3) << 8);
                    const uint8_t sg = x[i].qs[32 + 4 * ib + l];
                    for (int j = 0; j < 8; ++j)
                        *y++ = dl * iq2s_grid_byte(g, j) * ((sg >> j) & 1 ? -1.f : 1.f);
                }
            }
        }
    } else if (type == ORC_Q5_0) {
        const blk_q5_0 * x = vx;
        for (int64_t i = 0; i < k / 32; ++i) {
            const float d = orc_fp16_to_fp32(x[i].d);
            uint32_t qh;
            memcpy(&qh, x[i].qh, 4);
            for (int j = 0; j < 16; ++j) {
                const int x0 = ((x[i].qs[j] & 0x0F) | (((qh >> j) & 1) << 4)) - 16;
                const int x1 = ((x[i].qs[j] >> 4) | (((qh >> (j + 16)) & 1) << 4)) - 16;
                y[j] = x0 * d;
                y[j + 16] = x1 * d;
            }
            y += 32;
        }
    } else if (type == ORC_IQ4_NL) {
        const blk_iq4_nl * x = vx;
        for (int64_t i = 0; i < k / 32; ++i) {
            const float d = orc_fp16_to_fp32(x[i].d);
            for (int j = 0; j < 16; ++j) {
                y[j] = d * iq4nl_values[x[i].qs[j] & 0xf];
                y[j + 16] = d * iq4nl_values[x[i].qs[j] >> 4];
            }
            y += 32;
        }
    } else {
        abort();
    }
}

/* ------------------------------------------------- activation quantisers */

static void quant_q8_K(const float * x, blk_q8_K * y, int64_t k) {
    for (int64_t i = 0; i < k / QK_K; ++i, x += QK_K) {
        float max = 0, amax = 0;
        for (int j = 0; j < QK_K; ++j) {
            const float ax = fabsf(x[j]);
            if (ax > amax) { amax = ax; max = x[j]; }
        }
        if (!amax) {
            memset(&y[i], 0, sizeof(blk_q8_K));
            continue;
        }
        const float iscale = -127.f / max;
        for (int j = 0; j < QK_K; ++j) {
            int v = (int)rintf(iscale * x[j]);    /* nearest_int: RNE */
            y[i].qs[j] = (int8_t)(v < 127 ? v : 127);
        }
        for (int j = 0; j < 16; ++j) {
            int s = 0;
            for (int l = 0; l < 16; ++l) s += y[i].qs[16 * j + l];
            y[i].bsums[j] = (int16_t)s;
        }
        y[i].d = 1 / iscale;
    }
}

static void quant_q8_0_x86(const float * x, blk_q8_0 * y, int64_t k) {
    for (int64_t i = 0; i < k / 32; ++i, x += 32) {
        float amax = 0;
        for (int j = 0; j < 32; ++j) amax = fmaxf(amax, fabsf(x[j]));
        const float d = amax / 127.f;
        y[i].d = orc_fp32_to_fp16(d);
        const float id = amax != 0.0f ? 127.f / amax : 0.0f;
        for (int j = 0; j < 32; ++j) y[i].qs[j] = (int8_t)rintf(x[j] * id);
    }
}

static void quant_q8_1_gpu(const float * x, blk_q8_1 * y, int64_t k) {
    for (int64_t i = 0; i < k / 32; ++i, x += 32) {
        float amax = 0;
        for (int j = 0; j < 32; ++j) amax = fmaxf(amax, fabsf(x[j]));
        /* the device sums with a butterfly (xor 16, 8, 4, 2, 1) */
        float s[32];
        for (int j = 0; j < 32; ++j) s[j] = x[j];
        for (int off = 16; off >= 1; off >>= 1) {
            float t[32];
            for (int j = 0; j < 32; ++j) t[j] = s[j] + s[j ^ off];
            memcpy(s, t, sizeof(s));
        }
        const float d = amax / 127.0f;
        for (int j = 0; j < 32; ++j) y[i].qs[j] = (int8_t)(amax == 0.0f ? 0 : roundf(x[j] / d));
        y[i].d = orc_fp32_to_fp16(d);
        y[i].s = orc_fp32_to_fp16(s[0]);
    }
}

void orc_quantize_act(int act_type, const float * x, void * y, int64_t k) {
    switch (act_type) {
        case ORC_Q8_K: quant_q8_K(x, y, k); break;
        case ORC_Q8_0: quant_q8_0_x86(x, y, k); break;
        case ORC_Q8_1: quant_q8_1_gpu(x, y, k); break;
        default: abort();
    }
}

int orc_act_type(int wtype, int act_mode) {
    if (act_mode == ORC_ACT_Q8_1 || act_mode == ORC_ACT_Q8_1_MMA) return ORC_Q8_1;
    return (wtype == ORC_Q4_K || wtype == ORC_IQ2_S) ? ORC_Q8_K : ORC_Q8_0;
}

/* ------------------------------------------------------------- vec_dot */

static float dot_q4_K_q8_K(int64_t n, const blk_q4_K * x, const blk_q8_K * y) {
    float sums[8] = {0};
    float sumf = 0;
    for (int64_t i = 0; i < n / QK_K; ++i) {
        int sc[8], mn[8];
        for (int j = 0; j < 8; ++j) q4k_scale_min(j, x[i].scales, &sc[j], &mn[j]);
        int summ = 0;
        for (int j = 0; j < 16; ++j) summ += y[i].bsums[j] * mn[j / 2];
        /* aux32[l] accumulates lane l (of 8) of every 8-wide chunk, as the
         * generic kernel does; the integer result is order-free. */
        int32_t aux32[8] = {0};
        for (int j = 0; j < 8; ++j) {            /* sub-block of 32 */
            const uint8_t * q4 = x[i].qs + 32 * (j / 2);
            const int shift = (j & 1) ? 4 : 0;
            for (int l = 0; l < 32; ++l) {
                const int a = (q4[l] >> shift) & 0xF;
                aux32[l % 8] += sc[j] * (a * y[i].qs[32 * j + l]);
            }
        }
        const float d = orc_fp16_to_fp32(x[i].d) * y[i].d;
        for (int l = 0; l < 8; ++l) sums[l] += d * aux32[l];
        const float dmin = orc_fp16_to_fp32(x[i].dmin) * y[i].d;
        sumf -= dmin * summ;
    }
    for (int l = 0; l < 8; ++l) sumf += sums[l];
    return sumf;
}

static float dot_iq2_s_q8_K(int64_t n, const blk_iq2_s * x, const blk_q8_K * y) {
    float sumf = 0;
    for (int64_t i = 0; i < n / QK_K; ++i) {
        const float d = orc_fp16_to_fp32(x[i].d) * y[i].d;
        const int8_t * q8 = y[i].qs;
        int bsum = 0;
        for (int ib = 0; ib < 8; ++ib) {
            const int ls1 = 1 + 2 * (x[i].scales[ib] & 0xf);
            const int ls2 = 1 + 2 * (x[i].scales[ib] >> 4);
            int s12[2] = {0, 0};
            for (int l = 0; l < 4; ++l) {
                const int g = x[i].qs[4 * ib + l] | (((x[i].qh[ib] >> (2 * l)) & 3) << 8);
                const uint8_t sg = x[i].qs[32 + 4 * ib + l];
                for (int j = 0; j < 8; ++j)
                    s12[l / 2] += q8[j] * iq2s_grid_byte(g, j) * ((sg >> j) & 1 ? -1 : 1);
                q8 += 8;
            }
            bsum += ls1 * s12[0] + ls2 * s12[1];
        }
        sumf += d * bsum;
    }
    return 0.125f * sumf;
}

static float dot_q5_0_q8_0(int64_t n, const blk_q5_0 * x, const blk_q8_0 * y) {
    float sumf = 0;
    for (int64_t i = 0; i < n / 32; ++i) {
        uint32_t qh;
        memcpy(&qh, x[i].qh, 4);
        int s0 = 0, s1 = 0;
        for (int j = 0; j < 16; ++j) {
            const int x0 = ((x[i].qs[j] & 0x0F) | (((qh >> j) & 1) << 4)) - 16;
            const int x1 = ((x[i].qs[j] >> 4) | (((qh >> (j + 16)) & 1) << 4)) - 16;
            s0 += x0 * y[i].qs[j];
            s1 += x1 * y[i].qs[j + 16];
        }
        sumf += (orc_fp16_to_fp32(x[i].d) * orc_fp16_to_fp32(y[i].d)) * (s0 + s1);
    }
    return sumf;
}

static float dot_iq4_nl_q8_0(int64_t n, const blk_iq4_nl * x, const blk_q8_0 * y) {
    float sumf = 0;
    for (int64_t i = 0; i < n / 32; ++i) {
        const float d = orc_fp16_to_fp32(y[i].d) * orc_fp16_to_fp32(x[i].d);
        int s1 = 0, s2 = 0;
        for (int j = 0; j < 16; ++j) {
            s1 += y[i].qs[j] * iq4nl_values[x[i].qs[j] & 0xf];
            s2 += y[i].qs[j + 16] * iq4nl_values[x[i].qs[j] >> 4];
        }
        sumf += d * (s1 + s2);
    }
    return sumf;
}

/* q8_1 mode: the ggml-cuda arithmetic, accumulated per 32-block in double
 * (the device's partial-sum order is a launch detail; what is fixed is the
 * per-block integer math and the fp16 rounding of the q8_1 scales). */
static float dot_q4_K_q8_1(int64_t n, const blk_q4_K * x, const blk_q8_1 * y) {
    double acc = 0;
    for (int64_t i = 0; i < n / QK_K; ++i) {
        const float dm = orc_fp16_to_fp32(x[i].d), mm = orc_fp16_to_fp32(x[i].dmin);
        float sd = 0, sm = 0;
        for (int j = 0; j < 8; ++j) {
            int sc, m;
            q4k_scale_min(j, x[i].scales, &sc, &m);
            const blk_q8_1 * b = &y[i * 8 + j];
            const uint8_t * q4 = x[i].qs + 32 * (j / 2);
            const int shift = (j & 1) ? 4 : 0;
            int dot = 0, sq = 0;
            for (int l = 0; l < 32; ++l) {
                dot += ((q4[l] >> shift) & 0xF) * b->qs[l];
                sq += b->qs[l];
            }
            const float d8 = orc_fp16_to_fp32(b->d);
            sd += d8 * (float)(dot * sc);
            sm += d8 * (float)(sq * m);
        }
        acc += (double)(dm * sd - mm * sm);
    }
    return (float)acc;
}

static float dot_iq2_s_q8_1(int64_t n, const blk_iq2_s * x, const blk_q8_1 * y) {
    double acc = 0;
    for (int64_t i = 0; i < n / QK_K; ++i) {
        for (int ib = 0; ib < 8; ++ib) {
            const blk_q8_1 * b = &y[i * 8 + ib];
            const int ls0 = x[i].scales[ib] & 0x0F, ls1 = x[i].scales[ib] >> 4;
            int s[2] = {0, 0};
            for (int l = 0; l < 4; ++l) {
                const int g = x[i].qs[4 * ib + l] | (((x[i].qh[ib] >> (2 * l)) & 3) << 8);
                const uint8_t sg = x[i].qs[32 + 4 * ib + l];
                for (int j = 0; j < 8; ++j)
                    s[l / 2] += b->qs[8 * l + j] * iq2s_grid_byte(g, j) * ((sg >> j) & 1 ? -1 : 1);
            }
            /* integer (2 ls + 1) / 8 with C truncation, as the device does */
            const int sumi = (s[0] * ls0 + s[1] * ls1 + (s[0] + s[1]) / 2) / 4;
            const float d = orc_fp16_to_fp32(x[i].d) * orc_fp16_to_fp32(b->d);
            acc += (double)(d * sumi);
        }
    }
    return (float)acc;
}

static float dot_q5_0_q8_1(int64_t n, const blk_q5_0 * x, const blk_q8_1 * y) {
    double acc = 0;
    for (int64_t i = 0; i < n / 32; ++i) {
        uint32_t qh;
        memcpy(&qh, x[i].qh, 4);
        int sumi = 0;
        for (int j = 0; j < 16; ++j) {
            const int x0 = (x[i].qs[j] & 0x0F) | (((qh >> j) & 1) << 4);
            const int x1 = (x[i].qs[j] >> 4) | (((qh >> (j + 16)) & 1) << 4);
            sumi += x0 * y[i].qs[j] + x1 * y[i].qs[j + 16];
        }
        const float d5 = orc_fp16_to_fp32(x[i].d);
        const float d8 = orc_fp16_to_fp32(y[i].d), s8 = orc_fp16_to_fp32(y[i].s);
        acc += (double)(d5 * (sumi * d8 - 16.0f * s8));
    }
    return (float)acc;
}

static float dot_iq4_nl_q8_1(int64_t n, const blk_iq4_nl * x, const blk_q8_1 * y) {
    double acc = 0;
    for (int64_t i = 0; i < n / 32; ++i) {
        int sumi = 0;
        for (int j = 0; j < 16; ++j) {
            sumi += y[i].qs[j] * iq4nl_values[x[i].qs[j] & 0xf];
            sumi += y[i].qs[j + 16] * iq4nl_values[x[i].qs[j] >> 4];
        }
        acc += (double)(orc_fp16_to_fp32(x[i].d) * orc_fp16_to_fp32(y[i].d) * sumi);
    }
    return (float)acc;
}

/* ORC_ACT_Q8_1_MMA's IQ2_S: each 16-value half of a 32-block scaled by
 * (2 ls + 1) exactly (mmq.cuh:2881-2945 keeps d (2 ls + 1) / 8 as a float;
 * the integer form here is the same value), the block's sum times d d8 / 8. */
static float dot_iq2_s_q8_1_mma(int64_t n, const blk_iq2_s * x, const blk_q8_1 * y) {
    double acc = 0;
    for (int64_t i = 0; i < n / QK_K; ++i) {
        for (int ib = 0; ib < 8; ++ib) {
            const blk_q8_1 * b = &y[i * 8 + ib];
            const int ls0 = x[i].scales[ib] & 0x0F, ls1 = x[i].scales[ib] >> 4;
            int s[2] = {0, 0};
            for (int l = 0; l < 4; ++l) {
                const int g = x[i].qs[4 * ib + l] | (((x[i].qh[ib] >> (2 * l)) & 3) << 8);
                const uint8_t sg = x[i].qs[32 + 4 * ib + l];
                for (int j = 0; j < 8; ++j)
                    s[l / 2] += b->qs[8 * l + j] * iq2s_grid_byte(g, j) * ((sg >> j) & 1 ? -1 : 1);
            }
            const int sum8 = s[0] * (2 * ls0 + 1) + s[1] * (2 * ls1 + 1);     /* 8 x the scaled sum, exact */
            const float d = orc_fp16_to_fp32(x[i].d) * orc_fp16_to_fp32(b->d);
            acc += (double)(d * (float)sum8) * 0.125;
        }
    }
    return (float)acc;
}

/* ORC_ACT_Q8_1_MMA's Q5_0: the weights as q - 16 (mmq.cuh load_tiles_q5_0),
 * d_w d8 sum (q - 16) a, without q8_1's stored sum s8. */
static float dot_q5_0_q8_1_mma(int64_t n, const blk_q5_0 * x, const blk_q8_1 * y) {
    double acc = 0;
    for (int64_t i = 0; i < n / 32; ++i) {
        uint32_t qh;
        memcpy(&qh, x[i].qh, 4);
        int sumi = 0;
        for (int j = 0; j < 16; ++j) {
            const int x0 = ((x[i].qs[j] & 0x0F) | (((qh >> j) & 1) << 4)) - 16;
            const int x1 = ((x[i].qs[j] >> 4) | (((qh >> (j + 16)) & 1) << 4)) - 16;
            sumi += x0 * y[i].qs[j] + x1 * y[i].qs[j + 16];
        }
        acc += (double)(orc_fp16_to_fp32(x[i].d) * orc_fp16_to_fp32(y[i].d) * (float)sumi);
    }
    return (float)acc;
}

float orc_vec_dot(int wtype, int act_mode, int64_t n, const void * w, const void * a) {
    if (act_mode == ORC_ACT_Q8_1_MMA) {
        switch (wtype) {
            case ORC_Q4_K:   return dot_q4_K_q8_1(n, w, a);
            case ORC_IQ2_S:  return dot_iq2_s_q8_1_mma(n, w, a);
            case ORC_Q5_0:   return dot_q5_0_q8_1_mma(n, w, a);
            case ORC_IQ4_NL: return dot_iq4_nl_q8_1(n, w, a);
        }
    } else if (act_mode == ORC_ACT_Q8_1) {
        switch (wtype) {
            case ORC_Q4_K:   return dot_q4_K_q8_1(n, w, a);
            case ORC_IQ2_S:  return dot_iq2_s_q8_1(n, w, a);
            case ORC_Q5_0:   return dot_q5_0_q8_1(n, w, a);
            case ORC_IQ4_NL: return dot_iq4_nl_q8_1(n, w, a);
        }
    } else {
        switch (wtype) {
            case ORC_Q4_K:   return dot_q4_K_q8_K(n, w, a);
            case ORC_IQ2_S:  return dot_iq2_s_q8_K(n, w, a);
            case ORC_Q5_0:   return dot_q5_0_q8_0(n, w, a);
            case ORC_IQ4_NL: return dot_iq4_nl_q8_0(n, w, a);
        }
    }
    abort();
}

void orc_matvec(int wtype, int act_mode, const void * w, int64_t nrows, int64_t ncols,
                const float * x, float * y) {
    const int at = orc_act_type(wtype, act_mode);
    void * xq = malloc(orc_row_size(at, ncols));
    orc_quantize_act(at, x, xq, ncols);
    const size_t rs = orc_row_size(wtype, ncols);
    for (int64_t r = 0; r < nrows; ++r)
        y[r] = orc_vec_dot(wtype, act_mode, ncols, (const char *)w + r * rs, xq);
    free(xq);
}

/* ---------------------------------------------------------------- GEGLU */

static float gelu_tanh(float x) {
    const float GELU_COEF_A = 0.044715f;
    const float SQRT_2_OVER_PI = 0.79788456080286535587989211986876f;
    return 0.5f * x * (1.0f + tanhf(SQRT_2_OVER_PI * x * (1.0f + GELU_COEF_A * x * x)));
}

void orc_geglu(const float * g, const float * u, float * out, int64_t n, int gelu_mode) {
    for (int64_t i = 0; i < n; ++i) {
        if (gelu_mode == ORC_GELU_TANH) {
            out[i] = gelu_tanh(g[i]) * u[i];
        } else if (g[i] <= -10.0f) {
            out[i] = 0.0f;
        } else if (g[i] >= 10.0f) {
            out[i] = g[i] * u[i];
        } else {
            /* table entry for fp16(g): fp16(gelu(float(fp16(g)))) */
            const float gh = orc_fp16_to_fp32(orc_fp32_to_fp16(g[i]));
            out[i] = orc_fp16_to_fp32(orc_fp32_to_fp16(gelu_tanh(gh))) * u[i];
        }
    }
}

/* --------------------------------------------------------------- router */

void orc_router(const float * x, int64_t T, const float * w_r, const float * bias,
                int64_t d, int64_t n_expert, int64_t top_k,
                int32_t * ids, float * w, float * probs) {
    /* tokens are independent: a parallel loop gives the serial loop's bits */
    #pragma omp parallel
    {
    float * p = malloc(sizeof(float) * n_expert);
    int32_t * order = malloc(sizeof(int32_t) * n_expert);
    #pragma omp for schedule(static)
    for (int64_t t = 0; t < T; ++t) {
        const float * xt = x + t * d;
        float mx = -INFINITY;
        for (int64_t e = 0; e < n_expert; ++e) {
            double acc = 0;                     /* exact-ish dot: order-free */
            for (int64_t k = 0; k < d; ++k) acc += (double)w_r[e * d + k] * xt[k];
            p[e] = (float)acc + (bias ? bias[e] : 0.0f);
            if (p[e] > mx) mx = p[e];
        }
        double sum = 0;
        for (int64_t e = 0; e < n_expert; ++e) {
            p[e] = expf(p[e] - mx);
            sum += p[e];
        }
        /* ggml scales by the float of 1/sum (ops.cpp:5435-5443) */
        const float inv = (float)(1.0 / sum);
        for (int64_t e = 0; e < n_expert; ++e) p[e] = p[e] * inv;
        if (probs) memcpy(probs + t * n_expert, p, sizeof(float) * n_expert);
        /* descending order; equal probabilities keep the lower index first */
        for (int64_t e = 0; e < n_expert; ++e) order[e] = (int32_t)e;
        for (int64_t a = 0; a < top_k; ++a) {
            int64_t best = a;
            for (int64_t b = a + 1; b < n_expert; ++b)
                if (p[order[b]] > p[order[best]] ||
                    (p[order[b]] == p[order[best]] && order[b] < order[best])) best = b;
            int32_t tmp = order[a]; order[a] = order[best]; order[best] = tmp;
        }
        double sd = 0;                          /* sum_rows accumulates in double */
        for (int64_t a = 0; a < top_k; ++a) {
            ids[t * top_k + a] = order[a];
            w[t * top_k + a] = p[order[a]];
            sd += p[order[a]];
        }
        float s = (float)sd;
        if (s < 6.103515625e-5f) s = 6.103515625e-5f;
        for (int64_t a = 0; a < top_k; ++a) w[t * top_k + a] /= s;
    }
    free(p);
    free(order);
    }
}

/* ---------------------------------------------------------------- layer */

static uint64_t g_jitter_seed;

void orc_set_sum_jitter(uint64_t seed) { g_jitter_seed = seed; }

/* splitmix64 finaliser of the seed and a position */
static uint64_t jitter_hash(uint64_t a, uint64_t b) {
    uint64_t z = a * 0x9E3779B97F4A7C15ull + b + 0x632BE59BD9B4E5ull;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

static void jitter(float * v, int64_t n, uint64_t where) {
    if (!g_jitter_seed) return;
    for (int64_t i = 0; i < n; ++i)
        v[i] = nextafterf(v[i], (jitter_hash(g_jitter_seed ^ where, (uint64_t)i) & 1) ? INFINITY : -INFINITY);
}

static int pair_slot(const orc_layer * L, int32_t e) {
    if (e < 0 || e >= L->n_expert || !L->exp_slot) return -1;
    const int s = L->exp_slot[e];
    if (s >= 0 && s < L->k_slots && L->slot_state[s] == 2 && L->slot_exp[s] == e) return s;
    return -1;
}

void orc_moe_experts(const orc_layer * L, const float * x, int64_t T,
                     const int32_t * ids, const float * w, int act_mode, int gelu_mode,
                     float * out, float * y_pairs) {
    const int64_t D = L->d_model, F = L->n_ff, K = L->top_k;
    /* tokens are independent (each token's pairs, then its combine): a
     * parallel loop over tokens gives the serial loop's bits */
    #pragma omp parallel
    {
    float * gu = malloc(sizeof(float) * 2 * F);
    float * a = malloc(sizeof(float) * F);
    float * y = malloc(sizeof(float) * D * K);
    #pragma omp for schedule(dynamic, 1)
    for (int64_t t = 0; t < T; ++t) {
        for (int64_t k = 0; k < K; ++k) {
            const int32_t e = ids[t * K + k];
            const int s = pair_slot(L, e);
            const int gut = s >= 0 ? L->hot_gu_type : L->cold_gu_type;
            const int dnt = s >= 0 ? L->hot_dn_type : L->cold_dn_type;
            const int64_t idx = s >= 0 ? s : e;
            const char * wgu = (const char *)(s >= 0 ? L->hot_gu : L->cold_gu) +
                               (size_t)idx * 2 * F * orc_row_size(gut, D);
            const char * wdn = (const char *)(s >= 0 ? L->hot_dn : L->cold_dn) +
                               (size_t)idx * D * orc_row_size(dnt, F);
            orc_matvec(gut, act_mode, wgu, 2 * F, D, x + t * D, gu);
            jitter(gu, 2 * F, (uint64_t)(t * K + k) * 2);
            orc_geglu(gu, gu + F, a, F, gelu_mode);
            float * yk = y + k * D;
            orc_matvec(dnt, act_mode, wdn, D, F, a, yk);
            jitter(yk, D, (uint64_t)(t * K + k) * 2 + 1);
            const float * sc = s >= 0 ? L->s_hot : L->s_cold;
            if (sc) {
                const float f = sc[idx];
                for (int64_t r = 0; r < D; ++r) yk[r] = yk[r] * f;
            }
            if (y_pairs) memcpy(y_pairs + (t * K + k) * D, yk, sizeof(float) * D);
        }
        float * o = out + t * D;
        for (int64_t r = 0; r < D; ++r) o[r] = y[r] * w[t * K];
        for (int64_t k = 1; k < K; ++k)
            for (int64_t r = 0; r < D; ++r) o[r] = o[r] + y[k * D + r] * w[t * K + k];
    }
    free(gu);
    free(a);
    free(y);
    }
}
