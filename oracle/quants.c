/*
 * quants.c -- ggml K-quant block codecs and integer dot products, restated.
 * TEST INFRASTRUCTURE ONLY (see oracle.h).
 *
 * Block layouts are ggml's (llama.cpp bccbacd, un-vendored in the reference):
 *   Q4_K  144 B : fp16 d, fp16 dmin, 12 B packed 6-bit (scale, min) x 8, 128 B nibbles
 *   Q6_K  210 B : 128 B low nibbles, 64 B high 2-bit pairs, 16 int8 scales, fp16 d
 *   Q8_K  292 B : f32 d, 256 int8, 16 int16 sums of 16-value groups
 * The expert chain of the reference feeds Q4_K/Q6_K weights against Q8_K
 * activations (x2_cpu_expert_cost.cpp:7-9, 75-78, 124-126, 144).
 */
#include "oracle.h"

#include <math.h>
#include <string.h>

float or_h2f(uint16_t h) {
    const uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    uint32_t exp = (h >> 10) & 0x1f;
    uint32_t man = h & 0x3ffu;
    uint32_t bits;
    if (exp == 0) {
        if (man == 0) {
            bits = sign;
        } else {                      /* subnormal: renormalise */
            int e = -1;
            do { man <<= 1; e++; } while (!(man & 0x400u));
            man &= 0x3ffu;
            bits = sign | ((uint32_t)(127 - 15 - e) << 23) | (man << 13);
        }
    } else if (exp == 31) {
        bits = sign | 0x7f800000u | (man << 13);
    } else {
        bits = sign | ((exp + 127 - 15) << 23) | (man << 13);
    }
    float f;
    memcpy(&f, &bits, 4);
    return f;
}

/* round to nearest even, as the x86 F16C conversion ggml uses */
uint16_t or_f2h(float f) {
    uint32_t x;
    memcpy(&x, &f, 4);
    const uint32_t sign = (x >> 16) & 0x8000u;
    const uint32_t ax = x & 0x7fffffffu;
    if (ax >= 0x7f800000u) {                       /* inf / nan */
        return (uint16_t)(sign | 0x7c00u | (ax > 0x7f800000u ? 0x200u : 0));
    }
    if (ax >= 0x477ff000u) {                       /* rounds to >= 65520: inf */
        return (uint16_t)(sign | 0x7c00u);
    }
    if (ax < 0x38800000u) {                        /* below 2^-14: subnormal half */
        if (ax < 0x33000000u) {                    /* < 2^-25: rounds to 0 */
            return (uint16_t)sign;
        }
        const uint32_t e = ax >> 23;               /* 102..112 */
        const uint32_t m = (ax & 0x7fffffu) | 0x800000u;
        const uint32_t shift = 126 - e;            /* 14..24 */
        uint32_t r = m >> shift;
        const uint32_t rem = m & ((1u << shift) - 1);
        const uint32_t half = 1u << (shift - 1);
        if (rem > half || (rem == half && (r & 1))) r++;
        return (uint16_t)(sign | r);
    }
    uint32_t r = ((ax >> 13) - (112u << 10));      /* rebias exponent */
    const uint32_t rem = ax & 0x1fffu;
    if (rem > 0x1000u || (rem == 0x1000u && (r & 1))) r++;
    return (uint16_t)(sign | r);
}

static inline int nearest_even(float v) { return (int)rintf(v); }

static void q4k_scale_min(int j, const uint8_t *q, int *sc, int *m) {
    if (j < 4) {
        *sc = q[j] & 63;
        *m  = q[j + 4] & 63;
    } else {
        *sc = (q[j + 4] & 0xF) | ((q[j - 4] >> 6) << 4);
        *m  = (q[j + 4] >> 4)  | ((q[j] >> 6) << 4);
    }
}

/* Q4_K element e of a block: qs byte (e/64)*32 + e%32, low nibble for
 * e%64 < 32, high nibble otherwise; sub-block e/32 carries (scale, min). */
void or_dequant_q4k(const void *blocks, float *y, int64_t n) {
    const uint8_t *b = (const uint8_t *)blocks;
    for (int64_t i = 0; i < n / OR_QK; ++i, b += OR_Q4K_BYTES) {
        uint16_t hd, hm;
        memcpy(&hd, b, 2);
        memcpy(&hm, b + 2, 2);
        const float d = or_h2f(hd), dmin = or_h2f(hm);
        const uint8_t *scales = b + 4, *qs = b + 16;
        for (int e = 0; e < OR_QK; ++e) {
            int sc, m;
            q4k_scale_min(e / 32, scales, &sc, &m);
            const uint8_t byte = qs[(e / 64) * 32 + (e % 32)];
            const int q = (e % 64) < 32 ? (byte & 0xF) : (byte >> 4);
            y[i * OR_QK + e] = d * (float)sc * (float)q - dmin * (float)m;
        }
    }
}

/* Q6_K element e: half h = e/128, r = e%128, l = r%32, quarter g = r/32.
 * low nibble from ql[64h + l + 32*(g&1)] (>>4 for g >= 2), high two bits
 * from qh[32h + l] >> 2g; value - 32; scale index 8h + l/16 + 2g. */
void or_dequant_q6k(const void *blocks, float *y, int64_t n) {
    const uint8_t *b = (const uint8_t *)blocks;
    for (int64_t i = 0; i < n / OR_QK; ++i, b += OR_Q6K_BYTES) {
        const uint8_t *ql = b, *qh = b + 128;
        const int8_t *sc = (const int8_t *)(b + 192);
        uint16_t hd;
        memcpy(&hd, b + 208, 2);
        const float d = or_h2f(hd);
        for (int e = 0; e < OR_QK; ++e) {
            const int h = e / 128, r = e % 128, l = r % 32, g = r / 32;
            const uint8_t lo = ql[64 * h + l + 32 * (g & 1)];
            const int low = g >= 2 ? (lo >> 4) : (lo & 0xF);
            const int high = (qh[32 * h + l] >> (2 * g)) & 3;
            const int q = (low | (high << 4)) - 32;
            y[i * OR_QK + e] = d * (float)sc[8 * h + l / 16 + 2 * g] * (float)q;
        }
    }
}

/* ggml's reference Q8_K quantizer: the value of largest magnitude (first one
 * on a tie) maps to -127, iscale = -127/max, q = min(127, round_even(iscale*x)),
 * d = 1/iscale.  An all-zero block gets d = 0, q = 0 (and zero sums). */
void or_quant_q8k(const float *x, void *blocks, int64_t n) {
    uint8_t *b = (uint8_t *)blocks;
    for (int64_t i = 0; i < n / OR_QK; ++i, b += OR_Q8K_BYTES, x += OR_QK) {
        float amax = 0.0f, max = 0.0f;
        for (int j = 0; j < OR_QK; ++j) {
            const float ax = fabsf(x[j]);
            if (ax > amax) { amax = ax; max = x[j]; }
        }
        int8_t qs[OR_QK];
        int16_t bs[16];
        float d = 0.0f;
        if (amax == 0.0f) {
            memset(qs, 0, sizeof qs);
            memset(bs, 0, sizeof bs);
        } else {
            const float iscale = -127.0f / max;
            for (int j = 0; j < OR_QK; ++j) {
                const int v = nearest_even(iscale * x[j]);
                qs[j] = (int8_t)(v < 127 ? v : 127);
            }
            for (int g = 0; g < 16; ++g) {
                int s = 0;
                for (int j = 0; j < 16; ++j) s += qs[16 * g + j];
                bs[g] = (int16_t)s;
            }
            d = 1.0f / iscale;
        }
        memcpy(b, &d, 4);
        memcpy(b + 4, qs, OR_QK);
        memcpy(b + 4 + OR_QK, bs, 32);
    }
}

void or_dequant_q8k(const void *blocks, float *y, int64_t n) {
    const uint8_t *b = (const uint8_t *)blocks;
    for (int64_t i = 0; i < n / OR_QK; ++i, b += OR_Q8K_BYTES) {
        float d;
        memcpy(&d, b, 4);
        const int8_t *qs = (const int8_t *)(b + 4);
        for (int j = 0; j < OR_QK; ++j) y[i * OR_QK + j] = d * (float)qs[j];
    }
}

/* Per block: sumi = sum_j scale_j * <q4_j, q8_j> (exact int32),
 *            summ = sum_j min_j * (bsum_{2j} + bsum_{2j+1}) (exact int32),
 *            acc += d_w*d_x * sumi - dmin_w*d_x * summ   (fp32, block order). */
float or_dot_q4k_q8k(int n, const void *w, const void *q8) {
    const uint8_t *wb = (const uint8_t *)w, *xb = (const uint8_t *)q8;
    float acc = 0.0f;
    for (int i = 0; i < n / OR_QK; ++i, wb += OR_Q4K_BYTES, xb += OR_Q8K_BYTES) {
        uint16_t hd, hm;
        memcpy(&hd, wb, 2);
        memcpy(&hm, wb + 2, 2);
        float dx;
        memcpy(&dx, xb, 4);
        const int8_t *qx = (const int8_t *)(xb + 4);
        int16_t bs[16];
        memcpy(bs, xb + 4 + OR_QK, 32);
        const uint8_t *scales = wb + 4, *qs = wb + 16;
        int32_t sumi = 0, summ = 0;
        for (int j = 0; j < 8; ++j) {
            int sc, m;
            q4k_scale_min(j, scales, &sc, &m);
            const uint8_t *qb = qs + (j / 2) * 32;
            const int hi = j & 1;
            int32_t dot = 0;
            for (int l = 0; l < 32; ++l) {
                const int q = hi ? (qb[l] >> 4) : (qb[l] & 0xF);
                dot += q * qx[32 * j + l];
            }
            sumi += sc * dot;
            summ += m * (bs[2 * j] + bs[2 * j + 1]);
        }
        const float d = or_h2f(hd) * dx;
        const float dm = or_h2f(hm) * dx;
        acc += d * (float)sumi;
        acc -= dm * (float)summ;
    }
    return acc;
}

/* Per block: sumi = sum_g scale_g * <q6_g - 32, q8_g> over 16-value groups
 * (exact int32); acc += d_w*d_x * sumi (fp32, block order). */
float or_dot_q6k_q8k(int n, const void *w, const void *q8) {
    const uint8_t *wb = (const uint8_t *)w, *xb = (const uint8_t *)q8;
    float acc = 0.0f;
    for (int i = 0; i < n / OR_QK; ++i, wb += OR_Q6K_BYTES, xb += OR_Q8K_BYTES) {
        const uint8_t *ql = wb, *qh = wb + 128;
        const int8_t *sc = (const int8_t *)(wb + 192);
        uint16_t hd;
        memcpy(&hd, wb + 208, 2);
        float dx;
        memcpy(&dx, xb, 4);
        const int8_t *qx = (const int8_t *)(xb + 4);
        int32_t grp[16] = {0};
        for (int e = 0; e < OR_QK; ++e) {
            const int h = e / 128, r = e % 128, l = r % 32, g = r / 32;
            const uint8_t lo = ql[64 * h + l + 32 * (g & 1)];
            const int low = g >= 2 ? (lo >> 4) : (lo & 0xF);
            const int high = (qh[32 * h + l] >> (2 * g)) & 3;
            const int q = (low | (high << 4)) - 32;
            grp[8 * h + l / 16 + 2 * g] += q * qx[e];
        }
        int32_t sumi = 0;
        for (int g = 0; g < 16; ++g) sumi += sc[g] * grp[g];
        const float d = or_h2f(hd) * dx;
        acc += d * (float)sumi;
    }
    return acc;
}

double or_dot_deq_f64(int wtype, int n, const void *w, const void *q8) {
    /* Both operands dequantized exactly in double: Q4_K d*sc*q - dmin*m,
     * Q6_K d*sc*(q-32), Q8_K d*q.  No fp32 rounding anywhere. */
    float wf[OR_QK];
    const size_t wb = wtype == OR_TYPE_Q4K ? OR_Q4K_BYTES : OR_Q6K_BYTES;
    double acc = 0.0;
    for (int i = 0; i < n / OR_QK; ++i) {
        const uint8_t *blk = (const uint8_t *)w + (size_t)i * wb;
        const uint8_t *xb = (const uint8_t *)q8 + (size_t)i * OR_Q8K_BYTES;
        float dx;
        memcpy(&dx, xb, 4);
        const int8_t *qx = (const int8_t *)(xb + 4);
        if (wtype == OR_TYPE_Q4K) {
            uint16_t hd, hm;
            memcpy(&hd, blk, 2);
            memcpy(&hm, blk + 2, 2);
            const double d = or_h2f(hd), dmin = or_h2f(hm);
            const uint8_t *scales = blk + 4, *qs = blk + 16;
            for (int e = 0; e < OR_QK; ++e) {
                int sc, m;
                q4k_scale_min(e / 32, scales, &sc, &m);
                const uint8_t byte = qs[(e / 64) * 32 + (e % 32)];
                const int q = (e % 64) < 32 ? (byte & 0xF) : (byte >> 4);
                acc += (d * sc * q - dmin * m) * ((double)dx * qx[e]);
            }
        } else {
            or_dequant_q6k(blk, wf, OR_QK);    /* d*sc*(q-32) fits 24 bits: exact */
            for (int e = 0; e < OR_QK; ++e) acc += (double)wf[e] * ((double)dx * qx[e]);
        }
    }
    return acc;
}
