// mp_synth.h -- seeded synthetic weights and activations, identical on the
// host and on the device.
//
// Normal draws: the textbook sum-of-12-uniforms method on 10-bit uniforms
// taken from two SplitMix64 outputs:  z = (sum_{i<12} u_i - 6138) / 1024,
// u_i in [0, 1023].  Mean 0, variance 1 - 1/(12*1024^2), support [-6, 6].
// Every step is integer arithmetic or an exact float scaling, so the host and
// gfx950 produce the same bits without sharing a libm.
//
// Quantizers: ggml's reference Q4_K and Q6_K quantizers (make_qkx2_quants with
// weights av_x + |x|, 20-step scale search; make_qx_quants with x^2 weights,
// +-0.9 scale search), restated.  They only decide which valid blocks the
// synthetic experts hold: both the GPU path and the CPU oracle consume those
// bytes, so no check depends on matching ggml's bytes.  Compiled with
// -ffp-contract=off and IEEE division/sqrt on both sides, the host and device
// versions produce identical blocks (checked on the GPU).
#pragma once

#include <math.h>
#include <string.h>

#include "mp_format.h"

namespace mp {
namespace synth {

MP_HD uint64_t splitmix(uint64_t &s) {
    uint64_t z = (s += 0x9E3779B97F4A7C15ull);
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

// independent stream for a tuple of coordinates
MP_HD uint64_t key(uint64_t seed, uint64_t a, uint64_t b, uint64_t c, uint64_t d) {
    uint64_t s = seed ^ 0x6A09E667F3BCC909ull;
    s ^= splitmix(s) + a;
    s ^= splitmix(s) + b;
    s ^= splitmix(s) + c;
    s ^= splitmix(s) + d;
    splitmix(s);
    return s;
}

MP_HD float normal(uint64_t &s) {
    const uint64_t a = splitmix(s), b = splitmix(s);
    int32_t sum = 0;
    for (int i = 0; i < 6; ++i) {
        sum += (int32_t)((a >> (10 * i)) & 1023u);
        sum += (int32_t)((b >> (10 * i)) & 1023u);
    }
    return (float)(sum - 6138) * (1.0f / 1024.0f);
}

MP_HD int nearest(float v) { return (int)rintf(v); }

// ---- Q4_K ------------------------------------------------------------------
MP_HD float qkx2(const float *x, const float *w, uint8_t *L, float *the_min, uint8_t *Laux) {
    const int n = 32, nmax = 15, nstep = 20;
    const float rmin = -1.0f, rdelta = 0.1f;
    float mn = x[0], mx = x[0];
    float sum_w = w[0];
    float sum_x = sum_w * x[0];
    for (int i = 1; i < n; ++i) {
        if (x[i] < mn) mn = x[i];
        if (x[i] > mx) mx = x[i];
        sum_w += w[i];
        sum_x += w[i] * x[i];
    }
    if (mn > 0) mn = 0;
    if (mx == mn) {
        for (int i = 0; i < n; ++i) L[i] = 0;
        *the_min = -mn;
        return 0.0f;
    }
    float iscale = nmax / (mx - mn);
    float scale = 1 / iscale;
    float best_error = 0;
    for (int i = 0; i < n; ++i) {
        int l = nearest(iscale * (x[i] - mn));
        l = l < 0 ? 0 : (l > nmax ? nmax : l);
        L[i] = (uint8_t)l;
        float diff = scale * L[i] + mn - x[i];
        diff = diff * diff;
        best_error += w[i] * diff;
    }
    for (int is = 0; is <= nstep; ++is) {
        iscale = (rmin + rdelta * is + nmax) / (mx - mn);
        float sum_l = 0, sum_l2 = 0, sum_xl = 0;
        for (int i = 0; i < n; ++i) {
            int l = nearest(iscale * (x[i] - mn));
            l = l < 0 ? 0 : (l > nmax ? nmax : l);
            Laux[i] = (uint8_t)l;
            sum_l += w[i] * l;
            sum_l2 += w[i] * l * l;
            sum_xl += w[i] * l * x[i];
        }
        float D = sum_w * sum_l2 - sum_l * sum_l;
        if (D > 0) {
            float this_scale = (sum_w * sum_xl - sum_x * sum_l) / D;
            float this_min = (sum_l2 * sum_x - sum_l * sum_xl) / D;
            if (this_min > 0) {
                this_min = 0;
                this_scale = sum_xl / sum_l2;
            }
            float cur_error = 0;
            for (int i = 0; i < n; ++i) {
                float diff = this_scale * Laux[i] + this_min - x[i];
                diff = diff * diff;
                cur_error += w[i] * diff;
            }
            if (cur_error < best_error) {
                for (int i = 0; i < n; ++i) L[i] = Laux[i];
                best_error = cur_error;
                scale = this_scale;
                mn = this_min;
            }
        }
    }
    *the_min = -mn;
    return scale;
}

MP_HD void quantize_q4k(const float *x, uint8_t *out) {
    uint8_t L[QK], Laux[32];
    float wts[32], mins[8], scales[8];
    float max_scale = 0, max_min = 0;
    for (int j = 0; j < 8; ++j) {
        float sum_x2 = 0;
        for (int l = 0; l < 32; ++l) sum_x2 += x[32 * j + l] * x[32 * j + l];
        const float av_x = sqrtf(sum_x2 / 32);
        for (int l = 0; l < 32; ++l) wts[l] = av_x + fabsf(x[32 * j + l]);
        scales[j] = qkx2(x + 32 * j, wts, L + 32 * j, &mins[j], Laux);
        if (scales[j] > max_scale) max_scale = scales[j];
        if (mins[j] > max_min) max_min = mins[j];
    }
    const float inv_scale = max_scale > 0 ? 63.0f / max_scale : 0.0f;
    const float inv_min = max_min > 0 ? 63.0f / max_min : 0.0f;
    uint8_t *sc = out + 4;
    for (int j = 0; j < 12; ++j) sc[j] = 0;
    for (int j = 0; j < 8; ++j) {
        int ls = nearest(inv_scale * scales[j]);
        int lm = nearest(inv_min * mins[j]);
        ls = ls > 63 ? 63 : ls;
        lm = lm > 63 ? 63 : lm;
        if (j < 4) {
            sc[j] = (uint8_t)ls;
            sc[j + 4] = (uint8_t)lm;
        } else {
            sc[j + 4] = (uint8_t)((ls & 0xF) | ((lm & 0xF) << 4));
            sc[j - 4] |= (uint8_t)((ls >> 4) << 6);
            sc[j] |= (uint8_t)((lm >> 4) << 6);
        }
    }
    const uint16_t hd = f2h(max_scale / 63.0f), hm = f2h(max_min / 63.0f);
    out[0] = (uint8_t)(hd & 0xff);
    out[1] = (uint8_t)(hd >> 8);
    out[2] = (uint8_t)(hm & 0xff);
    out[3] = (uint8_t)(hm >> 8);
    for (int j = 0; j < 8; ++j) {
        int s, m;
        q4k_scale_min(j, sc, s, m);
        const float d = h2f(hd) * s;
        if (!(d != 0.0f)) continue;
        const float dm = h2f(hm) * m;
        for (int ii = 0; ii < 32; ++ii) {
            int l = nearest((x[32 * j + ii] + dm) / d);
            l = l < 0 ? 0 : (l > 15 ? 15 : l);
            L[32 * j + ii] = (uint8_t)l;
        }
    }
    uint8_t *q = out + 16;
    for (int j = 0; j < QK; j += 64) {
        for (int l = 0; l < 32; ++l) q[l] = (uint8_t)(L[j + l] | (L[j + l + 32] << 4));
        q += 32;
    }
}

// ---- Q6_K ------------------------------------------------------------------
MP_HD float qx(const float *x, int8_t *L) {
    const int n = 16, nmax = 32;
    float mx = 0, amax = 0;
    for (int i = 0; i < n; ++i) {
        const float ax = fabsf(x[i]);
        if (ax > amax) { amax = ax; mx = x[i]; }
    }
    if (amax < 1e-15f) {
        for (int i = 0; i < n; ++i) L[i] = 0;
        return 0.0f;
    }
    float iscale = -nmax / mx;
    float sumlx = 0, suml2 = 0;
    for (int i = 0; i < n; ++i) {
        int l = nearest(iscale * x[i]);
        l = l < -nmax ? -nmax : (l > nmax - 1 ? nmax - 1 : l);
        L[i] = (int8_t)(l + nmax);
        const float w = x[i] * x[i];
        sumlx += w * x[i] * l;
        suml2 += w * l * l;
    }
    float scale = suml2 != 0.0f ? sumlx / suml2 : 0.0f;
    float best = scale * sumlx;
    for (int is = -9; is <= 9; ++is) {
        if (is == 0) continue;
        iscale = -(nmax + 0.1f * is) / mx;
        sumlx = suml2 = 0;
        for (int i = 0; i < n; ++i) {
            int l = nearest(iscale * x[i]);
            l = l < -nmax ? -nmax : (l > nmax - 1 ? nmax - 1 : l);
            const float w = x[i] * x[i];
            sumlx += w * x[i] * l;
            suml2 += w * l * l;
        }
        if (suml2 > 0 && sumlx * sumlx > best * suml2) {
            for (int i = 0; i < n; ++i) {
                int l = nearest(iscale * x[i]);
                l = l < -nmax ? -nmax : (l > nmax - 1 ? nmax - 1 : l);
                L[i] = (int8_t)(nmax + l);
            }
            scale = sumlx / suml2;
            best = scale * sumlx;
        }
    }
    return scale;
}

MP_HD void quantize_q6k(const float *x, uint8_t *out) {
    int8_t L[QK];
    float scales[16];
    float max_scale = 0, max_abs = 0;
    for (int ib = 0; ib < 16; ++ib) {
        scales[ib] = qx(x + 16 * ib, L + 16 * ib);
        const float a = fabsf(scales[ib]);
        if (a > max_abs) { max_abs = a; max_scale = scales[ib]; }
    }
    for (int i = 0; i < Q6K_BYTES; ++i) out[i] = 0;
    if (max_abs < 1e-15f) return;
    const float iscale = -128.0f / max_scale;
    const uint16_t hd = f2h(1 / iscale);
    out[208] = (uint8_t)(hd & 0xff);
    out[209] = (uint8_t)(hd >> 8);
    int8_t *sc = (int8_t *)(out + 192);
    for (int ib = 0; ib < 16; ++ib) {
        int v = nearest(iscale * scales[ib]);
        sc[ib] = (int8_t)(v > 127 ? 127 : v);
    }
    for (int j = 0; j < 16; ++j) {
        const float d = h2f(hd) * sc[j];
        if (!(d != 0.0f)) continue;
        for (int ii = 0; ii < 16; ++ii) {
            int l = nearest(x[16 * j + ii] / d);
            l = l < -32 ? -32 : (l > 31 ? 31 : l);
            L[16 * j + ii] = (int8_t)(l + 32);
        }
    }
    uint8_t *ql = out, *qh = out + 128;
    for (int j = 0; j < QK; j += 128) {
        for (int l = 0; l < 32; ++l) {
            const uint8_t q1 = (uint8_t)L[j + l] & 0xF, q2 = (uint8_t)L[j + l + 32] & 0xF;
            const uint8_t q3 = (uint8_t)L[j + l + 64] & 0xF, q4 = (uint8_t)L[j + l + 96] & 0xF;
            ql[l] = (uint8_t)(q1 | (q3 << 4));
            ql[l + 32] = (uint8_t)(q2 | (q4 << 4));
            qh[l] = (uint8_t)(((uint8_t)L[j + l] >> 4) | (((uint8_t)L[j + l + 32] >> 4) << 2) |
                              (((uint8_t)L[j + l + 64] >> 4) << 4) | (((uint8_t)L[j + l + 96] >> 4) << 6));
        }
        ql += 64;
        qh += 32;
    }
}

// ---- what a synthetic expert holds ------------------------------------------
// Super-block `blk` of the expert (layer, expert): blocks are numbered in
// byte order through [up | gate | down]; each one is 256 N(0, sigma) draws from
// its own stream, quantized to the block's type.
struct ExpertShape {
    int H, I, down_type;
    MP_HD int n_up_blocks() const { return I * (H / QK); }
    MP_HD int n_blocks() const { return 2 * n_up_blocks() + H * (I / QK); }
    MP_HD uint64_t block_offset(int blk) const {
        const int nu = n_up_blocks();
        return blk < 2 * nu ? (uint64_t)blk * Q4K_BYTES
                            : 2ull * nu * Q4K_BYTES + (uint64_t)(blk - 2 * nu) * block_bytes(down_type);
    }
    MP_HD int block_type(int blk) const { return blk < 2 * n_up_blocks() ? TYPE_Q4K : down_type; }
};

MP_HD void expert_block(uint64_t seed, int layer, int expert, const ExpertShape &sh, int blk,
                        float sigma, uint8_t *out) {
    float x[QK];
    uint64_t s = key(seed, 1, (uint64_t)layer, (uint64_t)expert, (uint64_t)blk);
    for (int i = 0; i < QK; ++i) x[i] = normal(s) * sigma;
    if (sh.block_type(blk) == TYPE_Q4K) quantize_q4k(x, out);
    else quantize_q6k(x, out);
}

// n values of an N(0, sigma) vector identified by (kind, a, b)
// kinds 0 (router rows) and 1 (activations): N(0, sigma); kind 2 (router
// logits): uniform on [0, sigma), 24-bit grid, exact in fp32
constexpr int KIND_UNIFORM_LOGITS = 2;

MP_HD float vec_value(uint64_t seed, int kind, int a, int b, int i, float sigma) {
    uint64_t s = key(seed, 2 + (uint64_t)kind, (uint64_t)a, (uint64_t)b, (uint64_t)i);
    if (kind == KIND_UNIFORM_LOGITS) return (float)(splitmix(s) >> 40) * (1.0f / 16777216.0f) * sigma;
    return normal(s) * sigma;
}

}  // namespace synth
}  // namespace mp
