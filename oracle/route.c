/*
 * route.c -- router softmax, cache prior, top-k and gate weights, restated.
 * TEST INFRASTRUCTURE ONLY (see oracle.h for the canonical order).
 *
 * Reference: build_moe_ffn (llama.cpp, un-vendored; visible as context in
 * patches/0007-admission-gate-batched-tables-heat-file-cache-prior.patch:105-127):
 * probs = softmax(logits); selection = probs + prior (prior = delta where the
 * expert's table entry is not the dummy, patches/0007...:327-348, 783-790);
 * ids = top-k(selection); weights = probs[ids] / sum(probs[ids]).
 */
#include "oracle.h"

#include <math.h>
#include <string.h>

/* exp for x <= ~88: n = round_even(x*log2e), r = x - n*ln2 (two-part
 * Cody-Waite), degree-7 Taylor polynomial of e^r in Horner form with fmaf,
 * times 2^n built in the exponent field.  Returns 0 below -87 (probabilities
 * that small are irrelevant to selection and the weights). */
float or_expf(float x) {
    if (x < -87.0f) return 0.0f;
    if (x > 88.0f) x = 88.0f;
    const float n = rintf(x * 1.44269504088896341f);
    float r = fmaf(n, -0.693145751953125f, x);
    r = fmaf(n, -1.428606765330187045e-06f, r);
    float p = 1.9841269841269841e-04f;          /* 1/5040 */
    p = fmaf(p, r, 1.3888888888888889e-03f);    /* 1/720 */
    p = fmaf(p, r, 8.3333333333333333e-03f);    /* 1/120 */
    p = fmaf(p, r, 4.1666666666666667e-02f);    /* 1/24 */
    p = fmaf(p, r, 1.6666666666666667e-01f);    /* 1/6 */
    p = fmaf(p, r, 0.5f);
    p = fmaf(p, r, 1.0f);
    p = fmaf(p, r, 1.0f);
    const int32_t e = (int32_t)n + 127;
    uint32_t bits = (uint32_t)e << 23;
    float s;
    memcpy(&s, &bits, 4);
    return p * s;
}

/* the canonical 64-lane butterfly: p_j += p_{j^o} for o = 1, 2, 4, 8, 16, 32 */
static float canon_sum64(float p[64]) {
    for (int o = 1; o <= 32; o <<= 1) {
        float t[64];
        for (int j = 0; j < 64; ++j) t[j] = p[j] + p[j ^ o];
        memcpy(p, t, 64 * sizeof(float));
    }
    return p[0];
}

float or_row_logit(int H, const float *w, const float *x) {
    /* four quarters of the row, one per wavefront of the GPU's workgroup */
    const int Q = H / 4;
    float s[4];
    for (int q = 0; q < 4; ++q) {
        float p[64];
        for (int j = 0; j < 64; ++j) {
            float acc = 0.0f;
            for (int i = 0; i < Q / 256; ++i) {
                for (int c = 0; c < 4; ++c) {
                    const int k = Q * q + 256 * i + 4 * j + c;
                    acc = fmaf(w[k], x[k], acc);
                }
            }
            p[j] = acc;
        }
        s[q] = canon_sum64(p);
    }
    return ((s[0] + s[1]) + s[2]) + s[3];
}

static void softmax_topk(int E, int K, const float *logits, const float *prior, int prior_on_logits,
                         int32_t *ids, float *w, float *probs_out) {
    float m = logits[0];
    for (int e = 1; e < E; ++e) if (logits[e] > m) m = logits[e];
    float ex[1024], probs[1024], sel[1024];
    for (int e = 0; e < E; ++e) ex[e] = or_expf(logits[e] - m);
    float s = 0.0f;
    for (int c = 0; c < E / 64; ++c) {
        float p[64];
        memcpy(p, ex + 64 * c, sizeof p);
        const float cs = canon_sum64(p);
        s = c == 0 ? cs : s + cs;
    }
    for (int e = 0; e < E; ++e) {
        probs[e] = ex[e] / s;
        if (!prior) sel[e] = probs[e];
        else sel[e] = prior_on_logits ? logits[e] + prior[e] : probs[e] + prior[e];
    }
    unsigned char taken[1024] = {0};
    for (int k = 0; k < K; ++k) {
        int best = -1;
        for (int e = 0; e < E; ++e) {
            if (taken[e]) continue;
            if (best < 0 || sel[e] > sel[best]) best = e;   /* strict: lower id keeps a tie */
        }
        taken[best] = 1;
        ids[k] = best;
    }
    float wsum = 0.0f;
    for (int k = 0; k < K; ++k) wsum += probs[ids[k]];
    for (int k = 0; k < K; ++k) w[k] = probs[ids[k]] / wsum;
    if (probs_out) memcpy(probs_out, probs, (size_t)E * sizeof(float));
}

void or_route(int E, int H, int K, const float *W, const float *x, const float *bias,
              const float *prior, const int32_t *table, int32_t *ids, float *w,
              int32_t *slots, float *probs) {
    or_route_space(E, H, K, W, x, bias, prior, 0, table, ids, w, slots, probs);
}

void or_route_space(int E, int H, int K, const float *W, const float *x, const float *bias,
                    const float *prior, int prior_on_logits, const int32_t *table, int32_t *ids,
                    float *w, int32_t *slots, float *probs) {
    float logits[1024];
    for (int e = 0; e < E; ++e) {
        logits[e] = or_row_logit(H, W + (size_t)e * H, x);
        if (bias) logits[e] = logits[e] + bias[e];
    }
    softmax_topk(E, K, logits, prior, prior_on_logits, ids, w, probs);
    if (table && slots) {
        for (int k = 0; k < K; ++k) slots[k] = table[ids[k]];
    }
}

void or_route_logits(int E, int K, const float *logits, const float *prior,
                     int32_t *ids, float *w, float *probs) {
    softmax_topk(E, K, logits, prior, 0, ids, w, probs);
}
