/*
 * moep.c -- the MOEP expert predictor / evictor of the reference's cache,
 * restated.  TEST INFRASTRUCTURE ONLY (see oracle.h).
 *
 * Follows cpp/moe-predictor.cpp of the reference:
 *   file layout   :20-150 (MOEP v3: magic, eleven u32, the block table, the
 *                 layer list, priors, biases, weights; PCA models are not
 *                 loaded here -- the cache never scores them, 0006:539-552)
 *   score         :165-222 (bias, the picked rows in block order, z-score,
 *                 then the repeat prior on the prev ids)
 *   top-k         :224-238 (best first, the lower id first on equal scores)
 *   update        :241-305 (recall@8 of the prediction, one logistic SGD step
 *                 on the picked rows and the bias)
 * Arithmetic in the reference's order, fp32, no contraction (-ffp-contract=off).
 */
#include "oracle.h"

#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

struct or_moep {
    uint32_t E, n_layers, feat_dim, n_present;
    int32_t off[4];          /* first column of prev, cur, below, self_prev; -1 when absent */
    int32_t *index_of;       /* [n_layers]: row of the layer in the tables below, or -1 */
    float *prior;            /* [n_present] */
    float *bias;             /* [n_present][E] */
    float *w;                /* [n_present][feat_dim][E] */
};

static int rd(FILE *f, void *p, size_t n) { return fread(p, 1, n, f) == n; }

or_moep *or_moep_load(const char *path) {
    FILE *f = fopen(path, "rb");
    if (!f) return NULL;
    char magic[4];
    uint32_t h[11];
    or_moep *m = (or_moep *)calloc(1, sizeof(or_moep));
    int ok = rd(f, magic, 4) && memcmp(magic, "MOEP", 4) == 0 && rd(f, h, sizeof h) && h[0] == 3 && h[9] == 0;
    if (ok) {
        m->E = h[3];
        m->n_layers = h[4];
        m->feat_dim = h[6];
        m->n_present = h[7];
        for (int b = 0; b < 4; ++b) m->off[b] = -1;
        for (uint32_t i = 0; ok && i < h[8]; ++i) {
            uint32_t blk[3];
            ok = rd(f, blk, sizeof blk) && blk[0] >= 1 && blk[0] <= 4 && blk[2] == m->E;
            if (ok) m->off[blk[0] - 1] = (int32_t)blk[1];
        }
    }
    if (ok) {
        const size_t np = m->n_present, E = m->E;
        int32_t *layer_of = (int32_t *)malloc(4 * np + 4);
        m->prior = (float *)malloc(4 * np + 4);
        m->bias = (float *)malloc(4 * np * E + 4);
        m->w = (float *)malloc(4 * np * m->feat_dim * E + 4);
        ok = rd(f, layer_of, 4 * np) && rd(f, m->prior, 4 * np) && rd(f, m->bias, 4 * np * E) &&
             rd(f, m->w, 4 * np * m->feat_dim * E);
        m->index_of = (int32_t *)malloc(4 * (size_t)m->n_layers + 4);
        for (uint32_t l = 0; l < m->n_layers; ++l) m->index_of[l] = -1;
        for (size_t i = 0; ok && i < np; ++i) {
            ok = layer_of[i] >= 0 && (uint32_t)layer_of[i] < m->n_layers;
            if (ok) m->index_of[layer_of[i]] = (int32_t)i;
        }
        free(layer_of);
    }
    fclose(f);
    if (!ok) {
        or_moep_free(m);
        return NULL;
    }
    return m;
}

void or_moep_free(or_moep *m) {
    if (!m) return;
    free(m->index_of);
    free(m->prior);
    free(m->bias);
    free(m->w);
    free(m);
}

int or_moep_n_expert(const or_moep *m) { return (int)m->E; }

int or_moep_has_layer(const or_moep *m, int il) {
    return il >= 0 && (uint32_t)il < m->n_layers && m->index_of[il] >= 0;
}

void or_moep_score(const or_moep *m, int il, const or_moep_lists *in, float *out) {
    const uint32_t E = m->E;
    const int32_t row = m->index_of[il];
    const float *W = m->w + (size_t)row * m->feat_dim * E;
    memcpy(out, m->bias + (size_t)row * E, 4 * (size_t)E);
    for (int b = 0; b < 4; ++b) {
        if (m->off[b] < 0) continue;
        for (int i = 0; i < in->n[b]; ++i) {
            const int32_t e = in->ids[b][i];
            if (e < 0 || e >= (int32_t)E) continue;
            const float *r = W + (size_t)(m->off[b] + e) * E;
            for (uint32_t j = 0; j < E; ++j) out[j] += r[j];
        }
    }
    float mu = 0.0f;
    for (uint32_t j = 0; j < E; ++j) mu += out[j];
    mu /= (float)E;
    float var = 0.0f;
    for (uint32_t j = 0; j < E; ++j) {
        const float d = out[j] - mu;
        var += d * d;
    }
    const float sd = sqrtf(var / (float)E) + 1e-9f;
    for (uint32_t j = 0; j < E; ++j) out[j] = (out[j] - mu) / sd;
    const float pw = m->prior[row];
    if (pw != 0.0f)
        for (int i = 0; i < in->n[0]; ++i) {
            const int32_t e = in->ids[0][i];
            if (e >= 0 && e < (int32_t)E) out[e] += pw;
        }
}

/* k rounds of "the best remaining", a NaN score below every other */
int or_moep_top(const or_moep *m, const float *scores, int k, int32_t *out) {
    const int E = (int)m->E;
    if (k > E) k = E;
    if (k < 0) k = 0;
    uint8_t *used = (uint8_t *)calloc((size_t)E, 1);
    for (int r = 0; r < k; ++r) {
        int best = -1;
        for (int e = 0; e < E; ++e) {
            if (used[e]) continue;
            if (best < 0) { best = e; continue; }
            const float a = scores[e], b = scores[best];
            if (isnan(b) ? !isnan(a) : (!isnan(a) && a > b)) best = e;
        }
        used[best] = 1;
        out[r] = best;
    }
    free(used);
    return k;
}

float or_moep_update(or_moep *m, int il, const or_moep_lists *in, const int32_t *truth, int n_truth, float lr) {
    if (!or_moep_has_layer(m, il) || n_truth <= 0) return 0.0f;
    const uint32_t E = m->E;
    const int32_t row = m->index_of[il];
    float *s = (float *)malloc(4 * (size_t)E), *g = (float *)malloc(4 * (size_t)E);
    uint8_t *y = (uint8_t *)calloc((size_t)E, 1);
    or_moep_score(m, il, in, s);
    for (int i = 0; i < n_truth; ++i)
        if (truth[i] >= 0 && truth[i] < (int32_t)E) y[truth[i]] = 1;
    int32_t top[8];
    const int n = or_moep_top(m, s, 8, top);
    float hit = 0.0f;
    for (int i = 0; i < n; ++i) hit += y[top[i]] ? 1.0f : 0.0f;
    hit /= (float)n_truth;
    for (uint32_t j = 0; j < E; ++j) {
        const float p = 1.0f / (1.0f + expf(-s[j]));
        g[j] = (p - (y[j] ? 1.0f : 0.0f)) * lr;
    }
    float *W = m->w + (size_t)row * m->feat_dim * E;
    for (int b = 0; b < 4; ++b) {
        if (m->off[b] < 0) continue;
        for (int i = 0; i < in->n[b]; ++i) {
            const int32_t e = in->ids[b][i];
            if (e < 0 || e >= (int32_t)E) continue;
            float *r = W + (size_t)(m->off[b] + e) * E;
            for (uint32_t j = 0; j < E; ++j) r[j] -= g[j];
        }
    }
    float *bias = m->bias + (size_t)row * E;
    for (uint32_t j = 0; j < E; ++j) bias[j] -= g[j];
    free(s);
    free(g);
    free(y);
    return hit;
}
