/*
 * chain.c -- the ggml CPU expert chain and the weighted combine, restated.
 * TEST INFRASTRUCTURE ONLY (see oracle.h).
 *
 * Order of operations follows experiments/x2_cpu_expert_cost.cpp:115-156 (the
 * reference's own restatement of the engine's CPU chain): x -> Q8_K once; one
 * vec_dot per up and gate row; h = silu(gate) * up in fp32 (silu(g) =
 * g / (1 + exp(-g)), exp being the oracle's canonical or_expf, <= 2 ulp from
 * libm's expf, the same function the GPU kernels evaluate); h -> Q8_K; one
 * vec_dot per down row.  The combine is
 * out = sum_k w_k * y_k accumulated in k order (patches/0009-moe-sidecar.patch:
 * 697-703: experts = host_rows + cached_rows, times the weights, summed).
 *
 * Expert byte layout (the library's host store and slot pool): one expert is
 * [up: I rows x H/256 Q4_K blocks][gate: same][down: H rows x I/256 blocks].
 */
#include "oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

size_t or_expert_bytes(int H, int I, int down_type) {
    const size_t upb = (size_t)I * (H / OR_QK) * OR_Q4K_BYTES;
    const size_t db = (size_t)H * (I / OR_QK) * (down_type == OR_TYPE_Q4K ? OR_Q4K_BYTES : OR_Q6K_BYTES);
    return 2 * upb + db;
}

void or_expert_chain(int H, int I, int down_type, const void *up, const void *gate,
                     const void *down, const float *x, float *y, float *h_out) {
    const size_t rb_in = (size_t)(H / OR_QK) * OR_Q4K_BYTES;
    const size_t rb_dn = (size_t)(I / OR_QK) * (down_type == OR_TYPE_Q4K ? OR_Q4K_BYTES : OR_Q6K_BYTES);
    uint8_t *qx = (uint8_t *)malloc((size_t)(H / OR_QK) * OR_Q8K_BYTES);
    uint8_t *qh = (uint8_t *)malloc((size_t)(I / OR_QK) * OR_Q8K_BYTES);
    float *h = (float *)malloc((size_t)I * sizeof(float));
    or_quant_q8k(x, qx, H);
    for (int r = 0; r < I; ++r) {
        const float u = or_dot_q4k_q8k(H, (const uint8_t *)up + r * rb_in, qx);
        const float g = or_dot_q4k_q8k(H, (const uint8_t *)gate + r * rb_in, qx);
        h[r] = g / (1.0f + or_expf(-g)) * u;
    }
    or_quant_q8k(h, qh, I);
    for (int r = 0; r < H; ++r) {
        const uint8_t *row = (const uint8_t *)down + r * rb_dn;
        y[r] = down_type == OR_TYPE_Q4K ? or_dot_q4k_q8k(I, row, qh) : or_dot_q6k_q8k(I, row, qh);
    }
    if (h_out) memcpy(h_out, h, (size_t)I * sizeof(float));
    free(qx);
    free(qh);
    free(h);
}

void or_moe_layer(int H, int I, int down_type, int K, const void *const *experts,
                  const float *w, const float *x, float *out, int n_threads) {
    const size_t rb_in = (size_t)(H / OR_QK) * OR_Q4K_BYTES;
    const size_t rb_dn = (size_t)(I / OR_QK) * (down_type == OR_TYPE_Q4K ? OR_Q4K_BYTES : OR_Q6K_BYTES);
    const size_t up_bytes = (size_t)I * rb_in;
    const size_t q8x_b = (size_t)(H / OR_QK) * OR_Q8K_BYTES;
    const size_t q8h_b = (size_t)(I / OR_QK) * OR_Q8K_BYTES;
    uint8_t *qx = (uint8_t *)malloc(q8x_b);
    uint8_t *qh = (uint8_t *)malloc(q8h_b * (size_t)K);
    float *up = (float *)malloc(sizeof(float) * (size_t)I * K);
    float *gt = (float *)malloc(sizeof(float) * (size_t)I * K);
    float *h = (float *)malloc(sizeof(float) * (size_t)I * K);
    float *y = (float *)malloc(sizeof(float) * (size_t)H * K);
    if (n_threads < 1) n_threads = 1;
    or_quant_q8k(x, qx, H);
#pragma omp parallel num_threads(n_threads)
    {
#pragma omp for schedule(static) collapse(2)
        for (int k = 0; k < K; ++k) {
            for (int r = 0; r < 2 * I; ++r) {
                const uint8_t *e = (const uint8_t *)experts[k];
                if (r < I) up[k * I + r] = or_dot_q4k_q8k(H, e + (size_t)r * rb_in, qx);
                else gt[k * I + r - I] = or_dot_q4k_q8k(H, e + up_bytes + (size_t)(r - I) * rb_in, qx);
            }
        }
#pragma omp for schedule(static)
        for (int k = 0; k < K; ++k) {
            for (int r = 0; r < I; ++r) {
                const float g = gt[k * I + r];
                h[k * I + r] = g / (1.0f + or_expf(-g)) * up[k * I + r];
            }
            or_quant_q8k(h + (size_t)k * I, qh + (size_t)k * q8h_b, I);
        }
#pragma omp for schedule(static) collapse(2)
        for (int k = 0; k < K; ++k) {
            for (int r = 0; r < H; ++r) {
                const uint8_t *row = (const uint8_t *)experts[k] + 2 * up_bytes + (size_t)r * rb_dn;
                const uint8_t *q = qh + (size_t)k * q8h_b;
                y[(size_t)k * H + r] = down_type == OR_TYPE_Q4K ? or_dot_q4k_q8k(I, row, q)
                                                                : or_dot_q6k_q8k(I, row, q);
            }
        }
#pragma omp for schedule(static)
        for (int r = 0; r < H; ++r) {
            float acc = w[0] * y[r];
            for (int k = 1; k < K; ++k) acc = acc + w[k] * y[(size_t)k * H + r];
            out[r] = acc;
        }
    }
    free(qx);
    free(qh);
    free(up);
    free(gt);
    free(h);
    free(y);
}

void or_moe_tokens(int H, int I, int down_type, int T, int K, const void *store, size_t expert_bytes,
                   int n_store, const int32_t *ids, const float *w, const float *x, float *out,
                   float *h_out, int n_threads) {
    const size_t upb = (size_t)I * (H / OR_QK) * OR_Q4K_BYTES;
    if (n_threads < 1) n_threads = 1;
#pragma omp parallel num_threads(n_threads)
    {
        float *y = (float *)malloc(sizeof(float) * (size_t)H);
        float *h = (float *)malloc(sizeof(float) * (size_t)I);
#pragma omp for schedule(dynamic, 1)
        for (int t = 0; t < T; ++t) {
            float *o = out + (size_t)t * H;
            for (int k = 0; k < K; ++k) {
                const int e = ids[(size_t)t * K + k];
                if (e >= 0 && e < n_store) {
                    const uint8_t *b = (const uint8_t *)store + (size_t)e * expert_bytes;
                    or_expert_chain(H, I, down_type, b, b + upb, b + 2 * upb, x + (size_t)t * H, y, h);
                } else {
                    memset(y, 0, sizeof(float) * (size_t)H);
                    memset(h, 0, sizeof(float) * (size_t)I);
                }
                if (h_out) memcpy(h_out + ((size_t)t * K + k) * I, h, sizeof(float) * (size_t)I);
                const float wk = w[(size_t)t * K + k];
                for (int r = 0; r < H; ++r) {
                    const float v = (e >= 0 && e < n_store) ? wk * y[r] : 0.0f;
                    o[r] = k == 0 ? v : o[r] + v;
                }
            }
        }
        free(y);
        free(h);
    }
}

void or_dispatch(int T, int K, int E, const int32_t *ids, int32_t *counts,
                 int32_t *offsets, int32_t *perm) {
    memset(counts, 0, sizeof(int32_t) * (size_t)E);
    for (int i = 0; i < T * K; ++i) counts[ids[i]]++;
    offsets[0] = 0;
    for (int e = 0; e < E; ++e) offsets[e + 1] = offsets[e] + counts[e];
    int32_t *fill = (int32_t *)calloc((size_t)E, sizeof(int32_t));
    for (int i = 0; i < T * K; ++i) {
        const int e = ids[i];
        perm[offsets[e] + fill[e]++] = i;
    }
    free(fill);
}
