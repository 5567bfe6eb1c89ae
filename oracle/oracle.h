/*
 * oracle.h -- CPU restatement of the MoE decode hot path.
 *
 * TEST INFRASTRUCTURE ONLY.  Nothing in the product links, loads or calls this
 * code.  Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg
 * use it, and only to check the product's results (or, for the CPU baseline, as
 * the thing timed beside the GPU).
 *
 * What each part restates, and what pins it:
 *
 *   block codecs (Q4_K, Q6_K, Q8_K), quantize_q8k, dot_q4k_q8k, dot_q6k_q8k
 *       ggml at llama.cpp bccbacd (not vendored in the reference; the reference
 *       uses them through mul_mat_id, patches/0008-fused-cpu-moe-rows.patch:186-251
 *       and experiments/x2_cpu_expert_cost.cpp:115-156).  Restated from ggml's
 *       published block layouts.  Pinned by closed forms in tests/test_oracle_quants.py
 *       (integer exactness vs fp64 dequant-then-dot, all-zero / d=0 / dmin=0 /
 *       constant-code blocks, one-hot probes of every element position).
 *   or_expf, or_route
 *       build_moe_ffn's softmax -> (+ cache prior, patches/0007-...patch:109-124)
 *       -> argsort top-k -> get_rows -> renormalise.  Upstream reduction order and
 *       tie order are unpinned; this file fixes a canonical order (below) that the
 *       GPU router follows bit for bit.  Pinned by brute force against fp64
 *       softmax/sort on random and tie-heavy inputs, and by the reference's own
 *       integer-valued top-k case (cpp/test-moe-sidecar.cpp:155-217: lower id
 *       wins a tie).
 *   or_expert_chain, or_moe_layer, or_moe_tokens
 *       ggml CPU expert chain: quantize x to Q8_K once, one integer vec_dot per
 *       gate/up row, SwiGLU in fp32, quantize h to Q8_K, one vec_dot per down
 *       row (experiments/x2_cpu_expert_cost.cpp:115-156), weighted combine in k
 *       order (patches/0009-moe-sidecar.patch:697-703).  Pinned by fp64
 *       dequantise-then-dot on the same quantized operands.
 *   or_dispatch
 *       ggml mul_mat_id row mapping (per-expert counts + rows in (token, k)
 *       order, patches/0008-...patch:157-167 context).  Pinned by brute force.
 *   or_cache_*
 *       the slot-table state machine of patches 0006+0007+0008
 *       (observe: 0006:295-400, 0007:247-321, 0008:504-518; step: 0006:765-953,
 *       0007:655-771, 0008:607-660; admission 0007:398-429; tables 0007:327-396;
 *       map/route traces 0008:417-518).  Pinned by replaying the routes of the
 *       reference's engine-recorded traces
 *       (artifacts/x3_logits_1791160431756057451/{0..3}.routes-record.txt) and
 *       requiring every placement frame of {0..3}.map.txt.
 *   _ref/libref_predictor.so (ref_predictor_shim.cpp + the reference's own
 *       cpp/moe-predictor.cpp, built from where it lies by `make ref`)
 *       the MOEP predictor itself, not restated: what the product's
 *       moe_predictor_* is compared with (tests/test_moep.py, tests/golden/make_moep_golden.py).
 *   or_ahead, or_planner_*
 *       router lookahead (k_moe_ahead_scores/post, patches/0010-team-and-streaming.patch:382-474)
 *       and the just-in-time copy planner (moe_planner, 0010:777-909).  or_ahead is
 *       pinned by brute-force ranking (fp64 scores of the same products, crafted
 *       ties) and the table filter; the planner by the reference's own planner
 *       cases (cpp/test-moe-planner.cpp) and brute-force EDF checks.
 *
 * Canonical router order (shared with the GPU kernel):
 *   logit[e]  = s_0 + s_1 + s_2 + s_3 (left to right) over the row's four
 *               quarters of Q = H/4 values; s_q: 64 lane partials p_j, p_j
 *               accumulated with fmaf (from 0) over i = 0..Q/256-1, c = 0..3
 *               of W[e][Q q + 256 i + 4 j + c] * x[...], then a butterfly
 *               p_j += p_{j^o} for o = 1,2,4,8,16,32.  (H a multiple of 1024.)
 *   (+ bias[e], one fp32 add, when a steering bias is given)
 *   m         = max_e logit[e]
 *   ex[e]     = or_expf(logit[e] - m)
 *   s         = per 64-expert chunk the same butterfly sum, chunks added in order.
 *   p[e]      = ex[e] / s
 *   sel[e]    = p[e] + prior[e]           (only when a prior table is given;
 *               logit[e] + prior[e] in the logits-space variant)
 *   ids       = k largest sel, descending, lower id first on equal values
 *   wsum      = p[ids[0]] + p[ids[1]] + ... (left to right)
 *   w[k]      = p[ids[k]] / wsum
 */
#ifndef MOE_ORACLE_H
#define MOE_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define OR_QK 256
#define OR_Q4K_BYTES 144
#define OR_Q6K_BYTES 210
#define OR_Q8K_BYTES 292

enum { OR_TYPE_Q4K = 12, OR_TYPE_Q6K = 14 };  /* ggml type ids */

/* ---- fp16 ------------------------------------------------------------- */
float    or_h2f(uint16_t h);
uint16_t or_f2h(float f);

/* ---- block codecs ------------------------------------------------------ */
void  or_dequant_q4k(const void *blocks, float *y, int64_t n);
void  or_dequant_q6k(const void *blocks, float *y, int64_t n);
void  or_quant_q8k(const float *x, void *blocks, int64_t n);
void  or_dequant_q8k(const void *blocks, float *y, int64_t n);
/* one row of n weights against one Q8_K-quantized vector of n values */
float or_dot_q4k_q8k(int n, const void *w, const void *q8);
float or_dot_q6k_q8k(int n, const void *w, const void *q8);
/* fp64 reference of the same two products: dequantize both, dot in double */
double or_dot_deq_f64(int wtype, int n, const void *w, const void *q8);

/* ---- router ------------------------------------------------------------ */
float or_expf(float x);
/* W [E][H] row-major f32, x [H].  bias/prior/table may be NULL.
 * Writes ids[K], w[K]; slots[K] = table[ids[k]] when table and slots given;
 * probs[E] when given.  H % 256 == 0, E % 64 == 0, K <= E. */
void or_route(int E, int H, int K, const float *W, const float *x, const float *bias,
              const float *prior, const int32_t *table, int32_t *ids, float *w,
              int32_t *slots, float *probs);
/* as or_route; prior_on_logits = 1 adds the prior to the logits for the
 * selection instead of to the probabilities (weights stay unbiased) */
void or_route_space(int E, int H, int K, const float *W, const float *x, const float *bias,
                    const float *prior, int prior_on_logits, const int32_t *table, int32_t *ids,
                    float *w, int32_t *slots, float *probs);
/* softmax/top-k part only, from given logits (batched prefill input) */
void or_route_logits(int E, int K, const float *logits, const float *prior,
                     int32_t *ids, float *w, float *probs);

/* ---- expert chain ------------------------------------------------------ */
/* One expert at batch 1.  up/gate: Q4_K [I rows][H/256 blocks];
 * down: Q4_K or Q6_K [H rows][I/256 blocks].  y[H]. h_out[I] optional. */
void or_expert_chain(int H, int I, int down_type, const void *up, const void *gate,
                     const void *down, const float *x, float *y, float *h_out);
/* K experts + weighted combine: out[H] = sum_k w[k] * y_k (k in order).
 * experts[k] points at that expert's contiguous [up | gate | down] bytes.
 * n_threads > 1 parallelises rows with OpenMP (the CPU baseline). */
void or_moe_layer(int H, int I, int down_type, int K, const void *const *experts,
                  const float *w, const float *x, float *out, int n_threads);
size_t or_expert_bytes(int H, int I, int down_type);
/* A batch of T tokens: token t through experts ids[t][k] of a [n_store][expert_bytes]
 * store (an id outside it contributes zero), out[t] = sum_k w[t][k] y_{t,k} in k
 * order -- or_moe_layer's combine -- with OpenMP over tokens.  h_out [T][K][I]
 * (optional) receives each pair's SwiGLU activations. */
void or_moe_tokens(int H, int I, int down_type, int T, int K, const void *store, size_t expert_bytes,
                   int n_store, const int32_t *ids, const float *w, const float *x, float *out,
                   float *h_out, int n_threads);

/* ---- dispatch ---------------------------------------------------------- */
/* ids [T][K].  counts[E], offsets[E+1] (exclusive scan), perm[T*K]:
 * perm[offsets[e] + j] = t*K + k of the j-th pair routed to e, (t, k) order. */
void or_dispatch(int T, int K, int E, const int32_t *ids, int32_t *counts,
                 int32_t *offsets, int32_t *perm);

/* ---- slot-table state machine ------------------------------------------ */
typedef struct or_cache or_cache;

typedef struct {
    int32_t max_inserts;     /* default 2 */
    int32_t admit_mode;      /* 0 off, 1 heat, 2 window */
    int32_t admit_window;    /* default 8 */
    int32_t admit_half;      /* default 64 */
    float   admit_floor;     /* default 1.0 */
    int32_t batch_tables;    /* 0/1 */
    int32_t early_issue;     /* 0/1 */
    float   cache_prior;     /* delta, 0 = off */
    int32_t deterministic;   /* 1: publish in (layer, slot) order; 0: in scheduling order */
} or_knobs;

typedef struct {
    uint64_t n_steps, clock, n_hit, n_miss, n_uploads, n_scheduled, n_published,
             n_admit_ok, n_admit_denied, n_table_flushes;
} or_stats;

/* slots[l] = slot count of layer l (layer il = l). */
or_cache *or_cache_create(int n_layers, int n_experts, const int32_t *slots, const or_knobs *k);
void      or_cache_destroy(or_cache *c);
/* open trace writers (either may be NULL); writes the map header and frame 0 */
int       or_cache_trace_open(or_cache *c, const char *route_path, const char *map_path);
/* ids token-major [n_tok][n_ids] */
void      or_cache_observe(or_cache *c, int layer, const int32_t *ids, int n_ids, int n_tok);
void      or_cache_step(or_cache *c);
/* hold the job (layer, expert, slot) scheduled at step `sched_step` back for
 * one extra step: models an upload still copying at a live-mode boundary */
void      or_cache_hold_job(or_cache *c, int layer, int expert, int slot, uint64_t sched_step);
/* published placement of a layer: out[slot] = expert or -1 */
void      or_cache_frame(const or_cache *c, int layer, int32_t *out);
/* table mirror (expert -> slot or dummy) and prior mirror of a layer */
void      or_cache_table(const or_cache *c, int layer, int32_t *tbl, float *prior);
void      or_cache_stats(const or_cache *c, or_stats *s);
/* heat file (0007:431-485, warm start 0007:568-621, save 0007:745-752): counts of
 * every observed id, saved every 512 steps; on load halved, and the hottest
 * experts placed in slots 0.. before the first token.  Returns 0 (records and
 * placed experts in *n_records, *n_placed), -1 when the file cannot be used
 * (a refused header counts as zero records, as in the reference). */
int       or_cache_heat_file(or_cache *c, const char *path, long long *n_records, long long *n_placed);
/* LLAMA_MOE_CACHE_FREEZE (0008:825-832): no uploads from now on */
void      or_cache_freeze(or_cache *c);
/* LLAMA_MOE_MAP_REPLAY (0008:436-474, 559-565): force every step's recorded
 * placement; freezes the cache.  Returns 0, or -1 for a header that does not
 * match; or_cache_replay_error() != 0 once a frame was missing or malformed. */
int       or_cache_map_replay(or_cache *c, const char *path);
int       or_cache_replay_error(const or_cache *c);

/* ---- router lookahead and the copy planner (stream.c) ---------------------
 * or_ahead: the k best experts of target router W [E][H] applied to x * r
 * (best first, lower id on a tie, a NaN ranks with -inf), keeping those with
 * table[e] == dummy; returns how many were kept (ids[0..n-1]), -1 on bad sizes.
 * scores_out[E] (optional) receives the scores. */
int or_ahead(int E, int H, int k, const float *W, const float *x, const float *r,
             const int32_t *table, int32_t dummy, float *scores_out, int32_t *ids);

enum { OR_DROP_NONE = 0, OR_DROP_LATE = 1, OR_DROP_POSTED = 2 };
typedef struct or_planner or_planner;
typedef struct {
    int job;
    size_t offset, len;
    int last;
} or_chunk;
typedef struct {
    int target;
    int32_t expert;
    size_t bytes, sent;
    uint64_t deadline_ns;
    int dropped, drop;
} or_planner_job;
or_planner *or_planner_create(size_t chunk_bytes);
void or_planner_destroy(or_planner *p);
void or_planner_reset(or_planner *p);
/* the new job's id, or -1 (a job exists -- an earlier deadline tightens it --
 * or the target has read its table) */
int  or_planner_offer(or_planner *p, int target, int32_t expert, size_t bytes, uint64_t deadline_ns);
void or_planner_posted(or_planner *p, int target);
/* 1 and the next chunk in *out, or 0 when nothing can go now */
int  or_planner_next(or_planner *p, uint64_t free_at_ns, double bytes_per_ns, int hold_after, or_chunk *out);
int  or_planner_size(const or_planner *p);
void or_planner_get(const or_planner *p, int id, or_planner_job *out);
/* offered, duplicates, dropped late, dropped posted */
void or_planner_counters(const or_planner *p, uint64_t out[4]);

/* ---- just-in-time streaming in the state machine (0010) -------------------
 * Enable before any map trace is opened (chunk_bytes: largest copy per push,
 * 0 = 512 KiB, the reference's); needs early_issue and batch_tables,
 * and neither deterministic publication, replay nor freeze (-1 otherwise).
 * take: one lookahead record of source layer `layer` (targets[2], n[2],
 * ids[2][8]) at host time now_ns and GPU time t_ns; returns the jobs created.
 * posted: `layer` has read its table.  next: the planner's next chunk
 * (returns 0 when none).  land: job's copy and table word have landed.
 * observe_gpu: batch-1 observation with the slots the GPU used (n_slots =
 * absent), which also accounts streamed experts as in time or late.
 * stats: records, offered, landed, in time, late, unused, dropped late,
 * dropped posted, not sent (no free slot), GPU misses, bytes. */
int  or_cache_stream_enable(or_cache *c, int per_layer, int reserve, double gbps, size_t chunk_bytes);
int  or_cache_stream_take(or_cache *c, int layer, const int32_t *targets, const int32_t *n, const int32_t *ids,
                          uint64_t now_ns, uint64_t t_ns, size_t expert_bytes);
void or_cache_stream_posted(or_cache *c, int layer);
int  or_cache_stream_next(or_cache *c, uint64_t free_at_ns, int hold_after, or_chunk *out);
void or_cache_stream_land(or_cache *c, int job);
int  or_cache_stream_job(const or_cache *c, int job, int32_t *layer, int32_t *expert);
void or_cache_observe_gpu(or_cache *c, int layer, const int32_t *ids, const int32_t *gslots, int n_ids);
void or_cache_stream_stats(const or_cache *c, uint64_t out[11]);


/* ---- the MOEP predictor / evictor (moep.c; cpp/moe-predictor.cpp) ---------
 * Lists in block order prev, cur, below, self_prev (n = 0: absent).  load
 * returns NULL for a file it cannot use (PCA models included). */
typedef struct or_moep or_moep;
typedef struct {
    const int32_t *ids[4];
    int n[4];
} or_moep_lists;
or_moep *or_moep_load(const char *path);
void  or_moep_free(or_moep *m);
int   or_moep_n_expert(const or_moep *m);
int   or_moep_has_layer(const or_moep *m, int il);
void  or_moep_score(const or_moep *m, int il, const or_moep_lists *in, float *out);
int   or_moep_top(const or_moep *m, const float *scores, int k, int32_t *out);
float or_moep_update(or_moep *m, int il, const or_moep_lists *in, const int32_t *truth, int n_truth, float lr);

/* ---- the predictor's and evictor's hooks in the state machine (0006:295-427,
 * 0006:765-900, 0007:149-318, 0007:655-724) ------------------------------------
 * set_predictor: with early issue, after each layer is observed the
 * predictor scores the next layer from (its previous ids, this layer's ids)
 * and issues up to predict_top speculative uploads there, keeping max_inserts
 * free slots for the demand path; online_lr > 0 resolves each prediction
 * against the ids the target layer then routes to (one SGD step; the model is
 * the caller's and is updated in place).  A predictor turns early issue on.
 * set_evictor: victims are the lowest score of the evictor (recency breaks
 * ties) in both the scheduling and the pool top-up.  set_spec_probation:
 * speculative uploads are published with the oldest recency and protected
 * from eviction for one step.  Borrowed models: keep them alive while set. */
void or_cache_set_predictor(or_cache *c, or_moep *m, int predict_top, float online_lr);
void or_cache_set_evictor(or_cache *c, or_moep *m);
void or_cache_set_spec_probation(or_cache *c, int on);
/* resolved predictions, the sum of their recall@8, speculative uploads issued */
void or_cache_predictor_stats(const or_cache *c, uint64_t *n_updates, double *recall_sum, uint64_t *n_spec);

#ifdef __cplusplus
}
#endif
#endif
