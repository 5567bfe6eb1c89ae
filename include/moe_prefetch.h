/*
 * moe_prefetch.h -- C ABI of the MI355X MoE decode hot path (libmoeprefetch.so).
 *
 * Plain pointers, sizes and int status codes; no C++ or torch types.  Device
 * pointers are HIP device (HBM) addresses, `stream` is a hipStream_t passed as
 * void* (null = the default stream).  Every call is safe to make from one
 * host thread at a time per handle; calls on different handles are
 * independent.
 *
 * Reference interfaces each entry point replaces (paths relative to the
 * reference repository; patch line numbers are inside the .patch files):
 *   moe_memcpy_h2d_batch    ggml_backend_cuda_memcpy_h2d_batch, patches/0006-online-predictor-batched-uploads-slot-profile.patch:52-87
 *   moe_cache_create        llama_moe_cache_init, patches/0006-...:482-763 (knobs 0006:501-539, 0007:492-506, 0008:536-569)
 *   moe_cache_destroy       llama_moe_cache_shutdown (owner-scoped teardown), patches/0009-moe-sidecar.patch:1021-1056
 *   moe_cache_lookup        llama_moe_cache_lookup, patches/0008-fused-cpu-moe-rows.patch:1310 context (llama-moecache.h:60-70)
 *   moe_cache_observe       moe_obs_cb (ggml_set_moe_obs_callback), patches/0006-...:295-400, 0007:247-321, 0008:504-518
 *   moe_cache_step          llama_moe_cache_step, patches/0006-...:765-953, 0007:655-771, 0008:607-660
 *   moe_cache_requires_sync llama_moe_cache_requires_sync, patches/0008-...:362-369, 601-605
 *   moe_cache_trace_open    LLAMA_MOE_ROUTE_TRACE / LLAMA_MOE_MAP_RECORD writers, patches/0008-...:417-518
 *   moe_cache_stats         LLAMA_MOE_STATS counters, patches/0006-...:928-953, 0007:758-770
 *   moe_route               build_moe_ffn router: mul_mat(ffn_gate_inp) -> soft_max -> (+ prior, 0007:109-124)
 *                           -> argsort_top_k -> get_rows -> normalise (llama.cpp llama-graph.cpp, un-vendored)
 *   moe_experts             build_moe_ffn expert chain: mul_mat_id(up/gate) -> swiglu -> mul_mat_id(down)
 *                           -> mul(weights) -> sum over k (0008:372-390, 0009:684-704; CPU twin ggml_cpu_moe_rows 0008:186-251)
 *   moe_decode_layer        one cached MoE layer of the decode graph (0009:659-705)
 *   moe_cache_set_shared    the shared-expert FFN build_moe_ffn's callers add beside the routed
 *                           experts (ffn_*_shexp; llama.cpp, un-vendored), always resident
 *   moe_decode_token        llama_context::decode for one token over every cached layer followed by
 *                           llama_moe_cache_step (0008:362-369)
 *   moe_decode_batch        the same for a batch of tokens: the observe callback sees ids [n_tok][K]
 *                           token-major (0006:295-400); the reference's cached graph handles one token
 *                           (0007:114); here batches are served from the same slots
 *   moe_pool_*              the slab/slot store behind src/prefetch_engine.py ExpertCache (:45-168)
 *   moe_dispatch            ggml mul_mat_id's batch row mapping (per-expert counts + mmid_row_mapping,
 *                           visible in 0008:157-167): histogram, exclusive scan, stable (token, k) order
 *   moe_grouped_experts     build_moe_ffn at n_tokens > 1: mul_mat_id(up/gate) -> swiglu ->
 *                           mul_mat_id(down) -> mul(weights) over the dispatched pairs (un-vendored upstream;
 *                           the reference's cache path stops at one token, 0007:114)
 *   moe_combine             the sum over k of the weighted expert rows (0009:697-703, order per 0009:355)
 *   moe_quant_rows          ggml's quantize_row_q8_K of the activations, in the form the matrix cores read
 * No counterpart in the reference: moe_host_alloc/free (the reference pins the model buffer
 * through ggml's CUDA_Host buffer type), moe_synth_* (seeded synthetic weights and inputs).
 */
#ifndef MOE_PREFETCH_H
#define MOE_PREFETCH_H

#include <stdbool.h>
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- status ------------------------------------------------------------ */
#define MOE_OK          0
#define MOE_ERR_ARG    -1   /* bad argument or unsupported shape */
#define MOE_ERR_HIP    -2   /* a HIP runtime call failed */
#define MOE_ERR_NOMEM  -3   /* allocation failed */
#define MOE_ERR_STATE  -4   /* call not valid in the current state */
#define MOE_ERR_IO     -5   /* trace file could not be opened or written */
#define MOE_ERR_TIMEOUT -6  /* an upload did not finish in time */

#define MOE_TYPE_Q4K 12     /* ggml type ids */
#define MOE_TYPE_Q6K 14

#define MOE_DTYPE_F32  0    /* activation element types */
#define MOE_DTYPE_BF16 1

const char *moe_last_error(void);   /* message of the last failure on this thread */
int moe_abi_version(void);

/* ---- host memory -------------------------------------------------------- */
/* Pinned host memory, mapped for device access (the expert store). */
void *moe_host_alloc(size_t bytes);
int moe_host_free(void *p);
/* Device address of pinned host memory from moe_host_alloc (NULL if it is not
 * device-mapped).  Kernels read absent experts through this address. */
void *moe_host_device_ptr(void *host);
/* HBM allocations for callers without a device allocator of their own. */
void *moe_device_alloc(size_t bytes);
int moe_device_free(void *p);
int moe_device_synchronize(void);
/* Synchronous copy between any two addresses the HIP runtime knows. */
int moe_memcpy(void *dst, const void *src, size_t bytes);

/* ---- batched host->device copy ----------------------------------------- */
/* n copies on this library's per-thread copy stream and ONE synchronise.
 * Returns false on any error, after synchronising; the caller treats the
 * whole batch as not done.  n <= 0 returns true. */
bool moe_memcpy_h2d_batch(int device, void **dst, const void **src, const size_t *sizes, int n);

/* ---- synthetic inputs (no counterpart in the reference) ------------------ */
/* Experts e0 .. e0+n-1 of `layer`, [up|gate|down] layout, each at out + e*stride.
 * Weights N(0, sigma) quantized to Q4_K (up, gate) and down_type (down). */
int moe_synth_experts(uint64_t seed, int layer, int e0, int n, int H, int I, int down_type,
                      float sigma, void *out_dev, size_t stride, void *stream);
int moe_synth_experts_host(uint64_t seed, int layer, int e0, int n, int H, int I, int down_type,
                           float sigma, void *out_host, size_t stride, int n_threads);
/* out[(a - a0)][(b - b0)][i] = value (kind, a, b, i), n values per (a, b).
 * kinds: 0 router rows (a = layer, b = expert), 1 activations (a = token, b = layer): N(0, sigma);
 *        2 router logits (a = token, b = layer): uniform on [0, sigma). */
int moe_synth_vec(uint64_t seed, int kind, int a0, int na, int b0, int nb, int n, float sigma,
                  float *out_dev, void *stream);
/* Measurement only (no counterpart in the reference): the average duration,
 * from dispatch-stamped events, of a plain streaming-read kernel over `bytes`,
 * each of `iters` launches reading a fresh window of the device buffer `buf`
 * (cold for the caches when buf_bytes is well above 256 MiB). */
int moe_probe_stream_read(const void *buf, size_t buf_bytes, size_t bytes, int iters, double *avg_us,
                          void *stream);
int moe_synth_vec_host(uint64_t seed, int kind, int a0, int na, int b0, int nb, int n, float sigma,
                       float *out_host);
size_t moe_expert_bytes(int H, int I, int down_type);

/* ---- kernels --------------------------------------------------------------- */
typedef struct {
    const float *W;        /* dev [E][H] router weights, f32 */
    const float *x;        /* dev [n_tok][H] */
    const float *bias;     /* dev [n_tok][E] or NULL: added to the logits */
    const float *prior;    /* dev [E] or NULL: added to the probabilities for selection only */
    const int32_t *table;  /* dev [E] or NULL: expert -> slot (n_slots = absent) */
    int32_t dummy;         /* slot written when table is NULL */
    int32_t prior_on_logits; /* 0: prior added to the probabilities (the reference's
                                LLAMA_MOE_CACHE_PRIOR); 1: added to the logits */
    int32_t E, H, K, n_tok;
    int32_t *ids;          /* dev out [n_tok][K], descending selection, lower id first on ties */
    float *w;              /* dev out [n_tok][K], probs[ids] / sum(probs[ids]) */
    int32_t *slots;        /* dev out [n_tok][K] */
    float *probs;          /* dev out [n_tok][E] or NULL */
    uint8_t *q8x;          /* dev out [n_tok][H/256] Q8_K blocks of x (292 B each); may be NULL
                              with given logits */
    void *workspace;       /* dev, moe_route_workspace_bytes(); zero before first use */
    const float *logits;   /* dev [n_tok][E] or NULL: given router logits (W and x unused for
                              them; bias still added) */
} moe_route_desc;

typedef struct {
    const int32_t *ids;       /* dev [K] */
    const int32_t *slots;     /* dev [K] */
    const float *w;           /* dev [K] */
    const uint8_t *slot_pool; /* dev [n_slots][slot_bytes] */
    uint64_t slot_bytes;
    int32_t n_slots;
    const uint8_t *host_store;  /* device address (moe_host_device_ptr) of the pinned
                                   [n_experts][expert_bytes] store; absent experts are read from it */
    uint64_t expert_bytes;
    int32_t n_experts;          /* experts in host_store; an id outside it contributes zero */
    const uint8_t *q8x;       /* dev [H/256] Q8_K of x (from moe_route) */
    float *out;               /* dev [H] */
    int32_t accumulate;       /* 1: out += sum_k w_k y_k */
    int32_t H, I, K, down_type;
    void *workspace;          /* dev, moe_experts_workspace_bytes(); zero before first use */
    const uint8_t *shared;    /* dev or NULL: an always-on shared expert ([up|gate|down], expert_bytes),
                                 weight 1, added after the K routed experts */
} moe_experts_desc;

size_t moe_route_workspace_bytes(int E, int n_tok);
size_t moe_experts_workspace_bytes(int I, int K);
int moe_route(const moe_route_desc *d, void *stream);
int moe_experts(const moe_experts_desc *d, void *stream);

/* The same expert chain on the host CPU (the reference's CPU path for
 * missed experts, P8:186-251 / experiments/x2_cpu_expert_cost.cpp:115-156):
 * rows[k][H] = W_down,k . Q8_K(silu(W_gate,k . x) * (W_up,k . x)) for the n
 * experts at host addresses experts[k] ([up][gate][down] bytes), given the
 * Q8_K of x (host, [H/256][292]).  n_threads workers (the caller included);
 * AVX-512 VNNI integer dots when the CPU has them, or the portable path
 * (portable != 0 forces it).  Results equal the device kernels' bit for bit.
 * The worker threads of each n_threads are started by the first call and kept;
 * calls from several threads run one at a time. */
int moe_cpu_experts(const void *const *experts, int n, const uint8_t *q8x, int H, int I, int down_type, float *rows,
                    int n_threads, int portable);
/* No counterpart in the reference (its sidecar serves one token).  The same
 * chain for groups of tokens that share an expert, as CPU-assisted batched
 * decode runs it: group k applies experts[k] to the next count[k] tokens of
 * q8x ([tokens][H/256][292]); rows [tokens][H].  Each block of an expert's
 * rows is read from memory once for all of its tokens; results equal
 * moe_cpu_experts token by token. */
int moe_cpu_experts_tokens(const void *const *experts, int n_groups, const int32_t *count, const uint8_t *q8x,
                           int H, int I, int down_type, float *rows, int n_threads);
int moe_cpu_has_vnni(void);

/* ---- cache runtime --------------------------------------------------------- */
typedef struct moe_cache moe_cache;

#define MOE_ADMIT_OFF    0
#define MOE_ADMIT_HEAT   1
#define MOE_ADMIT_WINDOW 2

#define MOE_PUBLISH_FIFO    0  /* wait for the previous step's copies, publish in scheduling order */
#define MOE_PUBLISH_SORTED  1  /* LLAMA_MOE_DETERMINISTIC=1: wait, publish in (layer, slot) order */
#define MOE_PUBLISH_LIVE    2  /* publish only copies already finished, in finishing order */

typedef struct {
    int32_t n_layers, n_experts, n_expert_used;  /* L, E, K */
    int32_t hidden, intermediate;                /* H (2048), I (256, 512 or 768) */
    int32_t n_slots;                             /* default slots per layer (--moe-expert-cache) */
    const int32_t *slot_profile;                 /* [n_layers] slots per layer or NULL (LLAMA_MOE_SLOT_PROFILE) */
    const int32_t *down_type;                    /* [n_layers] MOE_TYPE_* or NULL = all Q4_K */
    int32_t max_inserts;                         /* --moe-expert-cache-inserts, default 2 */
    int32_t admit_mode;                          /* LLAMA_MOE_ADMIT */
    int32_t admit_window;                        /* LLAMA_MOE_ADMIT_WINDOW, default 8 */
    int32_t admit_half;                          /* LLAMA_MOE_ADMIT_HALF, default 64 */
    float admit_floor;                           /* LLAMA_MOE_ADMIT_FLOOR, default 1 */
    int32_t batch_tables;                        /* LLAMA_MOE_BATCH_TABLES */
    int32_t early_issue;                         /* LLAMA_MOE_EARLY_ISSUE */
    float cache_prior;                           /* LLAMA_MOE_CACHE_PRIOR (delta) */
    int32_t prior_on_logits;                     /* 0: delta on probabilities (the reference), 1: on logits */
    int32_t publish;                             /* MOE_PUBLISH_*; LLAMA_MOE_DETERMINISTIC=1 is SORTED */
    int32_t device;                              /* HIP device; < 0: state machine only (no GPU, no
                                                    weights: every upload completes at once) */
} moe_cache_config;

typedef struct {
    uint64_t n_steps, clock, n_hit, n_miss, n_uploads, n_scheduled, n_copied, n_published;
    uint64_t n_admit_ok, n_admit_denied, n_table_flushes;
    uint64_t bytes_uploaded;
    double publication_wait_us;                  /* time step() spent waiting for copies */
    uint64_t n_staged;                           /* uploads copied from the HBM staging area */
    uint64_t n_cpu_served;                       /* absent experts computed on the host CPU */
    double sidecar_wait_us, sidecar_cpu_us;      /* host time waiting for the GPU's posts / computing */
    double host_boundary_us;                     /* batch-1 decode: host time after the token's GPU work
                                                    (observe, step, table flush) before it returns */
    uint64_t n_evicted;                          /* resident experts evicted by the steps for uploads */
    /* with moe_cache_set_upload_stats: finished uploads from the pinned store
     * (host to device) and from the staging area (device to device), and the
     * sum of their copies' durations on the upload streams (events recorded
     * around each copy) */
    uint64_t n_upload_h2d, n_upload_d2d;
    double upload_h2d_us, upload_d2d_us;
} moe_cache_stats;

typedef struct {
    int32_t il, n_slots, n_experts, down_type;
    uint64_t slot_bytes, expert_bytes;
    uint8_t *slot_pool;         /* dev [n_slots][slot_bytes] */
    int32_t *dev_table;         /* dev [E]: slot or n_slots */
    float *prior;               /* dev [E] or NULL when cache_prior == 0 */
    const uint8_t *host_store;  /* registered pinned store or NULL */
    const float *router;        /* registered router weights or NULL */
} moe_layer_view;

int moe_cache_create(const moe_cache_config *cfg, moe_cache **out);
int moe_cache_destroy(moe_cache *c);
/* register caller-owned memory: pinned [E][expert_bytes] store, device [E][H] router */
int moe_cache_set_host_store(moe_cache *c, int layer, const void *experts, size_t expert_bytes);
int moe_cache_set_router(moe_cache *c, int layer, const float *W_dev);
/* Copy an always-on shared expert of `layer` into HBM (host or device source,
 * the layer's expert_bytes; NULL removes it).  Decoding adds it with weight 1
 * after the routed experts; the cache never evicts or counts it. */
int moe_cache_set_shared(moe_cache *c, int layer, const void *expert, size_t expert_bytes);
int moe_cache_lookup(moe_cache *c, int layer, moe_layer_view *out);
int moe_cache_trace_open(moe_cache *c, const char *route_path, const char *map_path);
/* host ids, token-major [n_tok][n_ids] */
int moe_cache_observe(moe_cache *c, int layer, const int32_t *ids, int n_ids, int n_tok);
/* between graph executions only: publish, schedule uploads, flush tables */
int moe_cache_step(moe_cache *c);
int moe_cache_requires_sync(const moe_cache *c);
int moe_cache_frame(moe_cache *c, int layer, int32_t *out);   /* out[slot] = expert or -1 */
int moe_cache_table(moe_cache *c, int layer, int32_t *tbl, float *prior);  /* host mirrors */
int moe_cache_stats_get(moe_cache *c, moe_cache_stats *out);
/* Per-upload timing (LLAMA_MOE_UPLOAD_STATS, patches/0006:689-703), off by
 * default: each upload's copy is bracketed by two events on its stream, read
 * when the step publishes it (the n_upload_* / upload_*_us statistics). */
int moe_cache_set_upload_stats(moe_cache *c, int on);
int moe_cache_sync(moe_cache *c);  /* wait for every upload in flight */
/* Heat file, LLAMA_MOE_HEAT_FILE (patches/0007:431-485 load/save, 568-621 warm
 * start, 745-752 periodic save): from now on every observed id is counted and
 * the counts are written to `path` every 512 steps ("moe-heat 1 <layers>
 * <experts>", then "<il> <expert> <count>"; via <path>.tmp and a rename).  If
 * `path` holds this cache's dimensions, its counts are loaded halved and the
 * hottest experts of every layer are copied into slots 0.. before the first
 * token (a reserve of max_inserts slots is kept free with early issue).  Call
 * after registering the host stores and before the first step. */
int moe_cache_heat_file(moe_cache *c, const char *path, int64_t *n_records, int64_t *n_placed);
/* LLAMA_MOE_CACHE_FREEZE (patches/0008:496-500, 825-832): no uploads from now on */
int moe_cache_freeze(moe_cache *c);
/* LLAMA_MOE_MAP_REPLAY (patches/0008:436-474, 559-565): every step ends with
 * the placement `path` recorded for it (a moe_cache_trace_open map file),
 * copying mismatched slots from the host store; freezes the cache.  Call
 * before the first step, after registering the stores; exclusive with a map
 * record.  A step whose frame is missing fails. */
int moe_cache_map_replay(moe_cache *c, const char *path);

/* ---- router lookahead and just-in-time streaming ---------------------------
 * LLAMA_MOE_STREAM (patches/0010-team-and-streaming.patch:957-1021 state,
 * 1096-1129 map record, 1183-1210 accounting, 1466-1760 take/reap/issue/
 * loop/adopt, 1671-1790 init).  Layer L's router launch also scores the
 * routers of layers L+1 and L+2 on L's input rescaled by g_T / g_L (which is
 * rmsnorm(residual_L) * g_T) and posts, per target, its top-k experts whose
 * table word is the dummy.  A host mover thread turns them into copies on its
 * own stream, earliest deadline first in 512 KiB chunks, dropping what would
 * land after the target reads its table; after an expert's last chunk it
 * writes the expert's table word (slot | STREAM_BIT) on the same stream.  The
 * GPU's kernels read the table at system scope and posts say which slot each
 * routed expert was read from, so an expert that landed in time is a hit of
 * this very token.  At the boundary the landed experts join the cache (routed
 * ones as recently used, the others as the first to go) and every word is
 * rewritten without the bit.  Batch-1 decode only. */
typedef struct {
    int32_t on;                /* 0 off, 1 on */
    int32_t per_layer;         /* LLAMA_MOE_STREAM_PER_LAYER, default 4: streamed experts per layer per token */
    int32_t reserve;           /* LLAMA_MOE_STREAM_RESERVE, default 2: extra free slots kept per layer */
    int32_t top_k;             /* LLAMA_MOE_STREAM_TOPK, default 8 (<= 8): candidates scored per target */
    double gbps;               /* LLAMA_MOE_STREAM_GBPS, default 45.7: the copy engine's rate for deadlines */
    int32_t chunk_kib;         /* LLAMA_MOE_STREAM_CHUNK_KIB (no counterpart in the reference): largest copy per push; 0 (default):
                                  a whole expert per push (the reference used 512 KiB) */
} moe_stream_config;

typedef struct {
    uint64_t records, offered, landed, in_time, late, unused, dropped_late, dropped_posted, not_sent,
             gpu_miss, bytes;
    double lead_us[3];         /* mean time from a prediction d layers ahead to its target's table read, d = 1, 2 */
    uint64_t lead_n[3];
    double tau_us;             /* the running estimate of GPU time per layer */
    int32_t failed;            /* a copy or channel error stopped streaming for this cache */
} moe_stream_stats;

/* The RMS-norm weight g_L [H] (host, copied) that produced layer L's router
 * input; the lookahead of L onto T uses g_T / g_L (a zero weight skips the
 * pair).  Set for every layer before moe_cache_set_streaming. */
int moe_cache_set_norm(moe_cache *c, int layer, const float *g_host, int n);
/* Needs early issue, no deterministic publication, replay or freeze, and no
 * open map record (the stream's map frames are written one step late); on a
 * live cache also the routers and norm weights of every layer.  On a host-only
 * cache (device < 0) it turns on the bookkeeping for the scripted calls below. */
int moe_cache_set_streaming(moe_cache *c, const moe_stream_config *cfg);
int moe_cache_stream_stats(moe_cache *c, moe_stream_stats *out);
/* Batch-1 observation with the slots the GPU read (n_slots = absent): the
 * route trace prints those slots, and streamed experts count as in time (the
 * GPU read their slot) or late.  The batch-1 decode uses it internally. */
int moe_cache_observe_gpu(moe_cache *c, int layer, const int32_t *ids, const int32_t *gpu_slots, int n_ids);
/* Scripted streaming on a host-only cache, the mover's steps one by one:
 * take one lookahead record of source `layer` (targets[2], n[2], ids[2][8])
 * at host time now_ns and GPU time t_ns, each job an expert of expert_bytes
 * (returns jobs created); posted: `layer` read its table; next: the next chunk
 * with the copy engine free at free_at_ns and jobs beyond hold_after held
 * (hold_after < 0: none) -- returns 1 and the chunk, 0 when none; land: the
 * job's last chunk and table word arrived; job: slot (and target layer,
 * expert) of a job, < 0 when none. */
typedef struct {
    int32_t job;
    uint64_t offset, len;
    int32_t last;
} moe_stream_chunk;
int moe_cache_stream_take(moe_cache *c, int layer, const int32_t *targets, const int32_t *n, const int32_t *ids,
                          uint64_t now_ns, uint64_t t_ns, uint64_t expert_bytes);
int moe_cache_stream_posted(moe_cache *c, int layer);
int moe_cache_stream_next(moe_cache *c, uint64_t free_at_ns, int hold_after, moe_stream_chunk *out);
int moe_cache_stream_land(moe_cache *c, int job);
int moe_cache_stream_job(moe_cache *c, int job, int32_t *layer, int32_t *expert);

/* The lookahead alone (k_moe_ahead_scores/_post, patches/0010:382-474), for
 * checking: runs the batch-1 router of d (n_tok 1) with n_targets (1..2)
 * target routers W[t] [E][H] (device), ratios r[t] [H] (device) and tables
 * tbl[t] [E] (device, dummy[t] = absent), and writes the record: out_n[t] and
 * out_ids[t][0..n-1] (host, int32 [2] and [2][8]), the top_k experts of
 * W[t] . (x * r[t]) with the dummy table word, best first, lower id on a tie.
 * Synchronous. */
typedef struct {
    int32_t n_targets, top_k;
    const float *W[2];
    const float *r[2];
    const int32_t *tbl[2];
    int32_t dummy[2];
} moe_ahead_desc;
int moe_route_ahead(const moe_route_desc *d, const moe_ahead_desc *a, int32_t *out_n, int32_t *out_ids,
                    void *stream);

/* The copy planner of the mover (moe_planner, patches/0010:777-909), exported
 * so that its decisions can be checked: offer returns a job id or -1; next
 * returns 1 and a chunk, or 0; get fills target, expert, bytes, sent,
 * deadline, dropped, drop reason (0 none, 1 late, 2 layer posted);
 * counters: offered, duplicates, dropped late, dropped posted. */
typedef struct moe_planner moe_planner;
typedef struct {
    int32_t target, expert;
    uint64_t bytes, sent, deadline_ns;
    int32_t dropped, drop;
} moe_planner_job;
moe_planner *moe_planner_create(uint64_t chunk_bytes);
void moe_planner_destroy(moe_planner *p);
void moe_planner_reset(moe_planner *p);
int moe_planner_offer(moe_planner *p, int target, int32_t expert, uint64_t bytes, uint64_t deadline_ns);
void moe_planner_posted(moe_planner *p, int target);
int moe_planner_next(moe_planner *p, uint64_t free_at_ns, double bytes_per_ns, int hold_after, moe_stream_chunk *out);
int moe_planner_size(const moe_planner *p);
int moe_planner_get(const moe_planner *p, int id, moe_planner_job *out);
void moe_planner_counters(const moe_planner *p, uint64_t out[4]);

/* ---- MOEP expert predictor / evictor (host) --------------------------------
 * moe_predictor of the reference (cpp/moe-predictor.h:35-106, .cpp:21-362):
 * per-layer linear scores over multi-hot id lists -- prev (the next layer's
 * ids of the previous token), cur (this layer's), below (the layer below's),
 * self_prev (this layer's previous ones) -- z-scored per row plus a repeat
 * prior on prev; top-k with the lower id first on a tie; a logistic SGD step
 * per resolved prediction; MOEP v3 files read strictly and written back.
 * Errors: a status code and moe_last_error(). */
typedef struct moe_predictor moe_predictor;
typedef struct {
    uint32_t n_expert, n_layers, feat_dim, top_k, d_model, n_comp, n_present;
    int32_t has_pca;
    int32_t off_pca, off_prev, off_cur, off_below, off_self_prev;   /* column offsets, -1 absent */
} moe_predictor_info;
typedef struct {
    const int32_t *ids[4];     /* prev, cur, below, self_prev (NULL: empty) */
    int32_t n[4];
} moe_predictor_lists;
int moe_predictor_load(const char *path, moe_predictor **out);
void moe_predictor_free(moe_predictor *p);
int moe_predictor_info_get(const moe_predictor *p, moe_predictor_info *out);
int moe_predictor_has_layer(const moe_predictor *p, int layer);
int moe_predictor_score(const moe_predictor *p, int layer, const moe_predictor_lists *in, float *out);
/* the k best ids of scores[n_expert], best first: returns how many (min(k, n_expert)) */
int moe_predictor_top_k(const moe_predictor *p, const float *scores, int k, int32_t *out);
/* one SGD step (learning rate lr) towards the ids `truth`; *recall = recall@8 before it */
int moe_predictor_update(moe_predictor *p, int layer, const moe_predictor_lists *in, const int32_t *truth,
                         int n_truth, float lr, float *recall);
int moe_predictor_save(const moe_predictor *p, const char *path);

/* The cache's use of the models (patches/0006:295-427 and 765-922,
 * patches/0007:149-168, 232-242, 330-355, 655-724; the reference's knobs
 * LLAMA_MOE_PREDICTOR, LLAMA_MOE_PREDICT_TOP, LLAMA_MOE_ONLINE_LR,
 * LLAMA_MOE_PREDICTOR_SAVE, LLAMA_MOE_EVICTOR, LLAMA_MOE_SPEC_PROBATION).
 * Models are borrowed: keep them alive until the cache is destroyed or the
 * hook is cleared (NULL).  Call between tokens.
 *
 * moe_cache_set_predictor: after each layer is observed, its model scores
 * the next layer from (the next layer's ids of the previous token, this
 * layer's ids); up to predict_top of the best absent experts are copied into
 * the next layer's spare slots (speculative uploads, never below max_inserts
 * spare slots; in heat admission each must be hotter than the expert it would
 * displace).  The spare pool kept at each step grows by predict_top.  Turns
 * early issue on.  online_lr > 0: each prediction is resolved against the ids
 * the layer then routes to with one SGD step on the model (updated in place);
 * save_path (or NULL): the model is written there every 200000 updates.
 * predict_top <= 0 or p NULL removes the predictor.
 * moe_cache_set_evictor: eviction victims are the lowest score of the model
 * (features: the next layer's previous ids, this layer's ids, the layer
 * below's, this layer's previous ones; recency breaks ties), in the step's
 * scheduling and in the early path's pool top-up; LRU for layers the model
 * lacks.  NULL restores LRU.
 * moe_cache_set_spec_probation: speculative uploads are published with the
 * oldest recency and cannot be evicted at their first step.
 * Errors: MOE_ERR_ARG for a model with a PCA block or a different expert count. */
int moe_cache_set_predictor(moe_cache *c, moe_predictor *p, int predict_top, float online_lr, const char *save_path);
int moe_cache_set_evictor(moe_cache *c, moe_predictor *p);
int moe_cache_set_spec_probation(moe_cache *c, int on);
/* resolved predictions, the sum of their recall@8, speculative uploads issued */
int moe_cache_predictor_stats(const moe_cache *c, uint64_t *n_updates, double *recall_sum, uint64_t *n_spec);

/* Kernel time of the decode, from HIP events stamped by each launch's
 * dispatch on the stream it runs on (off by default; set before decoding;
 * the token's launches then run eagerly).  With the fused layer (split 0)
 * layer_ms is filled; with split 3 route_ms, gateup_hbm_ms and
 * down_hbm_ms (one launch each, every expert); with splits 1 and 2 resident
 * and absent experts run as separate launches.  Bytes count the expert
 * weights the GPU read, by source (the host's share of absent experts under
 * CPU-assisted serving is not counted). */
typedef struct {
    double route_ms;                       /* route_logits + route_select */
    double gateup_hbm_ms, down_hbm_ms;     /* resident experts */
    double gateup_host_ms, down_host_ms;   /* absent experts (pinned store over PCIe) */
    uint64_t n_layers;                     /* layer decodes timed */
    uint64_t gateup_hbm_bytes, down_hbm_bytes, gateup_host_bytes, down_host_bytes;
    double layer_ms;                       /* split 0: the fused layer launch */
    uint64_t layer_hbm_bytes;              /* its router rows + resident (and shared) experts' bytes */
    uint64_t layer_host_bytes;             /* its absent experts' bytes read from the pinned store */
    /* moe_decode_batch: the grouped up/gate and down launches of the routed
     * experts (each layer's launches waited for: timing mode serialises the
     * host's share behind them); weights by source, one read per expert with
     * pairs on the GPU; pairs the GPU computed */
    double grouped_gateup_ms, grouped_down_ms;
    uint64_t grouped_launches, grouped_pairs;
    uint64_t grouped_gateup_hbm_bytes, grouped_down_hbm_bytes, grouped_gateup_host_bytes, grouped_down_host_bytes;
} moe_kernel_times;
int moe_cache_set_timing(moe_cache *c, int on);
/* split: 0 (default) the fused layer -- router GEMV, selection, every routed
 * expert's gate/up and down rows and the weighted combine in one launch,
 * resident and absent experts alike (moe_decode_token without streaming, and
 * moe_decode_layer; streaming uses split 3's launches);
 * 3 router GEMV, selection, gate/up and down as four launches; 1 resident and
 * absent experts as separate launches on two streams, forked and joined per
 * layer; 2 the same launches one after the other on one stream.
 * graph: 1 (default) replay each token's launches as one captured HIP graph,
 * except that a token of at most 8 layers without CPU-assisted serving or
 * streaming launches its layers directly: a graph launch costs ~30 us of
 * latency against ~11 us for a kernel launch (ROCm 7, MI355X), and direct
 * launches need no copies of x, out or the sequence number; 2 always the
 * graph; 0 always direct launches.  Timing mode launches directly.  Every
 * path gives the same bits.  MOE_ERR_ARG for split outside 0..3 or graph
 * outside 0..2. */
int moe_cache_set_decode_path(moe_cache *c, int split, int graph);
/* Bound of every wait inside the fused decode launch (default 0.5 s): a
 * workgroup that waits longer for another gives up and exits, and the token
 * fails with MOE_ERR_HIP (moe_decode_token, or moe_cache_step after per-layer
 * calls).  No counterpart in the reference, whose layer runs as separate
 * launches with no waits between workgroups; for callers that want failures
 * reported sooner, and for tests that force the give-up from the host.
 * MOE_ERR_ARG outside (0, 60]. */
int moe_cache_set_wait_bound(moe_cache *c, double seconds);
/* Staged uploads (default on; no counterpart in the reference, which uploads
 * from the host store, P6:428-440): moe_decode_token's kernels also write each
 * expert they read from the pinned store into an HBM staging area ([L][K]
 * experts, allocated at the first token), and an upload scheduled for one of
 * them in that token's step copies it device to device instead of over PCIe.
 * The bytes, slots, publication and traces are the same either way. */
int moe_cache_set_staging(moe_cache *c, int on);
/* CPU-assisted serving of absent experts (the reference's sidecar,
 * patches/0009: MOE_POST P9:277-320, MOE_JOIN P9:322-359, sidecar_serve
 * P9:841-912).  With n_threads > 0, the decode launches of moe_decode_token
 * and moe_decode_layer post each layer's logits (or ids) and Q8_K(x) to mapped
 * host memory; the calling thread and
 * n_threads - 1 workers compute the absent experts whose rank r among the
 * layer's absent experts (k order) has r % den < num, from the pinned store,
 * while the GPU runs the others; a join kernel waits (at most 2 s, bounded
 * by the GPU wall clock) for the host's rows and combines sum_k w_k y_k in k
 * order.  Outputs, ids and cache traces are identical to the GPU-only path.
 * Needs split 0 or 3.  n_threads <= 0 turns it off. */
int moe_cache_set_sidecar(moe_cache *c, int n_threads, int num, int den);
/* The serving channel's self-test (the reference's sidecar self-test before it
 * enables the sidecar, patches/0009:436-472, 914-925), over the exchange the
 * decode uses: in each of n_rounds a kernel posts a seeded pattern as tagged
 * words, the calling thread checks them and writes a row pattern back and
 * answers, the kernel checks the rows.  Every wait on either side is bounded by
 * timeout_s.  withhold_from >= 0: the host stops answering from that round on
 * (the kernel's bounded wait then ends it; for tests).  *n_bad receives the
 * failed exchanges; MOE_ERR_HIP when any failed.  moe_cache_set_sidecar runs
 * 10000 rounds the first time it is turned on and refuses, loudly, on a
 * failure (serving stays GPU-only). */
int moe_cache_sidecar_selftest(moe_cache *c, int n_rounds, int withhold_from, double timeout_s, int *n_bad);
/* CPU-assisted serving in moe_decode_batch (no counterpart in the reference,
 * whose sidecar serves one token, P9:841-912): per layer the routing comes
 * back to the host, which computes the pairs of the absent experts whose rank
 * r among the layer's absent experts (ascending id) has r % den < num -- each
 * expert's rows read once for all its tokens -- while the GPU's grouped
 * products skip them and read the other absent experts from the pinned store;
 * the combine then takes the host's weighted rows in k order.  The same
 * outputs, ids and traces.  num = den = 0 (the default): the share set by
 * moe_cache_set_sidecar.  Active while moe_cache_set_sidecar is on. */
int moe_cache_set_sidecar_batch(moe_cache *c, int num, int den);
/* Per served layer since the last call: (host wait us, host compute us,
 * experts computed), up to max_rows rows into out [rows][3]; returns rows. */
int moe_cache_sidecar_log(moe_cache *c, float *out, int max_rows);
int moe_cache_kernel_times(moe_cache *c, moe_kernel_times *out);

/* One layer at batch 1, the per-layer graph op (the cached chain and, with
 * CPU-assisted serving, its post and join, patches/0009:659-705): route x
 * (+bias), run the K experts, out = sum_k w_k y_k.  ids_dev/w_dev receive the
 * layer's routing (dev [K]) when not NULL.  Split 0 (the default) runs the
 * fused launch, split 3 the four launches.  Each call carries a sequence
 * number of its own, so a layer's input may be computed from the layer below
 * (x_{l+1} = x_l + out_l) between calls.  With CPU-assisted serving a call
 * returns once its layer is launched: the cache's server thread waits for the
 * layer's post, computes the host's share of its absent experts and answers,
 * layer after layer in call order, while the caller launches the next layers
 * (they queue behind the layer's join on the GPU, as a token's graph does).
 * A serving failure ends the joins of the layers still queued and is reported
 * by the next call, moe_cache_observe or moe_cache_step.
 * Drive a token as the reference does: every layer in order, the ids observed
 * (moe_cache_observe, after each layer or at the end; the call compares them
 * with the host's routing and stages the experts the kernels read from the
 * pinned store for the uploads), then moe_cache_step, which also checks the
 * launches' bounded waits (MOE_ERR_HIP if one ran out).  Calls of one cache
 * run one at a time on one stream; not with just-in-time streaming
 * (MOE_ERR_STATE: streaming decodes whole tokens). */
int moe_decode_layer(moe_cache *c, int layer, const float *x, const float *bias, float *out,
                     int32_t *ids_dev, float *w_dev, void *stream);
/* One decode token over every layer: x dev [L][H], bias dev [L][E] or NULL,
 * out dev [L][H]; then the routed ids come back (one copy), are observed in
 * layer order and the cache steps.  ids_host [L][K] receives them when not NULL.
 * The call returns with out complete in device memory.  When the layers are
 * launched directly without CPU-assisted serving or streaming (at most 8
 * layers, graph mode 0 or 1, no timing), the fused launches publish the ids
 * into mapped memory as tagged words and the call returns once all of them
 * carry the token's number, without synchronising the stream: the last launch
 * may still be retiring, and work enqueued later on the stream orders after it
 * as usual. */
int moe_decode_token(moe_cache *c, const float *x, const float *bias, float *out, int32_t *ids_host,
                     void *stream);

/* ---- batched path: prefill chunks and decode at batch > 1 ------------------- */
/* Dispatch of the (token, k) pairs of ids dev [n_tok][K] (pair i = t*K + k):
 * counts[e] pairs routed to expert e, offsets[e] = exclusive scan (offsets[E] =
 * pairs placed), perm[offsets[e] + r] = i of the r-th pair routed to e in pair
 * order.  Ids outside [0, E) are not placed.  E <= 256, n_tok * K <= 65535. */
int moe_dispatch(const int32_t *ids, int n_tok, int K, int E, int32_t *counts, int32_t *offsets,
                 int32_t *perm, void *stream);
/* Q8_K of n_rows rows of n values (n a multiple of 256), f32 or bf16: q16 the
 * int8 values as fp16 codes [n_rows][n], d the block scales [n_rows][n/256],
 * bsum16 the 16-value group sums as fp16 [n_rows][n/16].  All exact; the values
 * and scales are those of ggml's quantize_row_q8_K. */
int moe_quant_rows(const void *src, int src_type, int n_rows, int n, uint16_t *q16, float *d,
                   uint16_t *bsum16, void *stream);

typedef struct {
    const int32_t *offsets;     /* dev [E+1] from moe_dispatch */
    const int32_t *perm;        /* dev [n_tok*K] from moe_dispatch */
    const float *w;             /* dev [n_tok][K] gate weights */
    const void *x;              /* dev [n_tok][H] activations, MOE_DTYPE_F32 or MOE_DTYPE_BF16 */
    int32_t x_type;
    int32_t n_tok, K, E, H, I, down_type;
    const int32_t *table;       /* dev [E] slot per expert (>= n_slots: not resident) or NULL */
    const uint8_t *slot_pool;   /* dev [n_slots][slot_bytes] or NULL */
    uint64_t slot_bytes;
    int32_t n_slots;
    const uint8_t *store;       /* device address of [n_store][expert_bytes]: HBM, or pinned host
                                   memory through moe_host_device_ptr */
    uint64_t expert_bytes;
    int32_t n_store;            /* an expert neither resident nor in the store contributes zero */
    float *out;                 /* dev [n_tok][H] */
    int32_t accumulate;         /* 1: out += result */
    float *pair_out;            /* dev [n_tok*K][H] weighted expert rows in pair order, or NULL */
    float *h_out;               /* dev [n_tok*K][I] SwiGLU activations in dispatch order, or NULL */
    void *workspace;            /* dev, moe_grouped_workspace_bytes() */
    float *kernel_ms;           /* host [2] or NULL: when set the call waits for its kernels and
                                   stores the up/gate and down kernel durations (HIP events) */
    const uint8_t *shared;      /* dev or NULL: an always-on shared expert (expert_bytes), weight 1,
                                   added to every token after the routed experts */
} moe_grouped_desc;

size_t moe_grouped_workspace_bytes(int n_tok, int K, int H, int I);
/* Q8_K of x, up/gate over each expert's pairs with the SwiGLU, Q8_K of h, down
 * times the gate weight, and the sum over k (moe_combine) into out.  Every
 * pair must be placed by the dispatch (its id in [0, E)): the row of a pair
 * moe_dispatch left out is never written. */
int moe_grouped_experts(const moe_grouped_desc *d, void *stream);

/* No counterpart in the reference.  moe_grouped_experts for callers that
 * cannot allocate device memory (code under HIP graph capture, serving loops
 * and harnesses that forbid hipMalloc): the same kernels and results, with
 * the workspace in a static device array of MOE_GROUPED_STATIC_SCRATCH_BYTES
 * per device instead of d->workspace (which must be NULL; kernel_ms must be
 * NULL too).  Refuses, with MOE_ERR_ARG, a shape whose workspace
 * (moe_grouped_workspace_bytes) exceeds that: batch-64 decode at K = 8,
 * I = 768 needs 8.1 MiB (up to 126 tokens fit).  Calls no allocator.  Every call on one device
 * shares that device's array: calls that overlap on one device (two streams,
 * two threads) race and must be serialised by the caller. */
#define MOE_GROUPED_STATIC_SCRATCH_BYTES (16u << 20)
int moe_grouped_experts_static(const moe_grouped_desc *d, void *stream);
/* out[t] (+)= sum_k pair_rows[t*K + k], k ascending */
int moe_combine(const float *pair_rows, int n_tok, int K, int H, float *out, int accumulate, void *stream);

/* One decode step of n_tok tokens (batch > 1) over every layer: x dev [L][n_tok][H],
 * bias dev [L][n_tok][E] or NULL, out dev [L][n_tok][H].  Per layer: route (the
 * cache prior biases single-token selection only, so it applies when n_tok is 1,
 * patches/0007:114), dispatch, the grouped experts from HBM slots or the pinned
 * store, and the shared expert; then the routed ids come back in one copy, each
 * layer observes them token-major and the cache steps.  ids_host [L][n_tok][K]
 * receives them when not NULL.  n_tok <= 4096.  With CPU-assisted serving on, the
 * host computes its share of the absent experts when the share is not empty and
 * n_tok <= MOE_BATCH_HOST_MAX_TOKENS; larger batches run on the GPU alone. */
#define MOE_BATCH_HOST_MAX_TOKENS 64
int moe_decode_batch(moe_cache *c, const float *x, const float *bias, float *out, int n_tok, int32_t *ids_host,
                     void *stream);

/* ---- slab pool behind the Python ExpertCache ------------------------------- */
typedef struct moe_pool moe_pool;
int moe_pool_create(int n_layers, int capacity, size_t bytes_per_expert, int device, moe_pool **out);
int moe_pool_destroy(moe_pool *p);
/* async copy host -> slot on the pool's copy stream; records the slot's event */
int moe_pool_copy(moe_pool *p, int layer, int slot, const void *src_host, size_t bytes);
int moe_pool_ready(moe_pool *p, int layer, int slot);   /* 1 done, 0 in flight, <0 error */
int moe_pool_sync(moe_pool *p);
void *moe_pool_slot_ptr(moe_pool *p, int layer, int slot);

#ifdef __cplusplus
}
#endif
#endif
