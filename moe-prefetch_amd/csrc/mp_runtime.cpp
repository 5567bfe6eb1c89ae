// mp_runtime.cpp -- host side of libmoeprefetch.so: the C ABI, the per-layer
// expert-id -> slot state machine, uploads into the HBM slot pool on a side
// HIP stream, table publication, traces, and the batch-1 decode driver.
//
// State machine semantics follow llama-moecache.cpp as patched by 0006-0008 of
// the reference (file:line inside the .patch files):
//   observe   0006:295-400 (hit/miss, LRU clock, pending), 0007:247-321 (heat,
//             miss window), 0008:504-518 (route trace line)
//   issue     0006:241-293 early path; 0007:395-415 admission on it
//   step      0006:765-953, 0007:655-771: publish finished uploads, n_steps++,
//             per layer either schedule <= max_inserts uploads from the
//             pending misses (non-early) or top the free pool up (early),
//             heat decay, one batched table write
//   publish   0008:613-627 deterministic (sorted) variant
//   admission 0007:398-429; tables 0007:327-396; map trace 0008:417-489
// The data path is the library's own: one contiguous copy per expert
// ([up|gate|down] in the store and in the slot) on a dedicated stream,
// completion by hipEvent, tables in one pinned mirror flushed with one copy.
#include <hip/hip_runtime.h>
#include <immintrin.h>

#include <algorithm>
#include <array>
#include <atomic>
#include <chrono>
#include <condition_variable>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <deque>
#include <memory>
#include <map>
#include <mutex>
#include <string>
#include <thread>
#include <vector>

#include "../../include/moe_prefetch.h"
#include "mp_cpu.h"
#include "mp_format.h"
#include "mp_internal.h"
#include "mp_predictor.h"
#include "mp_stream.h"
#include "mp_synth.h"

namespace {

thread_local std::string g_err;

int fail(int code, const char *fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof buf, fmt, ap);
    va_end(ap);
    g_err = buf;
    return code;
}

#define HIPCHK(expr)                                                                            \
    do {                                                                                        \
        hipError_t e_ = (expr);                                                                 \
        if (e_ != hipSuccess) return fail(MOE_ERR_HIP, "%s: %s", #expr, hipGetErrorString(e_)); \
    } while (0)

constexpr uint64_t U64MAX = ~0ull;

size_t align_up(size_t v, size_t a) { return (v + a - 1) / a * a; }

struct Layer {
    int il = 0, S = 0, E = 0, down_type = mp::TYPE_Q4K;
    uint64_t expert_bytes = 0, slot_bytes = 0;
    uint8_t *pool = nullptr;                  // dev [S][slot_bytes]
    const uint8_t *store_host = nullptr;      // host address of the pinned store
    const uint8_t *store_dev = nullptr;       // device view of it
    const float *router = nullptr;
    uint8_t *shared = nullptr;                // dev: the always-on shared expert (owned) or null
    std::vector<int32_t> slot_expert, expert_slot, free_slots, pending;
    std::vector<int32_t> staged;              // [K] expert read from the store at k this token (staged), or -1
    std::vector<uint32_t> use_count;          // heat file: observations per expert (empty: no heat file)
    std::vector<uint64_t> slot_last_use, slot_protect, miss_last, miss_prev;
    std::vector<uint8_t> slot_in_flight;
    std::vector<float> heat;
    bool tbl_dirty = false;
    uint64_t n_hit = 0, n_miss = 0;
    // MOEP predictor / evictor (patches/0006:139-154): the ids this layer routed
    // to this token and the token before, and the features of the last
    // prediction made for this layer (resolved when the layer routes)
    std::vector<int32_t> cur_ids, prev_ids, pend_prev, pend_cur;
    bool pend_valid = false;
};

struct Job {
    int li, expert, slot;
    hipEvent_t ev;     // live mode only
    bool spec;         // issued from a prediction, not a miss (patches/0007:168)
    hipEvent_t t0 = nullptr, t1 = nullptr;   // upload statistics: around the copy on its stream
    bool staged = false;                     // a device-to-device copy from the staging area
};

// Just-in-time streaming (LLAMA_MOE_STREAM; state as in patches/0010:957-1021).
// One job per planner job, same index: the slot it took and what the GPU made
// of it.  Between tokens the mover thread is idle and the cache's own thread
// owns all of this; during a token only the mover touches it.
struct StreamJob {
    int li, slot, d;
    int64_t ticket;           // the push that carried the last chunk and the table word (live)
    bool landed, in_time, late;
};

enum { SN_RECORDS, SN_OFFERED, SN_LANDED, SN_IN_TIME, SN_LATE, SN_UNUSED, SN_DROP_LATE, SN_DROP_POSTED,
       SN_NOT_SENT, SN_GPU_MISS, SN_BYTES, SN_COUNT };

struct Streamer {
    int per_layer = 4, reserve = 2, top_k = 8;
    double bytes_per_ns = 45.7, tau_ns = 103000.0;
    uint64_t margin_ns = 5000;
    size_t max_outstanding = 1u << 20;
    mps::Planner planner{512 * 1024};
    std::vector<StreamJob> jobs;
    std::vector<int32_t> mark;                 // [layer][E]: job + 1 while streamed this token
    std::vector<int> n_this_token;             // [layer]
    uint32_t last_layer = UINT32_MAX;
    uint64_t last_t_ns = 0;
    uint64_t n[SN_COUNT] = {};
    double lead_sum[3] = {0, 0, 0};
    uint64_t lead_n[3] = {0, 0, 0};
    std::vector<uint64_t> arrive_ns;           // [layer]: host time its record arrived this token, 0 if not
    std::vector<int32_t> rec_frame;            // map record: the boundary's frame, held back one step
    uint64_t rec_step = 0;
    bool rec_have = false;
    std::vector<std::array<int32_t, 3>> rec_used;   // (layer, slot, expert) used in time this token
    // live mode (a GPU cache): lookahead launch arguments, the copy queue, the mover thread
    bool live = false;
    std::vector<std::array<int32_t, 2>> targets;    // [layer]: lookahead targets, -1 none
    float *ratio = nullptr;                    // dev [layer][2][H]: g_T / g_L
    float *alog = nullptr;                     // dev [2][E]
    uint32_t *fresh = nullptr;                 // dev [layer]
    mp::AheadPost *post = nullptr, *post_d = nullptr;   // mapped host [layer]
    int32_t *words = nullptr;                  // pinned [max slots]: s | STREAM_BIT, sources of table writes
    hipStream_t stream = nullptr;              // the copy queue
    std::vector<hipEvent_t> ev;                // ring of pushes
    std::vector<int64_t> ev_ticket;
    int ev_head = 0, ev_count = 0;
    int64_t next_ticket = 1, done_ticket = 0;
    std::deque<std::pair<int64_t, size_t>> outstanding;   // (ticket, bytes) pushed, not landed
    std::thread thr;
    std::mutex m;
    std::condition_variable cv, cv_done;
    uint32_t gen = 0, gen_done = 0;            // tokens started / drained (guarded by m)
    bool quit = false;                         // guarded by m
    std::atomic<bool> stop{false};             // the token's GPU work is over: drain
    std::atomic<bool> failed{false};
    uint32_t seq = 0;                          // the token's sequence number
};

}  // namespace

struct moe_predictor {
    mpp::Predictor p;
};

// The server of layers decoded one by one with CPU-assisted serving: each
// call queues its layer, and this thread serves the host's share of the
// layers in call order, so a call returns once its layer is launched and the
// caller's next launches queue behind it on the GPU, as a token's graph does.
struct PlServer {
    struct Job {
        int layer;
        uint32_t seq;
        bool fused;
    };
    std::thread th;
    std::mutex m;
    std::condition_variable cv, cv_idle;
    std::deque<Job> q;
    int busy = 0;                      // queued and being served
    bool quit = false;
    int err = 0;                       // the first failure (MOE_OK = 0: none), reported at the next sync point
    std::string msg;
};

struct moe_cache {
    moe_cache_config cfg{};
    bool host_only = false;            // device < 0: state machine only, no HIP calls
    std::vector<Layer> L;
    int H = 0, I = 0, E = 0, K = 0;
    // tables: device copies and pinned host mirrors, [L][E]
    int32_t *d_tbl = nullptr, *h_tbl = nullptr;
    float *d_prior = nullptr, *h_prior = nullptr;
    // kernel scratch
    void *route_ws = nullptr, *exp_ws = nullptr;
    float *ypart = nullptr;            // [K + 1][H]: per-expert down rows between the two launches of a split
    int32_t *d_ids = nullptr, *d_slots = nullptr, *h_ids = nullptr;
    uint64_t *h_pub = nullptr, *h_pub_d = nullptr;  // [L * K + 1] tagged words the fused launches publish
    uint64_t *d_pub_ctr = nullptr;      // [L]: the fused combine's count of finished workgroups
    bool pub_on = false;                // this token's fused launches publish ids and completion
    float *d_w = nullptr;
    uint8_t *d_q8x = nullptr;
    uint8_t *pool_base = nullptr;
    hipStream_t up_stream = nullptr, tbl_stream = nullptr;
    hipStream_t host_stream = nullptr;     // absent-expert launches (fork/join per layer)
    hipEvent_t ev_route = nullptr, ev_hbm = nullptr, ev_host = nullptr;
    hipEvent_t up_mark = nullptr;
    std::deque<Job> jobs;              // issued, not yet published, in issue order
    std::vector<hipEvent_t> free_events;
    // staged uploads: a decode token's kernels also write every expert they read
    // from the pinned store into stage [L][K][stage_stride] (HBM); an upload of
    // such an expert in the step that follows is a device-to-device copy on
    // stg_stream instead of a PCIe transfer.  The next token's kernels wait for
    // ev_stg before they overwrite the staging area.
    bool staging = true;
    uint8_t *stage = nullptr;
    size_t stage_stride = 0;
    bool stage_valid = false, stg_pending = false;
    hipStream_t stg_stream = nullptr;
    hipEvent_t ev_stg = nullptr;
    // a token that returned on its published words without synchronising: its
    // launches may still be retiring (their staging writes not yet written back),
    // so the step's first staged copy orders stg_stream behind them (ev_dec)
    hipStream_t dec_open = nullptr;
    hipEvent_t ev_dec = nullptr;
    uint64_t n_staged = 0;
    // CPU-assisted serving of absent experts (off while sc_den == 0): the
    // decode kernels post each layer's ids and Q8_K(x) to sc_post; the host
    // team computes the absent experts assigned to it into sc_rows and
    // answers in sc_resp; the join kernel combines.  Host addresses here,
    // device views in the *_d pointers.
    int sc_num = 0, sc_den = 0;
    mpc::Team *team = nullptr;
    mp::SidecarPost *sc_post = nullptr, *sc_post_d = nullptr;     // [L]
    mp::SidecarResp *sc_resp = nullptr, *sc_resp_d = nullptr;     // [L]
    float *sc_rows = nullptr, *sc_rows_d = nullptr;               // [L][K][H]
    uint32_t *d_seq = nullptr, *h_seq = nullptr;
    uint32_t sc_seq = 0;
    // fused layer launches (router, selection, gate/up, down and combine in
    // one launch): tagged exchange words, fx_words per layer; a bounded wait
    // that ran out writes the token's sequence number after the routed ids
    // (d_ids[L * K])
    uint64_t *fx = nullptr;
    size_t fx_words = 0;
    double fused_wait_s = 0.5;
    double sc_timeout_s = 2.0;
    std::vector<float> sc_h, sc_y;         // host scratch: h, and the rows before they are published
    std::vector<uint8_t> sc_q8h, sc_q8x;
    std::vector<int32_t> sc_ids;           // [L][K]: the ids each layer was served with this token
    uint64_t n_cpu_served = 0;
    double sc_wait_us = 0.0, sc_cpu_us = 0.0;   // host time waiting for posts / computing experts
    // heat file (LLAMA_MOE_HEAT_FILE), freeze (LLAMA_MOE_CACHE_FREEZE) and
    // placement-map replay (LLAMA_MOE_MAP_REPLAY)
    std::string heat_path;
    bool freeze = false;
    FILE *replay = nullptr;
    std::vector<float> sc_log;                  // per served layer: wait us, cpu us, experts (last 64K)
    // layers decoded one call at a time (moe_decode_layer), since the last
    // step: each call carries its own sequence number; what the token path
    // settles after its sync (the late-wait word, the host's routing against
    // the GPU's, which experts were staged, kernel times) is settled at the
    // layer's observe and at the step
    std::vector<uint8_t> pl_flags;              // [L]: PL_* bits
    std::vector<uint32_t> pl_seq;               // [L]: the call's sequence number
    std::vector<hipStream_t> pl_streams;        // streams the calls ran on
    bool pl_synced = false;                     // those streams were synchronised since the last call
    bool pl_hot = false;                        // the host team spins between layers
    std::unique_ptr<PlServer> pls;              // serves the host's share of those layers
    bool sc_tested = false;                     // the serving channel passed its self-test
    uint64_t clock = 0, n_steps = 0, n_uploads = 0, n_scheduled = 0, n_copied = 0, n_published = 0;
    uint64_t n_admit_ok = 0, n_admit_denied = 0, n_table_flushes = 0, bytes_uploaded = 0;
    uint64_t n_evicted = 0;            // resident experts the step evicted for an upload
    // upload statistics (LLAMA_MOE_UPLOAD_STATS, patches/0006:689-703): each
    // copy's own duration on its stream, from events recorded around it
    bool up_stats = false;
    std::vector<hipEvent_t> tfree;     // timing events, reused
    uint64_t n_up_h2d = 0, n_up_d2d = 0;
    double up_h2d_us = 0.0, up_d2d_us = 0.0;
    double wait_us = 0.0;
    double boundary_us = 0.0;          // batch-1 decode: host time from the token's sync to the return
    FILE *route = nullptr, *map = nullptr;
    // optional kernel timing: 8 events per layer, read back after the token's sync
    bool timing = false;
    std::vector<hipEvent_t> tev;
    moe_kernel_times kt{};
    // decode path: `split` runs resident and absent experts as separate launches
    // on two streams (fork/join per layer), otherwise one launch serves both;
    // `graph` replays the token's launches as one captured HIP graph over fixed
    // device buffers (x_buf, bias_buf, out_buf)
    int split = 0;                     // 0 fused layer launch, 1 fork/join over two streams,
                                       // 2 serial on one stream, 3 router, selection and experts unfused
    int graph = 1;                 // 0 direct launches, 1 a graph where it is faster, 2 always a graph
    hipStream_t cap_stream = nullptr;
    hipEvent_t ev_user = nullptr, ev_done = nullptr;
    float *x_buf = nullptr, *bias_buf = nullptr, *out_buf = nullptr;
    hipGraph_t g[2] = {nullptr, nullptr};
    hipGraphExec_t gx[2] = {nullptr, nullptr};
    int g_mode[2] = {-1, -1};          // (timing, split) the graph was captured with
    // batched decode (moe_decode_batch): buffers for up to b_cap tokens, grown on demand
    int b_cap = 0;
    int32_t *b_ids = nullptr, *b_slots = nullptr, *b_counts = nullptr, *b_offs = nullptr, *b_perm = nullptr;
    int32_t *bh_ids = nullptr;         // pinned host [L][b_cap][K]
    float *b_w = nullptr;
    uint8_t *b_q8x = nullptr;
    void *b_route_ws = nullptr, *b_ws = nullptr;
    // CPU-assisted batched decode: pinned copies of a layer's gate weights and
    // Q8_K(x); mapped [2][...] (by layer parity) host-expert flags per expert
    // and per pair, and the host's weighted rows
    int bs_cap = 0;
    int sb_num = 0, sb_den = 0;            // the host's share in batches (0/0: the batch-1 share)
    float *bs_w = nullptr;
    uint8_t *bs_q8 = nullptr;
    uint8_t *bs_mask = nullptr, *bs_mask_d = nullptr;
    uint8_t *bs_flag = nullptr, *bs_flag_d = nullptr;
    float *bs_rows = nullptr, *bs_rows_d = nullptr;
    hipEvent_t bs_ev = nullptr;
    std::vector<float> bs_h, bs_y;
    std::vector<uint8_t> bs_q8h;
    // router lookahead and just-in-time streaming
    Streamer *st = nullptr;
    std::vector<float> norm;                   // [layer][H] RMS-norm weights of the router inputs
    std::vector<uint8_t> has_norm;             // [layer]
    int32_t *h_slots = nullptr;                // pinned [layer][K]: the slots the GPU read this token
    std::atomic<int> sc_computing{-1};         // layer whose absent experts the host team is computing
    // MOEP predictor and evictor (LLAMA_MOE_PREDICTOR / _EVICTOR, patches/0006:186-212),
    // borrowed from the caller; the predictor is updated in place when online_lr > 0
    moe_predictor *pred = nullptr, *evict = nullptr;
    int predict_top = 0;
    float online_lr = 0.0f;
    std::string pred_save;                     // checkpoint path (LLAMA_MOE_PREDICTOR_SAVE), or empty
    uint64_t online_n = 0, n_spec = 0;
    double online_recall = 0.0;
    bool spec_probation = false;               // LLAMA_MOE_SPEC_PROBATION (patches/0007:149-153)
};

static void pl_server_stop(moe_cache *c);

struct moe_pool {
    int n_layers = 0, capacity = 0, device = 0;
    size_t bytes = 0;
    uint8_t *base = nullptr;
    hipStream_t stream = nullptr;
    std::vector<hipEvent_t> ev;     // [n_layers * capacity]
    std::vector<uint8_t> armed;
};

namespace {

// ---------------------------------------------------------------------------
// state machine pieces
void set_table_entry(moe_cache *c, Layer &ls, int expert, int v) {
    const size_t o = (size_t)ls.il * c->E + expert;
    c->h_tbl[o] = v;
    if (c->h_prior) c->h_prior[o] = v == ls.S ? 0.0f : c->cfg.cache_prior;
    ls.tbl_dirty = true;
}

// free slots a layer keeps at the boundary: the demand path's inserts and the
// streaming reserve (patches/0010:1135-1142)
int pool_target_of(const moe_cache *c) {
    if (c->freeze) return 0;
    return c->cfg.max_inserts + (c->pred ? c->predict_top : 0) + (c->st ? c->st->reserve : 0);
}

// expert `id` of layer `li` is being streamed in this token
bool streamed(const moe_cache *c, int li, int id) {
    return c->st && c->st->mark[(size_t)li * c->E + id] != 0;
}

uint64_t mono_ns() {
    return (uint64_t)std::chrono::duration_cast<std::chrono::nanoseconds>(
               std::chrono::steady_clock::now().time_since_epoch())
        .count();
}

int32_t lru_resident(const Layer &ls) {
    int32_t victim = -1;
    uint64_t best = U64MAX;
    for (int s = 0; s < ls.S; ++s) {
        if (ls.slot_in_flight[s] || ls.slot_expert[s] < 0) continue;
        if (ls.slot_last_use[s] < best) {
            best = ls.slot_last_use[s];
            victim = ls.slot_expert[s];
        }
    }
    return victim;
}

bool admit_ok(moe_cache *c, const Layer &ls, int id, int victim) {
    if (c->cfg.admit_mode == MOE_ADMIT_OFF || victim < 0) return true;
    bool ok = true;
    if (c->cfg.admit_mode == MOE_ADMIT_HEAT) {
        ok = ls.heat[id] > ls.heat[victim] * 1.25f + c->cfg.admit_floor;
    } else if (c->cfg.admit_mode == MOE_ADMIT_WINDOW) {
        ok = ls.miss_prev[id] != U64MAX && ls.miss_last[id] - ls.miss_prev[id] < (uint64_t)c->cfg.admit_window;
    }
    if (ok) c->n_admit_ok++;
    else c->n_admit_denied++;
    return ok;
}

hipEvent_t take_event(moe_cache *c) {
    if (!c->free_events.empty()) {
        hipEvent_t e = c->free_events.back();
        c->free_events.pop_back();
        return e;
    }
    hipEvent_t e = nullptr;
    if (hipEventCreateWithFlags(&e, hipEventDisableTiming) != hipSuccess) return nullptr;
    return e;
}

// hand one expert copy to the upload stream
int start_upload(moe_cache *c, int li, int expert, int slot, bool spec = false) {
    Layer &ls = c->L[li];
    Job j{li, expert, slot, nullptr, spec};
    if (c->host_only) {
        c->jobs.push_back(j);
        c->bytes_uploaded += ls.expert_bytes;
        return MOE_OK;
    }
    if (!ls.store_host) return fail(MOE_ERR_STATE, "layer %d has no host store registered", li);
    const uint8_t *staged = nullptr;
    if (c->stage_valid)
        for (int k = 0; k < c->K; ++k)
            if (ls.staged[k] == expert) staged = c->stage + ((size_t)li * c->K + k) * c->stage_stride;
    uint8_t *dst = ls.pool + (size_t)slot * ls.slot_bytes;
    hipStream_t s = staged ? c->stg_stream : c->up_stream;
    j.staged = staged != nullptr;
    if (c->up_stats) {
        for (hipEvent_t *e : {&j.t0, &j.t1}) {
            if (!c->tfree.empty()) {
                *e = c->tfree.back();
                c->tfree.pop_back();
            } else if (hipEventCreate(e) != hipSuccess) {
                return fail(MOE_ERR_HIP, "event creation failed");
            }
        }
        HIPCHK(hipEventRecord(j.t0, s));
    }
    if (staged) {
        if (c->dec_open) {
            HIPCHK(hipEventRecord(c->ev_dec, c->dec_open));
            HIPCHK(hipStreamWaitEvent(c->stg_stream, c->ev_dec, 0));
            c->dec_open = nullptr;
        }
        HIPCHK(hipMemcpyAsync(dst, staged, ls.expert_bytes, hipMemcpyDeviceToDevice, s));
        c->stg_pending = true;
        c->n_staged++;
    } else {
        HIPCHK(hipMemcpyAsync(dst, ls.store_host + (size_t)expert * ls.expert_bytes, ls.expert_bytes,
                              hipMemcpyHostToDevice, s));
    }
    if (j.t1) HIPCHK(hipEventRecord(j.t1, s));
    if (c->cfg.publish == MOE_PUBLISH_LIVE) {
        j.ev = take_event(c);
        if (!j.ev) return fail(MOE_ERR_HIP, "event creation failed");
        HIPCHK(hipEventRecord(j.ev, s));
    }
    c->jobs.push_back(j);
    c->bytes_uploaded += ls.expert_bytes;
    return MOE_OK;
}

// spec: the ids are a prediction (patches/0007:232-242)
int issue_uploads(moe_cache *c, int li, const int32_t *ids, int n, int budget, int min_keep, bool spec = false) {
    Layer &ls = c->L[li];
    int issued = 0;
    if (c->freeze) return 0;
    for (int i = 0; i < n && issued < budget; ++i) {
        const int id = ids[i];
        if (id < 0 || id >= ls.E) continue;
        if (ls.expert_slot[id] >= 0) continue;
        if (streamed(c, li, id)) continue;                    // being streamed in this token
        if ((int)ls.free_slots.size() <= min_keep) break;
        bool dup = false;
        for (const Job &j : c->jobs)
            if (j.li == li && j.expert == id) { dup = true; break; }
        if (dup) continue;
        const int slot = ls.free_slots.back();
        ls.free_slots.pop_back();
        ls.slot_in_flight[slot] = 1;
        int r = start_upload(c, li, id, slot, spec);
        if (r != MOE_OK) return r;
        c->n_uploads++;
        c->n_scheduled++;
        c->n_spec += spec;
        issued++;
    }
    return issued;
}

int flush_tables(moe_cache *c);

// copy expert e of layer ls from the pinned store into a slot (replay and
// warm start: synchronous, before any kernel reads the slot)
static int place_bytes(moe_cache *c, const Layer &ls, int e, int slot) {
    if (c->host_only) return MOE_OK;
    if (!ls.store_host) return fail(MOE_ERR_STATE, "layer %d: host store missing for a placement", ls.il);
    HIPCHK(hipMemcpyAsync(ls.pool + (size_t)slot * ls.slot_bytes, ls.store_host + (size_t)e * ls.expert_bytes,
                          ls.expert_bytes, hipMemcpyHostToDevice, c->up_stream));
    return MOE_OK;
}

// replay: this step's recorded frame becomes the placement, every table entry
// rewritten (patches/0008:436-474)
static int replay_frame(moe_cache *c) {
    unsigned long long step = 0;
    if (fscanf(c->replay, " step %llu", &step) != 1 || step != c->n_steps)
        return fail(MOE_ERR_STATE, "map replay: no frame for step %llu", (unsigned long long)c->n_steps);
    for (Layer &ls : c->L) {
        int il = -1;
        if (fscanf(c->replay, " map %d", &il) != 1 || il != ls.il)
            return fail(MOE_ERR_STATE, "map replay: step %llu has no frame for layer %d", step, ls.il);
        std::vector<int32_t> want(ls.S);
        std::vector<uint8_t> seen(ls.E, 0);
        for (auto &v : want) {
            if (fscanf(c->replay, "%d", &v) != 1 || v < -1 || v >= ls.E || (v >= 0 && seen[v]))
                return fail(MOE_ERR_STATE, "map replay: bad frame for layer %d at step %llu", ls.il, step);
            if (v >= 0) seen[v] = 1;
        }
        for (int s = 0; s < ls.S; ++s)
            if (want[s] >= 0 && ls.slot_expert[s] != want[s]) {
                const int r = place_bytes(c, ls, want[s], s);
                if (r != MOE_OK) return r;
            }
        std::fill(ls.expert_slot.begin(), ls.expert_slot.end(), -1);
        for (int e = 0; e < ls.E; ++e) set_table_entry(c, ls, e, ls.S);
        for (int s = 0; s < ls.S; ++s) {
            ls.slot_expert[s] = want[s];
            ls.slot_in_flight[s] = 0;
            if (want[s] >= 0) {
                ls.expert_slot[want[s]] = s;
                set_table_entry(c, ls, want[s], s);
            }
        }
    }
    if (!c->host_only) HIPCHK(hipStreamSynchronize(c->up_stream));
    return flush_tables(c);
}

void write_frame(moe_cache *c, uint64_t step, const std::vector<int32_t> &frame) {
    fprintf(c->map, "step %llu\n", (unsigned long long)step);
    size_t o = 0;
    for (const Layer &ls : c->L) {
        fprintf(c->map, "map %d", ls.il);
        for (int s = 0; s < ls.S; ++s) fprintf(c->map, " %d", frame[o + (size_t)s]);
        o += (size_t)ls.S;
        fputc('\n', c->map);
    }
    fflush(c->map);
}

int map_frame(moe_cache *c) {
    if (c->replay) {
        const int r = replay_frame(c);
        if (r != MOE_OK) return r;
    }
    if (!c->map) return MOE_OK;
    std::vector<int32_t> frame;
    for (const Layer &ls : c->L) {
        const size_t o = frame.size();
        frame.resize(o + (size_t)ls.S, -1);
        for (int e = 0; e < ls.E; ++e)
            if (ls.expert_slot[e] >= 0) frame[o + (size_t)ls.expert_slot[e]] = e;
    }
    Streamer *st = c->st;
    if (!st) {
        write_frame(c, c->n_steps, frame);
        return MOE_OK;
    }
    // streaming (patches/0010:1096-1129): the token after a boundary also used
    // the experts that streamed in before their layer read its table, so the
    // boundary's frame is written one step late with those experts in the
    // slots they used; a replay then gives every token what its GPU saw
    if (st->rec_have) {
        for (const auto &u : st->rec_used) {
            size_t o = 0;
            for (int l = 0; l < u[0]; ++l) o += (size_t)c->L[l].S;
            st->rec_frame[o + (size_t)u[1]] = u[2];
        }
        write_frame(c, st->rec_step, st->rec_frame);
    }
    st->rec_used.clear();
    st->rec_frame = std::move(frame);
    st->rec_step = c->n_steps;
    st->rec_have = true;
    return MOE_OK;
}

// "moe-heat 1 <layers> <experts>", then "<il> <expert> <count>" for every
// non-zero count; written to <path>.tmp and renamed (patches/0007:468-485)
static bool save_heat(const moe_cache *c) {
    const std::string tmp = c->heat_path + ".tmp";
    FILE *f = fopen(tmp.c_str(), "w");
    if (!f) return false;
    fprintf(f, "moe-heat 1 %zu %d\n", c->L.size(), c->E);
    for (const Layer &ls : c->L)
        for (int e = 0; e < ls.E; ++e)
            if (ls.use_count[e]) fprintf(f, "%d %d %u\n", ls.il, e, ls.use_count[e]);
    const bool ok = fclose(f) == 0;
    return ok && rename(tmp.c_str(), c->heat_path.c_str()) == 0;
}

int flush_tables(moe_cache *c) {
    bool any = false;
    for (Layer &ls : c->L) any |= ls.tbl_dirty;
    if (!any) return MOE_OK;
    if (c->host_only) {
        for (Layer &ls : c->L) ls.tbl_dirty = false;
        if (c->cfg.batch_tables) c->n_table_flushes++;
        return MOE_OK;
    }
    const size_t n = (size_t)c->cfg.n_layers * c->E;
    HIPCHK(hipMemcpyAsync(c->d_tbl, c->h_tbl, n * sizeof(int32_t), hipMemcpyHostToDevice, c->tbl_stream));
    if (c->d_prior)
        HIPCHK(hipMemcpyAsync(c->d_prior, c->h_prior, n * sizeof(float), hipMemcpyHostToDevice, c->tbl_stream));
    HIPCHK(hipStreamSynchronize(c->tbl_stream));
    for (Layer &ls : c->L) ls.tbl_dirty = false;
    if (c->cfg.batch_tables) c->n_table_flushes++;
    return MOE_OK;
}

void publish(moe_cache *c, const Job &j) {
    Layer &ls = c->L[j.li];
    ls.slot_expert[j.slot] = j.expert;
    ls.expert_slot[j.expert] = j.slot;
    if (j.spec && c->spec_probation) {
        // a guess is not evidence of reuse: oldest recency, and no eviction
        // through this step's top-up and the next token (n_steps goes up after
        // publication; patches/0007:655-668)
        ls.slot_last_use[j.slot] = 1;
        ls.slot_protect[j.slot] = c->n_steps + 1;
    } else {
        ls.slot_last_use[j.slot] = ++c->clock;
    }
    ls.slot_in_flight[j.slot] = 0;
    set_table_entry(c, ls, j.expert, j.slot);
    c->n_published++;
}

// ---- just-in-time streaming: the mover's bookkeeping ---------------------------
// layer `li` has read its table this token (patches/0010:1164-1181): its
// unfinished jobs are dropped, and the time since the records of the layers
// one and two before it arrived is the lead their predictions had
void stream_posted(moe_cache *c, int li, uint64_t now) {
    Streamer *st = c->st;
    st->planner.posted(li);
    for (int d = 1; d <= 2 && li - d >= 0; ++d) {
        const uint64_t a = st->arrive_ns[(size_t)(li - d)];
        if (a && now > a) {
            st->lead_sum[d] += (double)(now - a);
            st->lead_n[d]++;
        }
    }
}

// one lookahead record (patches/0010:1466-1530): candidates become planner
// jobs, each with a free slot of its target layer; t_ns is the GPU's time at
// the post (the time per layer is estimated from consecutive layers)
int stream_take(moe_cache *c, int layer, const int32_t *targets, const int32_t *n, const int32_t *ids,
                uint64_t now, uint64_t t_ns, uint64_t bytes_given) {
    Streamer *st = c->st;
    const int NL = (int)c->L.size();
    if (layer >= 0 && layer < NL) st->arrive_ns[(size_t)layer] = now;
    if (st->last_layer != UINT32_MAX && (uint32_t)layer == st->last_layer + 1 && t_ns > st->last_t_ns) {
        const double dt = (double)(t_ns - st->last_t_ns);
        if (dt > 10000.0 && dt < 1000000.0) st->tau_ns = 0.9 * st->tau_ns + 0.1 * dt;
    }
    st->last_layer = (uint32_t)layer;
    st->last_t_ns = t_ns;
    st->n[SN_RECORDS]++;
    int taken = 0;
    for (int t = 0; t < 2; ++t) {
        const int T = targets[t];
        if (T < 0 || T >= NL) continue;
        Layer &ls = c->L[(size_t)T];
        const int d = T - layer;
        const uint64_t lead = (uint64_t)(d * st->tau_ns);
        const uint64_t deadline = now + (lead > st->margin_ns ? lead - st->margin_ns : 0);
        const uint64_t bytes = bytes_given ? bytes_given : ls.expert_bytes;
        for (int j = 0; j < n[t] && j < mp::AHEAD_K; ++j) {
            const int e = ids[t * mp::AHEAD_K + j];
            if (e < 0 || e >= ls.E || ls.expert_slot[e] >= 0) continue;
            int32_t &mk = st->mark[(size_t)T * c->E + e];
            if (mk) {
                st->planner.offer(T, e, bytes, deadline);       // a job already: may tighten its deadline
                continue;
            }
            if (st->n_this_token[(size_t)T] >= st->per_layer) continue;
            if ((int)ls.free_slots.size() <= c->cfg.max_inserts) {
                st->n[SN_NOT_SENT]++;                           // the demand path keeps its share
                continue;
            }
            bool upl = false;
            for (const Job &jb : c->jobs)
                if (jb.li == T && jb.expert == e) { upl = true; break; }
            if (upl) continue;                                  // an upload of it is in flight
            const int id = st->planner.offer(T, e, bytes, deadline);
            if (id < 0) continue;                               // the layer has read its table already
            StreamJob sj{T, ls.free_slots.back(), d, 0, false, false, false};
            ls.free_slots.pop_back();
            ls.slot_in_flight[(size_t)sj.slot] = 1;
            st->jobs.push_back(sj);
            mk = id + 1;
            st->n_this_token[(size_t)T]++;
            st->n[SN_OFFERED]++;
            taken++;
        }
    }
    return taken;
}

bool stream_next(moe_cache *c, uint64_t free_at, int hold_after, mps::Chunk &ch) {
    Streamer *st = c->st;
    if (!st->planner.next(free_at, st->bytes_per_ns, hold_after, ch)) return false;
    st->n[SN_BYTES] += ch.len;
    return true;
}

void stream_land(moe_cache *c, int job) {
    Streamer *st = c->st;
    if (job < 0 || job >= (int)st->jobs.size() || st->jobs[(size_t)job].landed) return;
    st->jobs[(size_t)job].landed = true;
    st->n[SN_LANDED]++;
}

// the GPU's slots say whether each streamed expert made it (patches/0010:1183-1210)
void stream_account(moe_cache *c, int li, const int32_t *ids, const int32_t *gslots, int n_ids) {
    Streamer *st = c->st;
    const Layer &l0 = c->L[(size_t)li];
    for (int i = 0; i < n_ids; ++i) {
        const int id = ids[i];
        if (id < 0 || id >= l0.E) continue;
        const bool miss = gslots[i] >= l0.S;
        const int32_t m = st->mark[(size_t)li * c->E + id];
        if (!m) {
            st->n[SN_GPU_MISS] += miss;
            continue;
        }
        StreamJob &j = st->jobs[(size_t)m - 1];
        Layer &ls = c->L[(size_t)j.li];
        if (!miss && !j.in_time) {
            j.in_time = true;
            st->n[SN_IN_TIME]++;
            ls.n_hit++;
        } else if (miss && !j.in_time && !j.late) {
            j.late = true;
            st->n[SN_LATE]++;
            st->n[SN_GPU_MISS]++;
            ls.n_miss++;
        }
    }
}

// boundary, mover idle (patches/0010:1722-1760): landed experts join the
// cache -- routed ones as recently used, the others as the first to go --
// and the slots of the rest go back to the pool.  Every layer a table word
// was written for is flushed from the mirrors, which clears STREAM_BIT.
void stream_adopt(moe_cache *c) {
    Streamer *st = c->st;
    st->rec_used.clear();
    for (size_t k = 0; k < st->jobs.size(); ++k) {
        const StreamJob &sj = st->jobs[k];
        const int e = st->planner.get((int)k).expert;
        Layer &ls = c->L[(size_t)sj.li];
        ls.slot_in_flight[(size_t)sj.slot] = 0;
        if (sj.ticket > 0) ls.tbl_dirty = true;
        if (sj.in_time) st->rec_used.push_back({sj.li, sj.slot, e});
        if (sj.landed && ls.expert_slot[e] >= 0) {
            ls.free_slots.push_back(sj.slot);             // an upload of it was published meanwhile
            st->n[SN_UNUSED] += !sj.in_time && !sj.late;
            ls.tbl_dirty = true;
        } else if (sj.landed) {
            ls.slot_expert[(size_t)sj.slot] = e;
            ls.expert_slot[e] = sj.slot;
            ls.slot_last_use[(size_t)sj.slot] = sj.in_time || sj.late ? ++c->clock : 1;
            set_table_entry(c, ls, e, sj.slot);
            c->n_published++;
            if (!sj.in_time && !sj.late) st->n[SN_UNUSED]++;
        } else {
            ls.free_slots.push_back(sj.slot);
        }
        st->mark[(size_t)sj.li * c->E + e] = 0;
    }
    st->n[SN_DROP_LATE] = st->planner.n_drop_late;
    st->n[SN_DROP_POSTED] = st->planner.n_drop_posted;
    st->jobs.clear();
    st->planner.reset();
    std::fill(st->n_this_token.begin(), st->n_this_token.end(), 0);
    std::fill(st->arrive_ns.begin(), st->arrive_ns.end(), 0);
    st->last_layer = UINT32_MAX;
}

// ---- the mover thread (live): copy queue, planner, records -------------------
// The copy queue is one stream with a ring of events: a push is some copies
// then an event, and its ticket is done when that event has fired.  A push is
// ordered after every earlier one, which is what makes "the expert's last
// chunk, then its table word" safe as one push.
int64_t mover_done(Streamer *st) {
    while (st->ev_count > 0) {
        const hipError_t q = hipEventQuery(st->ev[(size_t)st->ev_head]);
        if (q == hipErrorNotReady) break;
        if (q != hipSuccess) return -1;
        st->done_ticket = st->ev_ticket[(size_t)st->ev_head];
        st->ev_head = (st->ev_head + 1) % (int)st->ev.size();
        st->ev_count--;
    }
    return st->done_ticket;
}

// ticket of the push, 0 when the ring is full, -1 on a HIP error
int64_t mover_push(Streamer *st, void *dst, const void *src, size_t len, void *wdst, const void *wsrc) {
    if (st->ev_count == (int)st->ev.size()) {
        if (mover_done(st) < 0) return -1;
        if (st->ev_count == (int)st->ev.size()) return 0;
    }
    if (hipMemcpyAsync(dst, src, len, hipMemcpyHostToDevice, st->stream) != hipSuccess) return -1;
    if (wdst && hipMemcpyAsync(wdst, wsrc, sizeof(int32_t), hipMemcpyHostToDevice, st->stream) != hipSuccess)
        return -1;
    const int i = (st->ev_head + st->ev_count) % (int)st->ev.size();
    if (hipEventRecord(st->ev[(size_t)i], st->stream) != hipSuccess) return -1;
    st->ev_ticket[(size_t)i] = st->next_ticket++;
    st->ev_count++;
    return st->ev_ticket[(size_t)i];
}

// copies whose event fired: the expert and its table word are on the device
void stream_reap(moe_cache *c, int64_t done) {
    Streamer *st = c->st;
    if (done < 0) {
        if (!st->failed.exchange(true)) fprintf(stderr, "moe-cache: stream copy queue error; streaming stops\n");
        return;
    }
    while (!st->outstanding.empty() && st->outstanding.front().first <= done) st->outstanding.pop_front();
    for (size_t k = 0; k < st->jobs.size(); ++k) {
        const StreamJob &j = st->jobs[k];
        if (j.ticket > 0 && j.ticket <= done && !j.landed) stream_land(c, (int)k);
    }
}

// hand the copy engine the next chunks, up to max_outstanding bytes queued
bool stream_issue(moe_cache *c) {
    Streamer *st = c->st;
    size_t queued = 0;
    for (const auto &o : st->outstanding) queued += o.second;
    bool any = false;
    while (queued < st->max_outstanding && st->outstanding.size() < 32) {
        // while the host computes a layer's absent experts, copies for later layers wait
        const int comp = c->sc_computing.load(std::memory_order_relaxed);
        const uint64_t free_at = mono_ns() + (uint64_t)((double)queued / st->bytes_per_ns);
        mps::Chunk ch;
        if (!stream_next(c, free_at, comp >= 0 ? comp + 1 : -1, ch)) break;
        const int e = st->planner.get(ch.job).expert;
        StreamJob &sj = st->jobs[(size_t)ch.job];
        const Layer &ls = c->L[(size_t)sj.li];
        uint8_t *dst = ls.pool + (size_t)sj.slot * ls.slot_bytes + ch.offset;
        const uint8_t *src = ls.store_host + (size_t)e * ls.expert_bytes + ch.offset;
        int32_t *wdst = ch.last ? c->d_tbl + (size_t)ls.il * c->E + e : nullptr;
        const int32_t *wsrc = ch.last ? st->words + sj.slot : nullptr;
        const int64_t ticket = mover_push(st, dst, src, ch.len, wdst, wsrc);
        if (ticket <= 0) {
            if (!st->failed.exchange(true))
                fprintf(stderr, "moe-cache: stream copy push failed (%lld); streaming stops\n", (long long)ticket);
            return any;
        }
        st->outstanding.push_back({ticket, ch.len});
        queued += ch.len;
        if (ch.last) sj.ticket = ticket;
        any = true;
    }
    return any;
}

// One generation per token: take each layer's lookahead record as it
// arrives (the layer has then read its table), keep the copy engine fed, and
// when the token's GPU work is over wait for the queued copies and hand the
// bookkeeping back to the cache's thread.
void mover_loop(moe_cache *c) {
    Streamer *st = c->st;
    if (hipSetDevice(c->cfg.device) != hipSuccess) st->failed = true;
    uint32_t served = 0;
    const int NL = (int)c->L.size();
    for (;;) {
        uint32_t gen;
        {
            std::unique_lock<std::mutex> lk(st->m);
            st->cv.wait(lk, [&] { return st->quit || st->gen != served; });
            if (st->quit) return;
            gen = st->gen;
        }
        const uint32_t seq = st->seq;
        int next = 0;
        int64_t last_done = st->done_ticket;
        while (!st->stop.load(std::memory_order_acquire)) {
            bool progress = false;
            while (!st->failed && next < NL &&
                   __atomic_load_n(&st->post[next].seq, __ATOMIC_ACQUIRE) == seq) {
                const mp::AheadPost rec = st->post[next];
                const uint64_t now = mono_ns();
                stream_posted(c, next, now);
                const uint64_t t = ((uint64_t)rec.t_hi << 32 | rec.t_lo) * 10;     // 100 MHz clock -> ns
                stream_take(c, next, rec.target, rec.n, &rec.ids[0][0], now, t, 0);
                ++next;
                progress = true;
            }
            if (!st->failed) {
                const int64_t done = mover_done(st);
                if (done != last_done) {
                    stream_reap(c, done);
                    last_done = done;
                    progress = true;
                }
                progress |= stream_issue(c);
            }
            if (!progress) _mm_pause();
        }
        // the token is over: what landed stays, the rest goes back at the boundary
        if (hipStreamSynchronize(st->stream) != hipSuccess) st->failed = true;
        stream_reap(c, st->failed ? -1 : mover_done(st));
        st->outstanding.clear();
        served = gen;
        {
            std::lock_guard<std::mutex> lk(st->m);
            st->gen_done = gen;
        }
        st->cv_done.notify_all();
    }
}

void stream_stop_thread(Streamer *st) {
    if (!st->thr.joinable()) return;
    st->stop.store(true, std::memory_order_release);      // ends a token the mover may still serve
    {
        std::lock_guard<std::mutex> lk(st->m);
        st->quit = true;
    }
    st->cv.notify_all();
    st->thr.join();
}

void stream_free(moe_cache *c) {
    Streamer *st = c->st;
    if (!st) return;
    stream_stop_thread(st);
    if (c->map && st->rec_have) write_frame(c, st->rec_step, st->rec_frame);   // the last boundary
    if (st->live) {
        if (st->stream) hipStreamSynchronize(st->stream);
        for (hipEvent_t e : st->ev)
            if (e) hipEventDestroy(e);
        if (st->stream) hipStreamDestroy(st->stream);
        hipFree(st->ratio);
        hipFree(st->alog);
        hipFree(st->fresh);
        if (st->post) hipHostFree(st->post);
        if (st->words) hipHostFree(st->words);
    }
    delete st;
    c->st = nullptr;
}

// the evictor's scores of layer li's experts, once per step (patches/0006:404-427);
// false when it has no model for the layer
bool evict_scores(const moe_cache *c, size_t li, std::vector<float> &out) {
    const Layer &ls = c->L[li];
    if (!c->evict || !c->evict->p.has_layer(ls.il)) return false;
    mpp::Lists in;
    auto set = [&in](int g, const std::vector<int32_t> &v) {
        in.ids[g] = v.data();
        in.n[g] = v.size();
    };
    set(1, ls.cur_ids);
    set(3, ls.prev_ids);
    if (li + 1 < c->L.size()) set(0, c->L[li + 1].prev_ids);
    if (li > 0) set(2, c->L[li - 1].cur_ids);
    out.resize((size_t)c->E);
    c->evict->p.score(ls.il, in, out.data());
    return true;
}

// victim among the slots that may go: with the evictor the lowest score
// (recency breaks ties: many cold experts share a near-zero score), else the
// least recently used (patches/0006:802-824)
struct VictimPick {
    bool use_model;
    const std::vector<float> &esc;
    int slot = -1;
    uint64_t best = U64MAX;
    float best_score = 3.4e38f;
    void offer(const Layer &ls, int s) {
        if (use_model) {
            const float sc = esc[(size_t)ls.slot_expert[s]];
            if (sc < best_score || (sc == best_score && ls.slot_last_use[s] < best)) {
                best_score = sc;
                best = ls.slot_last_use[s];
                slot = s;
            }
        } else if (ls.slot_last_use[s] < best) {
            best = ls.slot_last_use[s];
            slot = s;
        }
    }
};

int cache_step(moe_cache *c) {
    // 1) publish finished uploads (no kernel of the cache is running)
    if (!c->jobs.empty()) {
        std::vector<Job> done;
        if (c->host_only) {
            done.assign(c->jobs.begin(), c->jobs.end());
            c->jobs.clear();
            if (c->cfg.publish == MOE_PUBLISH_SORTED)
                std::stable_sort(done.begin(), done.end(), [](const Job &a, const Job &b) {
                    return a.li != b.li ? a.li < b.li : a.slot < b.slot;
                });
        } else if (c->cfg.publish == MOE_PUBLISH_LIVE) {
            while (!c->jobs.empty()) {
                const hipError_t q = hipEventQuery(c->jobs.front().ev);
                if (q == hipErrorNotReady) break;
                if (q != hipSuccess) return fail(MOE_ERR_HIP, "hipEventQuery: %s", hipGetErrorString(q));
                done.push_back(c->jobs.front());
                c->free_events.push_back(c->jobs.front().ev);
                c->jobs.pop_front();
            }
        } else {
            const auto t0 = std::chrono::steady_clock::now();
            HIPCHK(hipEventRecord(c->up_mark, c->up_stream));
            HIPCHK(hipEventSynchronize(c->up_mark));
            HIPCHK(hipStreamSynchronize(c->stg_stream));
            c->wait_us += std::chrono::duration<double, std::micro>(std::chrono::steady_clock::now() - t0).count();
            done.assign(c->jobs.begin(), c->jobs.end());
            c->jobs.clear();
            if (c->cfg.publish == MOE_PUBLISH_SORTED)
                std::stable_sort(done.begin(), done.end(), [](const Job &a, const Job &b) {
                    return a.li != b.li ? a.li < b.li : a.slot < b.slot;
                });
        }
        c->n_copied += done.size();
        for (Job &j : done) {
            if (j.t0) {             // the copy is done: its events have completed
                float ms = 0.0f;
                HIPCHK(hipEventElapsedTime(&ms, j.t0, j.t1));
                (j.staged ? c->n_up_d2d : c->n_up_h2d)++;
                (j.staged ? c->up_d2d_us : c->up_h2d_us) += 1e3 * ms;
                c->tfree.push_back(j.t0);
                c->tfree.push_back(j.t1);
                j.t0 = j.t1 = nullptr;
            }
            publish(c, j);
        }
    }
    if (c->st) stream_adopt(c);         // after the uploads: an expert both copied is kept once

    c->n_steps++;

    // 2) per layer
    std::vector<float> esc;
    for (size_t li = 0; li < c->L.size(); ++li) {
        Layer &ls = c->L[li];
        if (!c->cfg.early_issue) {
            if (ls.pending.empty()) continue;
            int budget = c->cfg.max_inserts;
            const bool use_model = evict_scores(c, li, esc);
            for (auto it = ls.pending.rbegin(); it != ls.pending.rend() && budget > 0; ++it) {
                const int id = *it;
                if (ls.expert_slot[id] >= 0) {
                    --budget;
                    continue;
                }
                int slot = -1;
                VictimPick vp{use_model, esc};
                for (int s = 0; s < ls.S; ++s) {
                    if (ls.slot_in_flight[s]) continue;
                    if (ls.slot_expert[s] < 0) { slot = s; break; }
                    if (ls.slot_protect[s] >= c->n_steps) continue;
                    vp.offer(ls, s);
                }
                if (slot < 0) slot = vp.slot;
                if (slot < 0) break;
                const int victim = ls.slot_expert[slot];
                if (!admit_ok(c, ls, id, victim)) continue;
                --budget;
                if (victim >= 0) {
                    ls.expert_slot[victim] = -1;
                    ls.slot_expert[slot] = -1;
                    set_table_entry(c, ls, victim, ls.S);
                    c->n_evicted++;
                }
                ls.slot_in_flight[slot] = 1;
                const int r = start_upload(c, (int)li, id, slot);
                if (r != MOE_OK) return r;
                c->n_scheduled++;
            }
            ls.pending.clear();
            continue;
        }
        ls.pending.clear();
        const int pool_target = pool_target_of(c);
        const bool use_model = evict_scores(c, li, esc);
        while ((int)ls.free_slots.size() < pool_target) {
            VictimPick vp{use_model, esc};
            for (int s = 0; s < ls.S; ++s) {
                if (ls.slot_in_flight[s] || ls.slot_expert[s] < 0) continue;
                if (ls.slot_protect[s] >= c->n_steps) continue;
                vp.offer(ls, s);
            }
            const int slot = vp.slot;
            if (slot < 0) break;
            const int victim = ls.slot_expert[slot];
            ls.expert_slot[victim] = -1;
            ls.slot_expert[slot] = -1;
            set_table_entry(c, ls, victim, ls.S);
            ls.free_slots.push_back(slot);
            c->n_evicted++;
        }
    }

    // after every eviction decision: this token's ids become the previous ones (patches/0006:915-922)
    if (c->evict)
        for (Layer &ls : c->L) ls.prev_ids = ls.cur_ids;

    // 3) heat decays on a clock
    if (c->cfg.admit_mode == MOE_ADMIT_HEAT && c->cfg.admit_half > 0 && c->n_steps % (uint64_t)c->cfg.admit_half == 0)
        for (Layer &ls : c->L)
            for (float &h : ls.heat) h *= 0.5f;

    // 4) every table edit of this step reaches the device in one transfer
    const int r = flush_tables(c);
    if (r != MOE_OK) return r;

    // 5) heat file every 512 steps (not while frozen), then the map frame
    if (!c->freeze && !c->heat_path.empty() && c->n_steps % 512 == 0 && !save_heat(c))
        fprintf(stderr, "moe-cache: heat file write FAILED: %s\n", c->heat_path.c_str());
    const int r2 = map_frame(c);
    if (c->route) fflush(c->route);
    return r2;
}

// gslots (batch 1 with streaming): the slots the GPU read, n_slots = absent
int cache_observe(moe_cache *c, int li, const int32_t *ids, int n_ids, int n_tok, const int32_t *gslots = nullptr) {
    Layer &ls = c->L[li];
    if (c->route) {
        fprintf(c->route, "route %llu %d %d %d", (unsigned long long)c->n_steps, ls.il, n_ids, n_tok);
        for (int i = 0; i < n_ids * n_tok; ++i) {
            int slot = (ids[i] >= 0 && ids[i] < ls.E) ? ls.expert_slot[ids[i]] : -1;
            if (gslots) slot = gslots[i] >= ls.S ? -1 : gslots[i];    // what the GPU used (0010:1147-1154)
            fprintf(c->route, " %d:%d", ids[i], slot);
        }
        fputc('\n', c->route);
    }
    std::vector<int32_t> observed;
    observed.reserve((size_t)n_ids * n_tok);
    for (int t = 0; t < n_tok; ++t) {
        for (int i = 0; i < n_ids; ++i) {
            const int id = ids[t * n_ids + i];
            if (id < 0 || id >= ls.E) continue;
            observed.push_back(id);
            if (!ls.heat.empty()) ls.heat[id] += 1.0f;
            if (!ls.use_count.empty()) ls.use_count[id]++;
            const int slot = ls.expert_slot[id];
            if (slot < 0 && streamed(c, li, id)) continue;      // the GPU's table decides (accounted below)
            if (slot >= 0) {
                ls.n_hit++;
                ls.slot_last_use[slot] = ++c->clock;
            } else {
                ls.n_miss++;
                if (!ls.miss_last.empty() && ls.miss_last[id] != c->n_steps) {
                    ls.miss_prev[id] = ls.miss_last[id];
                    ls.miss_last[id] = c->n_steps;
                }
                if (std::find(ls.pending.begin(), ls.pending.end(), id) == ls.pending.end())
                    ls.pending.push_back(id);
            }
        }
    }
    // the prediction made for this layer resolves against what it routed to
    // (patches/0006:323-363): one SGD step, a checkpoint every 200000
    if (c->pred && c->online_lr > 0.0f && ls.pend_valid && c->pred->p.has_layer(ls.il)) {
        mpp::Lists in;
        in.ids[0] = ls.pend_prev.data();
        in.n[0] = ls.pend_prev.size();
        in.ids[1] = ls.pend_cur.data();
        in.n[1] = ls.pend_cur.size();
        c->online_recall += c->pred->p.update(ls.il, in, observed.data(), observed.size(), c->online_lr);
        ls.pend_valid = false;
        c->online_n++;
        if (!c->pred_save.empty() && c->online_n % 200000 == 0) {
            std::string err;
            const std::string tmp = c->pred_save + ".tmp";
            if (!c->pred->p.save(tmp, err) || rename(tmp.c_str(), c->pred_save.c_str()) != 0)
                fprintf(stderr, "moe-cache: predictor checkpoint FAILED: %s\n", err.c_str());
        }
    }
    if (c->cfg.early_issue) {
        const int pool_target = pool_target_of(c);
        const int next_victim = c->cfg.admit_mode == MOE_ADMIT_OFF ? -1
                                : ((int)ls.free_slots.size() > pool_target ? -1 : lru_resident(ls));
        int r;
        if (c->cfg.admit_mode == MOE_ADMIT_OFF) {
            r = issue_uploads(c, li, ls.pending.data(), (int)ls.pending.size(), c->cfg.max_inserts, 0);
        } else {
            std::vector<int32_t> adm;
            for (int id : ls.pending)
                if (ls.expert_slot[id] < 0 && admit_ok(c, ls, id, next_victim)) adm.push_back(id);
            r = issue_uploads(c, li, adm.data(), (int)adm.size(), c->cfg.max_inserts, 0);
        }
        if (r < 0) return r;
        // the next layer's experts, predicted from its previous ids and this
        // layer's, copied into its spare slots; the demand path keeps
        // max_inserts of them (patches/0006:367-396, 0007:424-452)
        if (c->pred && c->pred->p.has_layer(ls.il) && (size_t)li + 1 < c->L.size()) {
            Layer &nls = c->L[(size_t)li + 1];
            mpp::Lists in;
            in.ids[0] = nls.cur_ids.data();
            in.n[0] = nls.cur_ids.size();
            in.ids[1] = observed.data();
            in.n[1] = observed.size();
            std::vector<float> sc((size_t)c->E);
            std::vector<int32_t> top((size_t)c->predict_top);
            c->pred->p.score(ls.il, in, sc.data());
            const int n_top = (int)c->pred->p.top(sc.data(), (size_t)c->predict_top, top.data());
            if (c->online_lr > 0.0f) {
                nls.pend_prev = nls.cur_ids;
                nls.pend_cur = observed;
                nls.pend_valid = true;
            }
            int n_issue = n_top;
            if (c->cfg.admit_mode == MOE_ADMIT_HEAT) {
                // a guess may only displace something colder than itself
                const int nv = (int)nls.free_slots.size() > pool_target ? -1 : lru_resident(nls);
                n_issue = 0;
                for (int k = 0; k < n_top; ++k) {
                    const int id = top[(size_t)k];
                    if (id >= 0 && id < nls.E && nls.expert_slot[id] < 0 && admit_ok(c, nls, id, nv))
                        top[(size_t)n_issue++] = id;
                }
            }
            r = issue_uploads(c, li + 1, top.data(), n_issue, c->predict_top, c->cfg.max_inserts, true);
            if (r < 0) return r;
        }
    }
    ls.cur_ids.swap(observed);
    if (gslots && c->st) stream_account(c, li, ids, gslots, n_ids);
    return MOE_OK;
}

int check_shape(int E, int H, int I, int K) {
    if (H != 2048) return fail(MOE_ERR_ARG, "hidden size %d unsupported (the kernels are built for 2048)", H);
    if (E <= 0 || E % 64 != 0 || E > 256) return fail(MOE_ERR_ARG, "n_experts %d must be a multiple of 64 <= 256", E);
    if (K <= 0 || K > 16 || K > E) return fail(MOE_ERR_ARG, "n_expert_used %d must be 1..16", K);
    if (I != 0 && (I % 256 != 0 || I > 768))
        return fail(MOE_ERR_ARG, "intermediate %d must be 256, 512 or 768", I);
    return MOE_OK;
}

size_t route_ws_bytes(int E, int n_tok) { return align_up((size_t)n_tok * E * 4, 256) + align_up((size_t)n_tok * 4, 256); }
// room for K routed experts and a shared one
size_t exp_ws_bytes(int I, int K) {
    const size_t k1 = (size_t)K + 1;
    return align_up(k1 * I * 4, 256) + align_up(k1 * (I / 256) * mp::Q8K_BYTES, 256) + align_up(k1 * 4, 256);
}

// seq: the token's sequence number on the device, or null and seq_val
int run_route(const moe_route_desc *d, hipStream_t st, hipEvent_t *ev = nullptr, mp::SidecarPost *post = nullptr,
              const uint32_t *seq = nullptr, const mp::RouteLaunch *ahead = nullptr, uint32_t seq_val = 0) {
    mp::RouteLaunch l{};
    if (ahead) l = *ahead;          // lookahead and table-freshness fields; the rest is set below
    l.W = d->W; l.x = d->x; l.bias = d->bias; l.prior = d->prior; l.table = d->table; l.dummy = d->dummy;
    l.prior_on_logits = d->prior_on_logits;
    l.E = d->E; l.H = d->H; l.K = d->K; l.n_tok = d->n_tok;
    uint8_t *ws = (uint8_t *)d->workspace;
    l.logits = (float *)ws;
    l.counter = (uint32_t *)(ws + align_up((size_t)d->n_tok * d->E * 4, 256));
    l.ids = d->ids; l.w = d->w; l.slots = d->slots; l.probs = d->probs; l.q8x = d->q8x;
    l.logits_in = d->logits;
    l.post = post;
    l.seq = seq;
    l.seq_val = seq_val;
    HIPCHK(mp::launch_route(l, st, ev));
    return MOE_OK;
}

int run_experts(const moe_experts_desc *d, hipStream_t st) {
    mp::ExpertArgs a{};
    a.ids = d->ids; a.slots = d->slots; a.w = d->w;
    a.slot_pool = d->slot_pool; a.slot_bytes = d->slot_bytes; a.n_slots = d->n_slots;
    a.host_store = d->host_store; a.expert_bytes = d->expert_bytes; a.n_experts = d->n_experts;
    a.q8x = d->q8x; a.out = d->out; a.accumulate = d->accumulate;
    a.H = d->H; a.I = d->I; a.K = d->K; a.down_type = d->down_type;
    a.shared = d->shared; a.n_shared = d->shared ? 1 : 0;
    uint8_t *ws = (uint8_t *)d->workspace;
    a.h = (float *)ws;
    size_t o = align_up((size_t)(d->K + 1) * d->I * 4, 256);
    a.q8h = ws + o;
    o += align_up((size_t)(d->K + 1) * (d->I / 256) * mp::Q8K_BYTES, 256);
    a.counter = (uint32_t *)(ws + o);
    HIPCHK(mp::launch_experts(a, st));
    return MOE_OK;
}

// A kernel read of unmapped memory faults the GPU: refuse anything the runtime
// does not know as device memory or device-mapped pinned memory.
int check_weight_ptrs(const char *who, const void *a, const void *b) {
    for (const void *p : {a, b}) {
        if (!p) continue;
        hipPointerAttribute_t at{};
        if (hipPointerGetAttributes(&at, p) != hipSuccess || (at.type != hipMemoryTypeDevice &&
                                                              at.type != hipMemoryTypeHost &&
                                                              at.type != hipMemoryTypeUnified))
            return fail(MOE_ERR_ARG, "%s: %p is not device memory or mapped pinned memory", who, p);
        if (at.type == hipMemoryTypeHost && at.devicePointer != p)
            return fail(MOE_ERR_ARG, "%s: pass the device address of pinned memory (moe_host_device_ptr)", who);
    }
    return MOE_OK;
}

// workspace of the batched expert path, offsets in bytes
struct GroupedWs {
    size_t xa, xdx, xbs, h, ha, hdx, hbs, ypair, sh_offs, sh_perm, sh_ones, total;
};

GroupedWs grouped_ws(int n_tok, int K, int H, int I) {
    const size_t T = (size_t)n_tok, P = (size_t)n_tok * K;
    GroupedWs w{};
    size_t o = 0;
    w.xa = o;    o += align_up(T * H * 2, 256);
    w.xdx = o;   o += align_up(T * (H / 256) * 4, 256);
    w.xbs = o;   o += align_up(T * (H / 16) * 2, 256);
    w.h = o;     o += align_up(P * 2 * I * 4, 256);   // up and gate rows
    w.ha = o;    o += align_up(P * I * 2, 256);
    w.hdx = o;   o += align_up(P * (I / 256) * 4, 256);
    w.hbs = o;   o += align_up(P * (I / 16) * 2, 256);
    w.ypair = o; o += align_up(P * H * 4, 256);
    w.sh_offs = o; o += 256;                              // shared expert: trivial dispatch
    w.sh_perm = o; o += align_up(T * 4, 256);
    w.sh_ones = o; o += align_up(T * 4, 256);
    w.total = o;
    return w;
}

void free_cache(moe_cache *c) {
    if (!c) return;
    stream_free(c);
    for (hipEvent_t e : c->tev) hipEventDestroy(e);
    if (c->host_only) {
        free(c->h_tbl);
        free(c->h_prior);
        if (c->route) fclose(c->route);
        if (c->replay) fclose(c->replay);
        if (c->map) fclose(c->map);
        delete c;
        return;
    }
    if (c->up_stream) hipStreamSynchronize(c->up_stream);
    if (c->stg_stream) hipStreamSynchronize(c->stg_stream);
    for (Job &j : c->jobs)
        for (hipEvent_t e : {j.ev, j.t0, j.t1})
            if (e) hipEventDestroy(e);
    for (hipEvent_t e : c->free_events) hipEventDestroy(e);
    for (hipEvent_t e : c->tfree) hipEventDestroy(e);
    if (c->up_mark) hipEventDestroy(c->up_mark);
    for (hipEvent_t e : {c->ev_route, c->ev_hbm, c->ev_host, c->ev_user, c->ev_done})
        if (e) hipEventDestroy(e);
    for (int i = 0; i < 2; ++i) {
        if (c->gx[i]) hipGraphExecDestroy(c->gx[i]);
        if (c->g[i]) hipGraphDestroy(c->g[i]);
    }
    if (c->host_stream) hipStreamDestroy(c->host_stream);
    if (c->cap_stream) hipStreamDestroy(c->cap_stream);
    hipFree(c->x_buf);
    hipFree(c->bias_buf);
    hipFree(c->out_buf);
    if (c->up_stream) hipStreamDestroy(c->up_stream);
    if (c->stg_stream) hipStreamDestroy(c->stg_stream);
    pl_server_stop(c);
    if (c->team) mpc::team_destroy(c->team);
    for (void *p : {(void *)c->sc_post, (void *)c->sc_resp, (void *)c->sc_rows, (void *)c->h_seq})
        if (p) hipHostFree(p);
    hipFree(c->d_seq);
    if (c->ev_stg) hipEventDestroy(c->ev_stg);
    if (c->ev_dec) hipEventDestroy(c->ev_dec);
    hipFree(c->stage);
    if (c->tbl_stream) hipStreamDestroy(c->tbl_stream);
    hipFree(c->pool_base);
    for (auto &ls : c->L) hipFree(ls.shared);
    for (void *p : {(void *)c->b_ids, (void *)c->b_slots, (void *)c->b_counts, (void *)c->b_offs, (void *)c->b_perm,
                    (void *)c->b_w, (void *)c->b_q8x, c->b_route_ws, c->b_ws})
        hipFree(p);
    if (c->bh_ids) hipHostFree(c->bh_ids);
    for (void *p : {(void *)c->bs_w, (void *)c->bs_q8, (void *)c->bs_mask, (void *)c->bs_flag, (void *)c->bs_rows})
        if (p) hipHostFree(p);
    if (c->bs_ev) hipEventDestroy(c->bs_ev);
    hipFree(c->d_tbl);
    hipFree(c->d_prior);
    hipFree(c->route_ws);
    hipFree(c->exp_ws);
    hipFree(c->ypart);
    hipFree(c->d_ids);
    hipFree(c->d_pub_ctr);
    hipFree(c->fx);
    hipFree(c->d_w);
    hipFree(c->d_q8x);
    if (c->h_tbl) hipHostFree(c->h_tbl);
    if (c->h_prior) hipHostFree(c->h_prior);
    if (c->h_ids) hipHostFree(c->h_ids);
    if (c->h_pub) hipHostFree(c->h_pub);
    if (c->route) fclose(c->route);
    if (c->map) fclose(c->map);
    if (c->replay) fclose(c->replay);
    delete c;
}

}  // namespace

// ===========================================================================
// C ABI
extern "C" {

const char *moe_last_error(void) { return g_err.c_str(); }
int moe_abi_version(void) { return 1; }

void *moe_host_alloc(size_t bytes) {
    void *p = nullptr;
    if (hipHostMalloc(&p, bytes, hipHostMallocMapped | hipHostMallocPortable) != hipSuccess) {
        fail(MOE_ERR_NOMEM, "hipHostMalloc(%zu) failed", bytes);
        return nullptr;
    }
    return p;
}

int moe_host_free(void *p) {
    if (p) HIPCHK(hipHostFree(p));
    return MOE_OK;
}

void *moe_host_device_ptr(void *host) {
    void *dev = nullptr;
    if (!host || hipHostGetDevicePointer(&dev, host, 0) != hipSuccess) {
        fail(MOE_ERR_ARG, "%p is not device-mapped pinned memory", host);
        return nullptr;
    }
    return dev;
}

void *moe_device_alloc(size_t bytes) {
    void *p = nullptr;
    if (hipMalloc(&p, bytes) != hipSuccess) {
        fail(MOE_ERR_NOMEM, "hipMalloc(%zu) failed", bytes);
        return nullptr;
    }
    return p;
}

int moe_device_free(void *p) {
    if (p) HIPCHK(hipFree(p));
    return MOE_OK;
}

int moe_device_synchronize(void) {
    HIPCHK(hipDeviceSynchronize());
    return MOE_OK;
}

int moe_memcpy(void *dst, const void *src, size_t bytes) {
    if (!dst || !src) return fail(MOE_ERR_ARG, "null pointer");
    HIPCHK(hipMemcpy(dst, src, bytes, hipMemcpyDefault));
    return MOE_OK;
}

bool moe_memcpy_h2d_batch(int device, void **dst, const void **src, const size_t *sizes, int n) {
    if (n <= 0) return true;
    if (!dst || !src || !sizes) {
        fail(MOE_ERR_ARG, "moe_memcpy_h2d_batch: null array");
        return false;
    }
    for (int i = 0; i < n; ++i)         // nothing is copied when any slice is unusable
        if (!dst[i] || !src[i]) {
            fail(MOE_ERR_ARG, "moe_memcpy_h2d_batch: slice %d of %d has a null address", i, n);
            return false;
        }
    if (hipSetDevice(device) != hipSuccess) return false;
    for (int i = 0; i < n; ++i) {
        if (hipMemcpyAsync(dst[i], src[i], sizes[i], hipMemcpyHostToDevice, hipStreamPerThread) != hipSuccess) {
            hipStreamSynchronize(hipStreamPerThread);
            fail(MOE_ERR_HIP, "batched copy %d of %d failed", i, n);
            return false;
        }
    }
    return hipStreamSynchronize(hipStreamPerThread) == hipSuccess;
}

size_t moe_expert_bytes(int H, int I, int down_type) { return (size_t)mp::expert_bytes(H, I, down_type); }

int moe_synth_experts(uint64_t seed, int layer, int e0, int n, int H, int I, int down_type, float sigma,
                      void *out_dev, size_t stride, void *stream) {
    if (H % 256 || I % 256 || n <= 0 || !out_dev) return fail(MOE_ERR_ARG, "bad synth_experts arguments");
    if (stride < mp::expert_bytes(H, I, down_type)) return fail(MOE_ERR_ARG, "stride below expert size");
    HIPCHK(mp::launch_synth_experts(seed, layer, e0, n, H, I, down_type, sigma, (uint8_t *)out_dev, stride,
                                    (hipStream_t)stream));
    return MOE_OK;
}

int moe_synth_experts_host(uint64_t seed, int layer, int e0, int n, int H, int I, int down_type, float sigma,
                           void *out_host, size_t stride, int n_threads) {
    if (H % 256 || I % 256 || n <= 0 || !out_host) return fail(MOE_ERR_ARG, "bad synth_experts arguments");
    if (stride < mp::expert_bytes(H, I, down_type)) return fail(MOE_ERR_ARG, "stride below expert size");
    const mp::synth::ExpertShape sh{H, I, down_type};
    const uint64_t nblk = (uint64_t)sh.n_blocks();
    const uint64_t total = nblk * (uint64_t)n;
    if (n_threads < 1) n_threads = 1;
    std::vector<std::thread> th;
    for (int t = 0; t < n_threads; ++t) {
        th.emplace_back([=]() {
            for (uint64_t i = (uint64_t)t; i < total; i += (uint64_t)n_threads) {
                const int e = (int)(i / nblk), blk = (int)(i % nblk);
                mp::synth::expert_block(seed, layer, e0 + e, sh, blk, sigma,
                                        (uint8_t *)out_host + (uint64_t)e * stride + sh.block_offset(blk));
            }
        });
    }
    for (auto &x : th) x.join();
    return MOE_OK;
}

int moe_synth_vec(uint64_t seed, int kind, int a0, int na, int b0, int nb, int n, float sigma, float *out_dev,
                  void *stream) {
    if (na <= 0 || nb <= 0 || n <= 0 || !out_dev) return fail(MOE_ERR_ARG, "bad synth_vec arguments");
    HIPCHK(mp::launch_synth_vec(seed, kind, a0, na, b0, nb, n, sigma, out_dev, (hipStream_t)stream));
    return MOE_OK;
}

int moe_probe_stream_read(const void *buf, size_t buf_bytes, size_t bytes, int iters, double *avg_us,
                          void *stream) {
    if (!buf || !avg_us || bytes < 16 || bytes > buf_bytes || iters < 1 || (uintptr_t)buf % 16)
        return fail(MOE_ERR_ARG, "moe_probe_stream_read: bad arguments");
    const hipStream_t st = (hipStream_t)stream;
    uint32_t *out = nullptr;
    hipEvent_t e0 = nullptr, e1 = nullptr;
    if (hipMalloc(&out, (size_t)mp::stream_read_blocks(bytes) * 4) != hipSuccess)
        return fail(MOE_ERR_NOMEM, "probe scratch");
    const size_t step = (bytes + 4095) / 4096 * 4096;
    double sum = 0.0;
    int r = MOE_OK;
    if (hipEventCreate(&e0) != hipSuccess || hipEventCreate(&e1) != hipSuccess) r = fail(MOE_ERR_HIP, "events");
    size_t off = 0;
    for (int i = 0; i < iters + 3 && r == MOE_OK; ++i) {   // 3 untimed; a fresh window each launch
        if (off + bytes > buf_bytes) off = 0;
        if (mp::launch_stream_read((const uint8_t *)buf + off, bytes, out, st, e0, e1) != hipSuccess ||
            hipEventSynchronize(e1) != hipSuccess) {
            r = fail(MOE_ERR_HIP, "stream read launch");
            break;
        }
        float ms = 0.0f;
        if (hipEventElapsedTime(&ms, e0, e1) != hipSuccess) r = fail(MOE_ERR_HIP, "event time");
        if (i >= 3) sum += ms * 1e3;
        off += step;
    }
    if (e0) hipEventDestroy(e0);
    if (e1) hipEventDestroy(e1);
    hipFree(out);
    if (r == MOE_OK) *avg_us = sum / iters;
    return r;
}

int moe_synth_vec_host(uint64_t seed, int kind, int a0, int na, int b0, int nb, int n, float sigma, float *out) {
    if (na <= 0 || nb <= 0 || n <= 0 || !out) return fail(MOE_ERR_ARG, "bad synth_vec arguments");
    size_t t = 0;
    for (int a = 0; a < na; ++a)
        for (int b = 0; b < nb; ++b)
            for (int i = 0; i < n; ++i) out[t++] = mp::synth::vec_value(seed, kind, a0 + a, b0 + b, i, sigma);
    return MOE_OK;
}

size_t moe_route_workspace_bytes(int E, int n_tok) { return route_ws_bytes(E, n_tok); }
size_t moe_experts_workspace_bytes(int I, int K) { return exp_ws_bytes(I, K); }

int moe_route(const moe_route_desc *d, void *stream) {
    if (!d || !d->ids || !d->w || !d->slots || !d->workspace) return fail(MOE_ERR_ARG, "moe_route: null argument");
    if (!d->logits && (!d->W || !d->x || !d->q8x))
        return fail(MOE_ERR_ARG, "moe_route: W, x and q8x are required without given logits");
    int r = check_shape(d->E, d->H, 0, d->K);
    if (r != MOE_OK) return r;
    if (d->n_tok < 1 || d->n_tok > 65535) return fail(MOE_ERR_ARG, "n_tok %d out of range", d->n_tok);
    return run_route(d, (hipStream_t)stream);
}

int moe_cpu_experts(const void *const *experts, int n, const uint8_t *q8x, int H, int I, int down_type, float *rows,
                    int n_threads, int portable) {
    if (!experts || !q8x || !rows || n < 0) return fail(MOE_ERR_ARG, "moe_cpu_experts: bad arguments");
    int r = check_shape(64, H, I, 1);
    if (r != MOE_OK) return r;
    if (I == 0) return fail(MOE_ERR_ARG, "intermediate size 0");
    if (down_type != MOE_TYPE_Q4K && down_type != MOE_TYPE_Q6K)
        return fail(MOE_ERR_ARG, "down type %d unsupported", down_type);
    std::vector<mpc::CpuExpert> e((size_t)n);
    for (int k = 0; k < n; ++k) {
        if (!experts[k]) return fail(MOE_ERR_ARG, "moe_cpu_experts: expert %d is null", k);
        e[k] = {(const uint8_t *)experts[k], q8x, rows + (size_t)k * H};
    }
    std::vector<float> h((size_t)n * I);
    std::vector<uint8_t> q8h((size_t)n * (I / 256) * mp::Q8K_BYTES);
    // one team per thread count, kept for later calls (a team's threads start
    // once, not per call); calls run one at a time
    static std::mutex m;
    static std::map<int, mpc::Team *> teams;
    std::lock_guard<std::mutex> lk(m);
    mpc::Team *&t = teams[n_threads < 1 ? 1 : n_threads];
    if (!t) t = mpc::team_create(n_threads < 1 ? 1 : n_threads);
    mpc::set_portable(portable != 0);
    mpc::experts(t, e.data(), n, H, I, down_type, h.data(), q8h.data());
    mpc::set_portable(false);
    return MOE_OK;
}

int moe_cpu_experts_tokens(const void *const *experts, int n_groups, const int32_t *count, const uint8_t *q8x,
                           int H, int I, int down_type, float *rows, int n_threads) {
    if (!experts || !count || !q8x || !rows || n_groups < 0) return fail(MOE_ERR_ARG, "moe_cpu_experts_tokens: bad arguments");
    int r = check_shape(64, H, I, 1);
    if (r != MOE_OK) return r;
    if (I == 0) return fail(MOE_ERR_ARG, "intermediate size 0");
    if (down_type != MOE_TYPE_Q4K && down_type != MOE_TYPE_Q6K)
        return fail(MOE_ERR_ARG, "down type %d unsupported", down_type);
    std::vector<mpc::CpuGroup> g((size_t)n_groups);
    int n = 0;
    for (int k = 0; k < n_groups; ++k) {
        if (!experts[k] || count[k] < 1) return fail(MOE_ERR_ARG, "moe_cpu_experts_tokens: group %d is empty", k);
        g[(size_t)k] = {(const uint8_t *)experts[k], n, count[k]};
        n += count[k];
    }
    const size_t q8row = (size_t)(H / 256) * mp::Q8K_BYTES;
    std::vector<const uint8_t *> q8p((size_t)n);
    std::vector<float *> yp((size_t)n);
    for (int j = 0; j < n; ++j) {
        q8p[(size_t)j] = q8x + (size_t)j * q8row;
        yp[(size_t)j] = rows + (size_t)j * H;
    }
    std::vector<float> h((size_t)n * I);
    std::vector<uint8_t> q8h((size_t)n * (I / 256) * mp::Q8K_BYTES);
    static std::mutex m;
    static std::map<int, mpc::Team *> teams;
    std::lock_guard<std::mutex> lk(m);
    mpc::Team *&t = teams[n_threads < 1 ? 1 : n_threads];
    if (!t) t = mpc::team_create(n_threads < 1 ? 1 : n_threads);
    mpc::experts_grouped(t, g.data(), n_groups, q8p.data(), yp.data(), H, I, down_type, h.data(), q8h.data());
    return MOE_OK;
}

int moe_cpu_has_vnni(void) { return mpc::has_vnni() ? 1 : 0; }

int moe_experts(const moe_experts_desc *d, void *stream) {
    if (!d || !d->ids || !d->slots || !d->w || !d->q8x || !d->out || !d->workspace)
        return fail(MOE_ERR_ARG, "moe_experts: null argument");
    int r = check_shape(64, d->H, d->I, d->K);
    if (r != MOE_OK) return r;
    if (d->I == 0) return fail(MOE_ERR_ARG, "intermediate size 0");
    if (d->down_type != MOE_TYPE_Q4K && d->down_type != MOE_TYPE_Q6K)
        return fail(MOE_ERR_ARG, "down type %d unsupported", d->down_type);
    if (!d->host_store && !d->slot_pool) return fail(MOE_ERR_ARG, "no weights");
    if (d->expert_bytes != mp::expert_bytes(d->H, d->I, d->down_type))
        return fail(MOE_ERR_ARG, "expert_bytes %llu does not match the shape", (unsigned long long)d->expert_bytes);
    if (d->slot_pool && (d->slot_bytes < d->expert_bytes || d->slot_bytes % 16))
        return fail(MOE_ERR_ARG, "slot_bytes must be >= expert_bytes and a multiple of 16");
    if (((uintptr_t)d->slot_pool | (uintptr_t)d->host_store | (uintptr_t)d->q8x) % 16)
        return fail(MOE_ERR_ARG, "weights and activations must be 16-byte aligned");
    const int r2 = check_weight_ptrs("moe_experts", d->slot_pool, d->host_store);
    if (r2 != MOE_OK) return r2;
    return run_experts(d, (hipStream_t)stream);
}

int moe_cache_create(const moe_cache_config *cfg, moe_cache **out) {
    if (!cfg || !out) return fail(MOE_ERR_ARG, "null argument");
    *out = nullptr;
    int r = check_shape(cfg->n_experts, cfg->hidden, cfg->intermediate, cfg->n_expert_used);
    if (r != MOE_OK) return r;
    if (cfg->n_layers <= 0 || cfg->n_layers > 4096) return fail(MOE_ERR_ARG, "n_layers %d", cfg->n_layers);
    if (cfg->intermediate == 0) return fail(MOE_ERR_ARG, "intermediate size 0");
    moe_cache *c = new moe_cache();
    c->cfg = *cfg;
    if (c->cfg.max_inserts <= 0) c->cfg.max_inserts = 2;
    if (c->cfg.admit_window <= 0) c->cfg.admit_window = 8;
    if (c->cfg.admit_half <= 0) c->cfg.admit_half = 64;
    if (c->cfg.cache_prior < 0) c->cfg.cache_prior = 0;
    c->cfg.slot_profile = nullptr;
    c->cfg.down_type = nullptr;
    c->H = cfg->hidden;
    c->I = cfg->intermediate;
    c->E = cfg->n_experts;
    c->K = cfg->n_expert_used;
    const int NL = cfg->n_layers, E = c->E;
    auto bail = [&](int code) { free_cache(c); return code; };
    c->host_only = cfg->device < 0;
    if (!c->host_only && hipSetDevice(cfg->device) != hipSuccess)
        return bail(fail(MOE_ERR_HIP, "hipSetDevice(%d)", cfg->device));

    c->L.resize(NL);
    size_t pool_total = 0;
    for (int l = 0; l < NL; ++l) {
        Layer &ls = c->L[l];
        ls.il = l;
        ls.E = E;
        ls.S = cfg->slot_profile ? cfg->slot_profile[l] : cfg->n_slots;
        if (ls.S <= 0 || ls.S > 4096) return bail(fail(MOE_ERR_ARG, "layer %d: %d slots", l, ls.S));
        ls.down_type = cfg->down_type ? cfg->down_type[l] : MOE_TYPE_Q4K;
        if (ls.down_type != MOE_TYPE_Q4K && ls.down_type != MOE_TYPE_Q6K)
            return bail(fail(MOE_ERR_ARG, "layer %d: down type %d", l, ls.down_type));
        ls.expert_bytes = mp::expert_bytes(c->H, c->I, ls.down_type);
        ls.slot_bytes = align_up(ls.expert_bytes, 256);
        pool_total += (size_t)ls.S * ls.slot_bytes;
        ls.slot_expert.assign(ls.S, -1);
        ls.expert_slot.assign(E, -1);
        ls.slot_last_use.assign(ls.S, 0);
        ls.slot_protect.assign(ls.S, 0);
        ls.slot_in_flight.assign(ls.S, 0);
        ls.staged.assign(c->K, -1);
        ls.free_slots.resize(ls.S);
        for (int s = 0; s < ls.S; ++s) ls.free_slots[s] = ls.S - 1 - s;
        if (cfg->admit_mode == MOE_ADMIT_HEAT) ls.heat.assign(E, 0.0f);
        if (cfg->admit_mode == MOE_ADMIT_WINDOW) {
            ls.miss_last.assign(E, U64MAX);
            ls.miss_prev.assign(E, U64MAX);
        }
    }
    const size_t nt = (size_t)NL * E;
    if (c->host_only) {
        c->h_tbl = (int32_t *)malloc(nt * 4);
        c->h_prior = c->cfg.cache_prior > 0 ? (float *)calloc(nt, 4) : nullptr;
        if (!c->h_tbl || (c->cfg.cache_prior > 0 && !c->h_prior)) return bail(fail(MOE_ERR_NOMEM, "tables"));
        for (int l = 0; l < NL; ++l)
            for (int e = 0; e < E; ++e) c->h_tbl[(size_t)l * E + e] = c->L[l].S;
        *out = c;
        return MOE_OK;
    }
    if (hipMalloc(&c->pool_base, pool_total) != hipSuccess)
        return bail(fail(MOE_ERR_NOMEM, "slot pool of %zu bytes", pool_total));
    size_t off = 0;
    for (Layer &ls : c->L) {
        ls.pool = c->pool_base + off;
        off += (size_t)ls.S * ls.slot_bytes;
    }
    if (hipMalloc(&c->d_tbl, nt * 4) != hipSuccess || hipHostMalloc(&c->h_tbl, nt * 4, 0) != hipSuccess)
        return bail(fail(MOE_ERR_NOMEM, "tables"));
    for (int l = 0; l < NL; ++l)
        for (int e = 0; e < E; ++e) c->h_tbl[(size_t)l * E + e] = c->L[l].S;
    if (c->cfg.cache_prior > 0) {
        if (hipMalloc(&c->d_prior, nt * 4) != hipSuccess || hipHostMalloc(&c->h_prior, nt * 4, 0) != hipSuccess)
            return bail(fail(MOE_ERR_NOMEM, "prior tables"));
        memset(c->h_prior, 0, nt * 4);
    }
    if (hipMemcpy(c->d_tbl, c->h_tbl, nt * 4, hipMemcpyHostToDevice) != hipSuccess ||
        (c->d_prior && hipMemcpy(c->d_prior, c->h_prior, nt * 4, hipMemcpyHostToDevice) != hipSuccess))
        return bail(fail(MOE_ERR_HIP, "initial table write"));
    const size_t rws = route_ws_bytes(E, 1), ews = exp_ws_bytes(c->I, c->K);
    if (hipMalloc(&c->route_ws, rws) != hipSuccess || hipMalloc(&c->exp_ws, ews) != hipSuccess ||
        hipMalloc(&c->ypart, ((size_t)c->K + 1) * c->H * 4) != hipSuccess ||
        hipMalloc(&c->d_ids, (2 * (size_t)NL * c->K + 64) * 4) != hipSuccess ||
        hipMalloc(&c->d_w, (size_t)NL * c->K * 4) != hipSuccess ||
        hipMalloc(&c->d_q8x, (size_t)(c->H / 256) * mp::Q8K_BYTES + 256) != hipSuccess ||
        hipHostMalloc(&c->h_ids, (2 * (size_t)NL * c->K + 64) * 4, 0) != hipSuccess ||
        hipHostMalloc((void **)&c->h_pub, ((size_t)NL * c->K + 1) * 8, hipHostMallocMapped | hipHostMallocCoherent) !=
            hipSuccess ||
        hipHostGetDevicePointer((void **)&c->h_pub_d, c->h_pub, 0) != hipSuccess ||
        hipMalloc(&c->d_pub_ctr, (size_t)NL * 8) != hipSuccess ||
        hipMalloc(&c->fx, (size_t)NL * mp::fused_words(c->K, c->I, c->H) * 8) != hipSuccess ||
        hipHostMalloc((void **)&c->h_seq, 64, hipHostMallocDefault) != hipSuccess ||
        hipMalloc(&c->d_seq, 64) != hipSuccess)
        return bail(fail(MOE_ERR_NOMEM, "decode scratch"));
    // ids [L][K], the late-wait word and padding, then slots [L][K]: one copy back
    // per token, or unpacked from the words the fused launches publish (h_pub)
    memset(c->h_pub, 0, ((size_t)NL * c->K + 1) * 8);
    c->d_slots = c->d_ids + (size_t)NL * c->K + 64;
    c->h_slots = c->h_ids + (size_t)NL * c->K + 64;
    // tag 0 is never a token's sequence number: zeroed exchange words are stale
    if (hipMemset(c->route_ws, 0, rws) != hipSuccess || hipMemset(c->exp_ws, 0, ews) != hipSuccess ||
        hipMemset(c->fx, 0, (size_t)NL * mp::fused_words(c->K, c->I, c->H) * 8) != hipSuccess ||
        hipMemset(c->d_ids, 0, ((size_t)NL * c->K + 64) * 4) != hipSuccess || hipMemset(c->d_seq, 0, 64) != hipSuccess ||
        hipMemset(c->d_pub_ctr, 0, (size_t)NL * 8) != hipSuccess)
        return bail(fail(MOE_ERR_HIP, "scratch clear"));
    c->fx_words = mp::fused_words(c->K, c->I, c->H);
    if (hipStreamCreateWithFlags(&c->up_stream, hipStreamNonBlocking) != hipSuccess ||
        hipStreamCreateWithFlags(&c->tbl_stream, hipStreamNonBlocking) != hipSuccess ||
        hipStreamCreateWithFlags(&c->host_stream, hipStreamNonBlocking) != hipSuccess ||
        hipEventCreateWithFlags(&c->up_mark, hipEventDisableTiming) != hipSuccess ||
        hipStreamCreateWithFlags(&c->stg_stream, hipStreamNonBlocking) != hipSuccess ||
        hipEventCreateWithFlags(&c->ev_stg, hipEventDisableTiming) != hipSuccess ||
        hipEventCreateWithFlags(&c->ev_dec, hipEventDisableTiming) != hipSuccess ||
        hipEventCreateWithFlags(&c->ev_route, hipEventDisableTiming) != hipSuccess ||
        hipEventCreateWithFlags(&c->ev_hbm, hipEventDisableTiming) != hipSuccess ||
        hipEventCreateWithFlags(&c->ev_host, hipEventDisableTiming) != hipSuccess ||
        hipStreamCreateWithFlags(&c->cap_stream, hipStreamNonBlocking) != hipSuccess ||
        hipEventCreateWithFlags(&c->ev_user, hipEventDisableTiming) != hipSuccess ||
        hipEventCreateWithFlags(&c->ev_done, hipEventDisableTiming) != hipSuccess)
        return bail(fail(MOE_ERR_HIP, "streams"));
    if (hipMalloc(&c->x_buf, (size_t)NL * c->H * 4) != hipSuccess ||
        hipMalloc(&c->bias_buf, (size_t)NL * E * 4) != hipSuccess ||
        hipMalloc(&c->out_buf, (size_t)NL * c->H * 4) != hipSuccess)
        return bail(fail(MOE_ERR_NOMEM, "decode buffers"));
    *out = c;
    return MOE_OK;
}

int moe_cache_destroy(moe_cache *c) {
    free_cache(c);
    return MOE_OK;
}

// captured token graphs hold kernel arguments: drop them when weights move
static void drop_graphs(moe_cache *c) {
    for (int i = 0; i < 2; ++i) {
        if (c->gx[i]) { hipGraphExecDestroy(c->gx[i]); c->gx[i] = nullptr; }
        if (c->g[i]) { hipGraphDestroy(c->g[i]); c->g[i] = nullptr; }
        c->g_mode[i] = -1;
    }
}

int moe_cache_set_host_store(moe_cache *c, int layer, const void *experts, size_t expert_bytes) {
    if (!c || layer < 0 || layer >= (int)c->L.size() || !experts) return fail(MOE_ERR_ARG, "bad arguments");
    if (c->host_only) return fail(MOE_ERR_STATE, "host-only cache (device < 0) holds no weights");
    Layer &ls = c->L[layer];
    if (expert_bytes != ls.expert_bytes)
        return fail(MOE_ERR_ARG, "layer %d expects %llu bytes per expert, got %zu", layer,
                    (unsigned long long)ls.expert_bytes, expert_bytes);
    void *dev = nullptr;
    HIPCHK(hipHostGetDevicePointer(&dev, const_cast<void *>(experts), 0));
    if (((uintptr_t)dev | (uintptr_t)experts) % 16) return fail(MOE_ERR_ARG, "host store must be 16-byte aligned");
    if (ls.store_dev != dev) drop_graphs(c);
    ls.store_host = (const uint8_t *)experts;
    ls.store_dev = (const uint8_t *)dev;
    if (c->sc_den > 0) mpc::prefault(c->team, ls.store_host, (size_t)ls.E * ls.expert_bytes);
    return MOE_OK;
}

int moe_cache_set_router(moe_cache *c, int layer, const float *W_dev) {
    if (!c || layer < 0 || layer >= (int)c->L.size() || !W_dev) return fail(MOE_ERR_ARG, "bad arguments");
    if ((uintptr_t)W_dev % 16) return fail(MOE_ERR_ARG, "router must be 16-byte aligned");
    if (c->L[layer].router != W_dev) drop_graphs(c);
    c->L[layer].router = W_dev;
    return MOE_OK;
}

int moe_cache_set_shared(moe_cache *c, int layer, const void *expert, size_t expert_bytes) {
    if (!c || layer < 0 || layer >= (int)c->L.size()) return fail(MOE_ERR_ARG, "bad arguments");
    if (c->host_only) return fail(MOE_ERR_STATE, "host-only cache (device < 0) holds no weights");
    Layer &ls = c->L[layer];
    if (!expert) {
        if (ls.shared) drop_graphs(c);
        hipFree(ls.shared);
        ls.shared = nullptr;
        return MOE_OK;
    }
    if (expert_bytes != ls.expert_bytes)
        return fail(MOE_ERR_ARG, "shared expert of %zu bytes, the layer's experts are %llu", expert_bytes,
                    (unsigned long long)ls.expert_bytes);
    if (c->K + 1 > 17) return fail(MOE_ERR_ARG, "a shared expert needs n_expert_used <= 16");
    HIPCHK(hipSetDevice(c->cfg.device));
    if (!ls.shared) {
        if (hipMalloc(&ls.shared, ls.expert_bytes) != hipSuccess)
            return fail(MOE_ERR_NOMEM, "shared expert of %llu bytes", (unsigned long long)ls.expert_bytes);
        drop_graphs(c);
    }
    HIPCHK(hipMemcpy(ls.shared, expert, expert_bytes, hipMemcpyDefault));
    return MOE_OK;
}

int moe_cache_lookup(moe_cache *c, int layer, moe_layer_view *out) {
    if (!c || !out || layer < 0 || layer >= (int)c->L.size()) return fail(MOE_ERR_ARG, "bad arguments");
    const Layer &ls = c->L[layer];
    out->il = ls.il;
    out->n_slots = ls.S;
    out->n_experts = ls.E;
    out->down_type = ls.down_type;
    out->slot_bytes = ls.slot_bytes;
    out->expert_bytes = ls.expert_bytes;
    out->slot_pool = ls.pool;
    out->dev_table = c->d_tbl + (size_t)layer * c->E;
    out->prior = c->d_prior ? c->d_prior + (size_t)layer * c->E : nullptr;
    out->host_store = ls.store_host;
    out->router = ls.router;
    return MOE_OK;
}

int moe_cache_trace_open(moe_cache *c, const char *route_path, const char *map_path) {
    if (!c) return fail(MOE_ERR_ARG, "null cache");
    if (route_path) {
        c->route = fopen(route_path, "w");
        if (!c->route) return fail(MOE_ERR_IO, "cannot open %s", route_path);
    }
    if (map_path) {
        if (c->replay) return fail(MOE_ERR_STATE, "a map is being replayed: it cannot be recorded too");
        c->map = fopen(map_path, "w");
        if (!c->map) return fail(MOE_ERR_IO, "cannot open %s", map_path);
        fprintf(c->map, "moe-map 1 %zu\n", c->L.size());
        for (const Layer &ls : c->L) fprintf(c->map, "layer %d %d %d\n", ls.il, ls.S, ls.E);
        map_frame(c);
    }
    return MOE_OK;
}

// the state of a layer decoded by moe_decode_layer since the last step
enum : uint8_t {
    PL_DECODED = 1,     // decoded since the last step
    PL_FUSED = 2,       // by the fused launch
    PL_SIDECAR = 4,     // the host served its share of the absent experts
    PL_STAGE = 8,       // the kernels staged the experts they read from the pinned store
    PL_AGAIN = 16,      // decoded more than once: nothing of it is staged, its routing is not compared
    PL_OBSERVED = 32,   // its ids were observed
};

static int pl_observe(moe_cache *c, int l, const int32_t *ids);
static int pl_step(moe_cache *c);

int moe_cache_observe(moe_cache *c, int layer, const int32_t *ids, int n_ids, int n_tok) {
    if (!c || !ids || layer < 0 || layer >= (int)c->L.size() || n_ids <= 0 || n_tok <= 0)
        return fail(MOE_ERR_ARG, "bad arguments");
    // a layer moe_decode_layer decoded: its record first (early issue may
    // upload from the staging area inside the observe)
    const bool pl = !c->pl_flags.empty() && (c->pl_flags[(size_t)layer] & PL_DECODED) && n_tok == 1 && n_ids == c->K;
    if (pl) {
        const int r = pl_observe(c, layer, ids);
        if (r != MOE_OK) return r;
    }
    c->stage_valid = pl;
    const int r = cache_observe(c, layer, ids, n_ids, n_tok);
    c->stage_valid = false;
    return r;
}

int moe_cache_step(moe_cache *c) {
    if (!c) return fail(MOE_ERR_ARG, "null cache");
    if (!c->pl_streams.empty()) return pl_step(c);
    return cache_step(c);
}

int moe_cache_requires_sync(const moe_cache *c) {
    return c && (c->cfg.publish == MOE_PUBLISH_SORTED || c->replay) ? 1 : 0;
}

int moe_cache_freeze(moe_cache *c) {
    if (!c) return fail(MOE_ERR_ARG, "null cache");
    c->freeze = true;
    c->cfg.max_inserts = 0;
    return MOE_OK;
}

int moe_cache_heat_file(moe_cache *c, const char *path, int64_t *n_records, int64_t *n_placed) {
    if (!c || !path) return fail(MOE_ERR_ARG, "bad arguments");
    if (c->n_steps != 0 || !c->jobs.empty()) return fail(MOE_ERR_STATE, "the heat file is read before the first step");
    for (const Layer &ls : c->L)
        for (int s = 0; s < ls.S; ++s)
            if (ls.slot_expert[s] >= 0) return fail(MOE_ERR_STATE, "the heat file needs an empty cache");
    if (!c->host_only)
        for (const Layer &ls : c->L)
            if (!ls.store_host) return fail(MOE_ERR_STATE, "layer %d: register the host store first", ls.il);
    c->heat_path = path;
    for (Layer &ls : c->L) ls.use_count.assign(ls.E, 0);
    // load (patches/0007:434-466): another model's dimensions are refused by name
    int64_t n_rec = 0, placed = 0;
    if (FILE *f = fopen(path, "r")) {
        int ver = 0, nl = 0, ne = 0;
        if (fscanf(f, "moe-heat %d %d %d", &ver, &nl, &ne) != 3 || ver != 1 || nl != (int)c->L.size() || ne != c->E) {
            fprintf(stderr, "moe-cache: HEAT FILE REFUSED: %s is v%d for %d layers x %d experts, this cache holds "
                            "%zu x %d\n", path, ver, nl, ne, c->L.size(), c->E);
        } else {
            int il = 0, e = 0;
            unsigned cnt = 0;
            while (fscanf(f, "%d %d %u", &il, &e, &cnt) == 3) {
                if (il < 0 || il >= (int)c->L.size() || e < 0 || e >= c->L[il].E) continue;
                c->L[il].use_count[e] = cnt / 2;     // halved, so an old workload fades
                n_rec++;
            }
        }
        fclose(f);
    }
    // warm start (patches/0007:568-611): hottest first into slots 0.., a reserve
    // for early issue; the hottest is the most recent use, so LRU evicts the
    // coldest of the warm set first
    if (n_rec > 0) {
        const int reserve = c->cfg.early_issue ? c->cfg.max_inserts + (c->pred ? c->predict_top : 0) : 0;
        for (Layer &ls : c->L) {
            std::vector<int32_t> order(ls.E);
            for (int e = 0; e < ls.E; ++e) order[e] = e;
            std::stable_sort(order.begin(), order.end(),
                             [&](int32_t a, int32_t b) { return ls.use_count[a] > ls.use_count[b]; });
            const int fill = std::max(0, ls.S - reserve);
            int slot = 0;
            for (int k = 0; k < ls.E && slot < fill; ++k) {
                const int e = order[k];
                if (ls.use_count[e] == 0) break;         // never routed to: not worth a slot on a guess
                const int r = place_bytes(c, ls, e, slot);
                if (r != MOE_OK) return r;
                ls.slot_expert[slot] = e;
                ls.expert_slot[e] = slot;
                ls.slot_last_use[slot] = (uint64_t)(fill - slot);
                set_table_entry(c, ls, e, slot);
                ++slot;
                ++placed;
            }
            c->clock = std::max<uint64_t>(c->clock, (uint64_t)fill);
            ls.free_slots.clear();
            for (int f2 = ls.S - 1; f2 >= slot; --f2) ls.free_slots.push_back(f2);   // lowest free on top
        }
        if (!c->host_only) HIPCHK(hipStreamSynchronize(c->up_stream));
        const int r = flush_tables(c);
        if (r != MOE_OK) return r;
    }
    fprintf(stderr, "moe-cache: heat file %s: %lld records, %lld experts placed before the first token%s\n", path,
            (long long)n_rec, (long long)placed, n_rec ? "" : " (COLD START - file missing, empty or refused)");
    if (n_records) *n_records = n_rec;
    if (n_placed) *n_placed = placed;
    return MOE_OK;
}

int moe_cache_map_replay(moe_cache *c, const char *path) {
    if (!c || !path) return fail(MOE_ERR_ARG, "bad arguments");
    if (c->map) return fail(MOE_ERR_STATE, "a map is being recorded: it cannot be replayed too");
    if (c->replay) return fail(MOE_ERR_STATE, "a map is already being replayed");
    if (c->n_steps != 0 || !c->jobs.empty()) return fail(MOE_ERR_STATE, "a replay starts before the first step");
    FILE *f = fopen(path, "r");
    if (!f) return fail(MOE_ERR_IO, "cannot open %s", path);
    int ver = 0, nl = 0;
    bool ok = fscanf(f, "moe-map %d %d", &ver, &nl) == 2 && ver == 1 && nl == (int)c->L.size();
    for (const Layer &ls : c->L) {
        int il = -1, s = 0, e = 0;
        ok = ok && fscanf(f, " layer %d %d %d", &il, &s, &e) == 3 && il == ls.il && s == ls.S && e == ls.E;
    }
    if (!ok) {
        fclose(f);
        return fail(MOE_ERR_ARG, "%s does not describe this cache's layers and slots", path);
    }
    c->replay = f;
    moe_cache_freeze(c);
    return map_frame(c);             // the frame of step 0, as at the reference's init (patches/0008:571)
}

// ---- router lookahead and just-in-time streaming ----------------------------
int moe_cache_set_norm(moe_cache *c, int layer, const float *g_host, int n) {
    if (!c || !g_host || layer < 0 || layer >= (int)c->L.size()) return fail(MOE_ERR_ARG, "bad arguments");
    if (n != c->H) return fail(MOE_ERR_ARG, "norm of %d values, the hidden size is %d", n, c->H);
    if (c->norm.empty()) {
        c->norm.assign(c->L.size() * (size_t)c->H, 0.0f);
        c->has_norm.assign(c->L.size(), 0);
    }
    memcpy(c->norm.data() + (size_t)layer * c->H, g_host, (size_t)n * sizeof(float));
    c->has_norm[(size_t)layer] = 1;
    return MOE_OK;
}

static int stream_live_init(moe_cache *c, Streamer *st) {
    const int NL = (int)c->L.size();
    for (const Layer &ls : c->L)
        if (!ls.router || !ls.store_host) return fail(MOE_ERR_STATE, "layer %d: router or host store missing", ls.il);
    // pairs (L, T = L+1, L+2): r = g_T / g_L, so W_T . (x_L * r) = W_T . (rmsnorm(residual_L) * g_T)
    std::vector<float> ratio((size_t)NL * 2 * c->H, 0.0f);
    st->targets.assign((size_t)NL, {-1, -1});
    int pairs = 0;
    for (int l = 0; l < NL; ++l) {
        for (int d = 1; d <= 2; ++d) {
            const int T = l + d;
            if (T >= NL || c->has_norm.empty() || !c->has_norm[(size_t)l] || !c->has_norm[(size_t)T]) continue;
            const float *gl = c->norm.data() + (size_t)l * c->H, *gt = c->norm.data() + (size_t)T * c->H;
            float *r = ratio.data() + ((size_t)l * 2 + (d - 1)) * c->H;
            bool ok = true;
            for (int i = 0; i < c->H && ok; ++i) {
                ok = std::fabs(gl[i]) >= 1e-12f;
                r[i] = gt[i] / gl[i];
            }
            if (!ok) {
                fprintf(stderr, "moe-cache: lookahead %d -> %d skipped: a zero norm weight in layer %d\n", l, T, l);
                continue;
            }
            st->targets[(size_t)l][(size_t)(d - 1)] = T;
            pairs++;
        }
    }
    if (!pairs) return fail(MOE_ERR_STATE, "no layer pair has norm weights: call moe_cache_set_norm for every layer");
    int max_s = 0;
    for (const Layer &ls : c->L) max_s = std::max(max_s, ls.S);
    const unsigned fl = hipHostMallocMapped | hipHostMallocCoherent;
    if (hipMalloc(&st->ratio, ratio.size() * sizeof(float)) != hipSuccess ||
        hipMalloc(&st->alog, 2 * (size_t)c->E * sizeof(float)) != hipSuccess ||
        hipMalloc(&st->fresh, (size_t)NL * sizeof(uint32_t)) != hipSuccess ||
        hipHostMalloc((void **)&st->post, (size_t)NL * sizeof(mp::AheadPost), fl) != hipSuccess ||
        hipHostMalloc((void **)&st->words, (size_t)max_s * sizeof(int32_t), 0) != hipSuccess)
        return fail(MOE_ERR_NOMEM, "streaming buffers");
    memset((void *)st->post, 0, (size_t)NL * sizeof(mp::AheadPost));
    for (int v = 0; v < max_s; ++v) st->words[v] = v | mp::STREAM_BIT;
    HIPCHK(hipHostGetDevicePointer((void **)&st->post_d, st->post, 0));
    HIPCHK(hipMemcpy(st->ratio, ratio.data(), ratio.size() * sizeof(float), hipMemcpyHostToDevice));
    HIPCHK(hipMemset(st->fresh, 0, (size_t)NL * sizeof(uint32_t)));
    HIPCHK(hipStreamCreateWithFlags(&st->stream, hipStreamNonBlocking));
    st->ev.assign(64, nullptr);
    st->ev_ticket.assign(64, 0);
    for (auto &e : st->ev) HIPCHK(hipEventCreateWithFlags(&e, hipEventDisableTiming));
    if (!c->h_seq) {
        if (hipHostMalloc((void **)&c->h_seq, 64, hipHostMallocDefault) != hipSuccess ||
            hipMalloc(&c->d_seq, 64) != hipSuccess)
            return fail(MOE_ERR_NOMEM, "sequence number");
        HIPCHK(hipMemset(c->d_seq, 0, 64));
    }
    st->live = true;
    st->thr = std::thread(mover_loop, c);
    return MOE_OK;
}

int moe_cache_set_streaming(moe_cache *c, const moe_stream_config *cfg) {
    if (!c || !cfg) return fail(MOE_ERR_ARG, "null argument");
    if (!cfg->on) {
        if (c->st) {
            if (!c->st->jobs.empty()) return fail(MOE_ERR_STATE, "streaming jobs still open: step first");
            stream_free(c);
            if (!c->host_only) drop_graphs(c);
        }
        return MOE_OK;
    }
    if (c->st) return fail(MOE_ERR_STATE, "streaming is on already");
    if (!c->cfg.early_issue) return fail(MOE_ERR_STATE, "streaming needs early issue (LLAMA_MOE_EARLY_ISSUE=1)");
    if (c->cfg.publish == MOE_PUBLISH_SORTED || c->replay || c->freeze)
        return fail(MOE_ERR_STATE, "streaming runs without deterministic publication, replay or freeze");
    if (c->map) return fail(MOE_ERR_STATE, "enable streaming before opening a map record");
    if (cfg->top_k < 0 || cfg->top_k > mp::AHEAD_K) return fail(MOE_ERR_ARG, "top_k %d: 1..%d", cfg->top_k, mp::AHEAD_K);
    Streamer *st = new Streamer();
    st->per_layer = cfg->per_layer > 0 ? cfg->per_layer : 4;
    st->reserve = cfg->reserve >= 0 ? cfg->reserve : 2;
    st->top_k = cfg->top_k > 0 ? cfg->top_k : 8;
    st->bytes_per_ns = cfg->gbps >= 1.0 ? cfg->gbps : 45.7;
    // one push per expert by default: each host-to-device copy costs a fixed
    // ~8 us on this GPU, so 512 KiB chunks move an expert at ~26 GB/s and a
    // whole expert goes at ~44 GB/s
    size_t chunk = (size_t)std::max(0, cfg->chunk_kib) << 10;
    if (!chunk)
        for (const Layer &ls : c->L) chunk = std::max(chunk, (size_t)ls.expert_bytes);
    if (!chunk) chunk = (size_t)mp::expert_bytes(c->H, c->I, MOE_TYPE_Q6K);
    st->planner = mps::Planner(chunk);
    st->max_outstanding = std::max<size_t>(st->max_outstanding, 2 * chunk);
    st->mark.assign(c->L.size() * (size_t)c->E, 0);
    st->n_this_token.assign(c->L.size(), 0);
    st->arrive_ns.assign(c->L.size(), 0);
    c->st = st;
    if (!c->host_only) {
        HIPCHK(hipSetDevice(c->cfg.device));
        const int r = stream_live_init(c, st);
        if (r != MOE_OK) {
            const std::string msg = g_err;
            stream_free(c);
            return fail(r, "%s", msg.c_str());
        }
        drop_graphs(c);
    }
    return MOE_OK;
}

int moe_cache_stream_stats(moe_cache *c, moe_stream_stats *out) {
    if (!c || !out) return fail(MOE_ERR_ARG, "null argument");
    memset(out, 0, sizeof(*out));
    const Streamer *st = c->st;
    if (!st) return MOE_OK;
    uint64_t v[SN_COUNT];
    memcpy(v, st->n, sizeof v);
    v[SN_DROP_LATE] = st->planner.n_drop_late > v[SN_DROP_LATE] ? st->planner.n_drop_late : v[SN_DROP_LATE];
    v[SN_DROP_POSTED] = st->planner.n_drop_posted > v[SN_DROP_POSTED] ? st->planner.n_drop_posted : v[SN_DROP_POSTED];
    out->records = v[SN_RECORDS];
    out->offered = v[SN_OFFERED];
    out->landed = v[SN_LANDED];
    out->in_time = v[SN_IN_TIME];
    out->late = v[SN_LATE];
    out->unused = v[SN_UNUSED];
    out->dropped_late = v[SN_DROP_LATE];
    out->dropped_posted = v[SN_DROP_POSTED];
    out->not_sent = v[SN_NOT_SENT];
    out->gpu_miss = v[SN_GPU_MISS];
    out->bytes = v[SN_BYTES];
    for (int d = 0; d < 3; ++d) {
        out->lead_n[d] = st->lead_n[d];
        out->lead_us[d] = st->lead_n[d] ? st->lead_sum[d] / (double)st->lead_n[d] / 1000.0 : 0.0;
    }
    out->tau_us = st->tau_ns / 1000.0;
    out->failed = st->failed ? 1 : 0;
    return MOE_OK;
}

int moe_cache_observe_gpu(moe_cache *c, int layer, const int32_t *ids, const int32_t *gpu_slots, int n_ids) {
    if (!c || !ids || !gpu_slots || layer < 0 || layer >= (int)c->L.size() || n_ids <= 0)
        return fail(MOE_ERR_ARG, "bad arguments");
    return cache_observe(c, layer, ids, n_ids, 1, c->st ? gpu_slots : nullptr);
}

static int scripted(moe_cache *c) {
    if (!c) return fail(MOE_ERR_ARG, "null cache");
    if (!c->st) return fail(MOE_ERR_STATE, "streaming is off");
    if (!c->host_only) return fail(MOE_ERR_STATE, "scripted streaming is for host-only caches (device < 0)");
    return MOE_OK;
}

int moe_cache_stream_take(moe_cache *c, int layer, const int32_t *targets, const int32_t *n, const int32_t *ids,
                          uint64_t now_ns, uint64_t t_ns, uint64_t expert_bytes) {
    const int r = scripted(c);
    if (r != MOE_OK) return r;
    if (!targets || !n || !ids || layer < 0 || layer >= (int)c->L.size()) return fail(MOE_ERR_ARG, "bad arguments");
    return stream_take(c, layer, targets, n, ids, now_ns, t_ns, expert_bytes);
}

int moe_cache_stream_posted(moe_cache *c, int layer) {
    const int r = scripted(c);
    if (r != MOE_OK) return r;
    stream_posted(c, layer, 0);
    return MOE_OK;
}

int moe_cache_stream_next(moe_cache *c, uint64_t free_at_ns, int hold_after, moe_stream_chunk *out) {
    const int r = scripted(c);
    if (r != MOE_OK) return r;
    mps::Chunk ch;
    if (!stream_next(c, free_at_ns, hold_after, ch)) return 0;
    if (out) *out = moe_stream_chunk{ch.job, ch.offset, ch.len, ch.last};
    return 1;
}

int moe_cache_stream_land(moe_cache *c, int job) {
    const int r = scripted(c);
    if (r != MOE_OK) return r;
    stream_land(c, job);
    return MOE_OK;
}

int moe_cache_stream_job(moe_cache *c, int job, int32_t *layer, int32_t *expert) {
    if (!c || !c->st || job < 0 || job >= (int)c->st->jobs.size()) return -1;
    if (layer) *layer = c->st->jobs[(size_t)job].li;
    if (expert) *expert = c->st->planner.get(job).expert;
    return c->st->jobs[(size_t)job].slot;
}

int moe_route_ahead(const moe_route_desc *d, const moe_ahead_desc *a, int32_t *out_n, int32_t *out_ids,
                    void *stream) {
    if (!d || !a || !out_n || !out_ids) return fail(MOE_ERR_ARG, "moe_route_ahead: null argument");
    if (d->n_tok != 1 || d->logits) return fail(MOE_ERR_ARG, "moe_route_ahead: batch-1 router GEMV only");
    if (a->n_targets < 1 || a->n_targets > 2 || a->top_k < 1 || a->top_k > mp::AHEAD_K || d->E > mp::MAX_E)
        return fail(MOE_ERR_ARG, "moe_route_ahead: %d targets, top %d, %d experts", a->n_targets, a->top_k, d->E);
    for (int t = 0; t < a->n_targets; ++t)
        if (!a->W[t] || !a->r[t] || !a->tbl[t]) return fail(MOE_ERR_ARG, "moe_route_ahead: target %d incomplete", t);
    hipStream_t st = (hipStream_t)stream;
    mp::AheadPost *rec = nullptr;
    float *alog = nullptr;
    uint32_t *fresh = nullptr;
    if (hipMalloc(&rec, sizeof(mp::AheadPost)) != hipSuccess || hipMalloc(&alog, 2 * (size_t)d->E * 4) != hipSuccess ||
        hipMalloc(&fresh, 4) != hipSuccess) {
        hipFree(rec);
        hipFree(alog);
        return fail(MOE_ERR_NOMEM, "moe_route_ahead scratch");
    }
    mp::RouteLaunch ah{};
    ah.an = a->n_targets;
    ah.ak = a->top_k;
    for (int t = 0; t < a->n_targets; ++t) {
        ah.aW[t] = a->W[t];
        ah.ar[t] = a->r[t];
        ah.atbl[t] = a->tbl[t];
        ah.adummy[t] = a->dummy[t];
        ah.atarget[t] = t;
    }
    ah.alog = alog;
    ah.apost = rec;
    ah.fresh = d->table ? fresh : nullptr;
    int r = run_route(d, st, nullptr, nullptr, nullptr, &ah);
    mp::AheadPost h{};
    if (r == MOE_OK && (hipMemcpyAsync(&h, rec, sizeof h, hipMemcpyDeviceToHost, st) != hipSuccess ||
                        hipStreamSynchronize(st) != hipSuccess))
        r = fail(MOE_ERR_HIP, "moe_route_ahead: copy back");
    hipFree(rec);
    hipFree(alog);
    hipFree(fresh);
    if (r != MOE_OK) return r;
    for (int t = 0; t < 2; ++t) {
        out_n[t] = h.n[t];
        for (int j = 0; j < mp::AHEAD_K; ++j) out_ids[t * mp::AHEAD_K + j] = j < h.n[t] ? h.ids[t][j] : -1;
    }
    return MOE_OK;
}

struct moe_planner {
    mps::Planner p;
    explicit moe_planner(uint64_t chunk) : p((size_t)chunk) {}
};

moe_planner *moe_planner_create(uint64_t chunk_bytes) { return chunk_bytes ? new moe_planner(chunk_bytes) : nullptr; }
void moe_planner_destroy(moe_planner *p) { delete p; }
void moe_planner_reset(moe_planner *p) {
    if (p) p->p.reset();
}
int moe_planner_offer(moe_planner *p, int target, int32_t expert, uint64_t bytes, uint64_t deadline_ns) {
    return p ? p->p.offer(target, expert, (size_t)bytes, deadline_ns) : -1;
}
void moe_planner_posted(moe_planner *p, int target) {
    if (p) p->p.posted(target);
}
int moe_planner_next(moe_planner *p, uint64_t free_at_ns, double bytes_per_ns, int hold_after, moe_stream_chunk *out) {
    if (!p || !out || !(bytes_per_ns > 0)) return 0;
    mps::Chunk ch;
    if (!p->p.next(free_at_ns, bytes_per_ns, hold_after, ch)) return 0;
    *out = moe_stream_chunk{ch.job, ch.offset, ch.len, ch.last};
    return 1;
}
int moe_planner_size(const moe_planner *p) { return p ? p->p.size() : 0; }
int moe_planner_get(const moe_planner *p, int id, moe_planner_job *out) {
    if (!p || !out || id < 0 || id >= p->p.size()) return -1;
    const mps::PlanJob &j = p->p.get(id);
    *out = moe_planner_job{j.target, j.expert, j.bytes, j.sent, j.deadline_ns, j.dropped, j.drop};
    return 0;
}
void moe_planner_counters(const moe_planner *p, uint64_t out[4]) {
    if (!p || !out) return;
    out[0] = p->p.n_offered;
    out[1] = p->p.n_dup;
    out[2] = p->p.n_drop_late;
    out[3] = p->p.n_drop_posted;
}

// ---- MOEP expert predictor ---------------------------------------------------------

static mpp::Lists to_lists(const moe_predictor_lists *in) {
    mpp::Lists l;
    if (!in) return l;
    for (int b = 0; b < 4; ++b) {
        l.ids[b] = in->ids[b];
        l.n[b] = in->ids[b] && in->n[b] > 0 ? (size_t)in->n[b] : 0;
    }
    return l;
}

int moe_predictor_load(const char *path, moe_predictor **out) {
    if (!path || !out) return fail(MOE_ERR_ARG, "moe_predictor_load: null argument");
    *out = nullptr;
    std::unique_ptr<moe_predictor> p(new moe_predictor());
    std::string err;
    if (!p->p.load(path, err)) return fail(MOE_ERR_IO, "%s", err.c_str());
    *out = p.release();
    return MOE_OK;
}

void moe_predictor_free(moe_predictor *p) { delete p; }

int moe_predictor_info_get(const moe_predictor *p, moe_predictor_info *out) {
    if (!p || !out) return fail(MOE_ERR_ARG, "null argument");
    const mpp::Predictor &q = p->p;
    *out = moe_predictor_info{q.shape.n_expert, q.shape.n_layers, q.shape.feat_dim, q.shape.top_k,
                              q.shape.d_model, q.shape.n_comp, (uint32_t)q.present.size(), q.has_pca() ? 1 : 0,
                              q.group_col[mpp::GROUP_PCA], q.group_col[mpp::GROUP_PREV],
                              q.group_col[mpp::GROUP_CUR], q.group_col[mpp::GROUP_BELOW],
                              q.group_col[mpp::GROUP_SELF_PREV]};
    return MOE_OK;
}

int moe_predictor_has_layer(const moe_predictor *p, int layer) { return p && p->p.has_layer(layer) ? 1 : 0; }

int moe_predictor_score(const moe_predictor *p, int layer, const moe_predictor_lists *in, float *out) {
    if (!p || !out) return fail(MOE_ERR_ARG, "null argument");
    if (!p->p.has_layer(layer)) return fail(MOE_ERR_ARG, "the predictor has no layer %d", layer);
    p->p.score(layer, to_lists(in), out);
    return MOE_OK;
}

int moe_predictor_top_k(const moe_predictor *p, const float *scores, int k, int32_t *out) {
    if (!p || !scores || !out || k < 0) return fail(MOE_ERR_ARG, "bad arguments");
    return (int)p->p.top(scores, (size_t)k, out);
}

int moe_predictor_update(moe_predictor *p, int layer, const moe_predictor_lists *in, const int32_t *truth,
                         int n_truth, float lr, float *recall) {
    if (!p || (n_truth > 0 && !truth)) return fail(MOE_ERR_ARG, "bad arguments");
    const float r = p->p.update(layer, to_lists(in), truth, n_truth > 0 ? (size_t)n_truth : 0, lr);
    if (recall) *recall = r;
    return MOE_OK;
}

int moe_predictor_save(const moe_predictor *p, const char *path) {
    if (!p || !path) return fail(MOE_ERR_ARG, "null argument");
    std::string err;
    if (!p->p.save(path, err)) return fail(MOE_ERR_IO, "%s", err.c_str());
    return MOE_OK;
}

// a model the cache can score for its layers: E columns, no PCA block
static int check_cache_model(const moe_cache *c, const moe_predictor *p, const char *who) {
    if (p->p.has_pca())
        return fail(MOE_ERR_ARG, "%s: the model has a PCA block over the hidden state, which the cache "
                    "cannot score (the reference disables such a predictor)", who);
    if ((int)p->p.shape.n_expert != c->E)
        return fail(MOE_ERR_ARG, "%s: the model scores %u experts, the cache has %d", who, p->p.shape.n_expert,
                    c->E);
    return MOE_OK;
}

int moe_cache_set_predictor(moe_cache *c, moe_predictor *p, int predict_top, float online_lr,
                            const char *save_path) {
    if (!c) return fail(MOE_ERR_ARG, "null cache");
    if (p && predict_top > 0) {
        const int r = check_cache_model(c, p, "moe_cache_set_predictor");
        if (r != MOE_OK) return r;
        if (!(online_lr >= 0.0f)) return fail(MOE_ERR_ARG, "moe_cache_set_predictor: online_lr %g < 0", online_lr);
        c->cfg.early_issue = 1;        // a predictor issues from the observation (patches/0006:558-562)
    }
    c->pred = p && predict_top > 0 ? p : nullptr;
    c->predict_top = predict_top > 0 ? predict_top : 0;
    c->online_lr = c->pred ? online_lr : 0.0f;
    c->pred_save = c->pred && save_path ? save_path : "";
    for (Layer &ls : c->L) ls.pend_valid = false;
    return MOE_OK;
}

int moe_cache_set_evictor(moe_cache *c, moe_predictor *p) {
    if (!c) return fail(MOE_ERR_ARG, "null cache");
    if (p) {
        const int r = check_cache_model(c, p, "moe_cache_set_evictor");
        if (r != MOE_OK) return r;
    }
    c->evict = p;
    return MOE_OK;
}

int moe_cache_set_spec_probation(moe_cache *c, int on) {
    if (!c) return fail(MOE_ERR_ARG, "null cache");
    c->spec_probation = on != 0;
    return MOE_OK;
}

int moe_cache_predictor_stats(const moe_cache *c, uint64_t *n_updates, double *recall_sum, uint64_t *n_spec) {
    if (!c) return fail(MOE_ERR_ARG, "null cache");
    if (n_updates) *n_updates = c->online_n;
    if (recall_sum) *recall_sum = c->online_recall;
    if (n_spec) *n_spec = c->n_spec;
    return MOE_OK;
}

int moe_cache_frame(moe_cache *c, int layer, int32_t *out) {
    if (!c || !out || layer < 0 || layer >= (int)c->L.size()) return fail(MOE_ERR_ARG, "bad arguments");
    const Layer &ls = c->L[layer];
    for (int s = 0; s < ls.S; ++s) out[s] = -1;
    for (int e = 0; e < ls.E; ++e)
        if (ls.expert_slot[e] >= 0) out[ls.expert_slot[e]] = e;
    return MOE_OK;
}

int moe_cache_table(moe_cache *c, int layer, int32_t *tbl, float *prior) {
    if (!c || layer < 0 || layer >= (int)c->L.size()) return fail(MOE_ERR_ARG, "bad arguments");
    if (tbl) memcpy(tbl, c->h_tbl + (size_t)layer * c->E, (size_t)c->E * 4);
    if (prior) {
        if (c->h_prior) memcpy(prior, c->h_prior + (size_t)layer * c->E, (size_t)c->E * 4);
        else memset(prior, 0, (size_t)c->E * 4);
    }
    return MOE_OK;
}

int moe_cache_stats_get(moe_cache *c, moe_cache_stats *s) {
    if (!c || !s) return fail(MOE_ERR_ARG, "bad arguments");
    memset(s, 0, sizeof *s);
    s->n_steps = c->n_steps;
    s->clock = c->clock;
    for (const Layer &ls : c->L) { s->n_hit += ls.n_hit; s->n_miss += ls.n_miss; }
    s->n_uploads = c->n_uploads;
    s->n_scheduled = c->n_scheduled;
    s->n_copied = c->n_copied;
    s->n_published = c->n_published;
    s->n_admit_ok = c->n_admit_ok;
    s->n_admit_denied = c->n_admit_denied;
    s->n_table_flushes = c->n_table_flushes;
    s->n_staged = c->n_staged;
    s->n_cpu_served = c->n_cpu_served;
    s->sidecar_wait_us = c->sc_wait_us;
    s->sidecar_cpu_us = c->sc_cpu_us;
    s->bytes_uploaded = c->bytes_uploaded;
    s->publication_wait_us = c->wait_us;
    s->host_boundary_us = c->boundary_us;
    s->n_evicted = c->n_evicted;
    s->n_upload_h2d = c->n_up_h2d;
    s->n_upload_d2d = c->n_up_d2d;
    s->upload_h2d_us = c->up_h2d_us;
    s->upload_d2d_us = c->up_d2d_us;
    return MOE_OK;
}

int moe_cache_set_upload_stats(moe_cache *c, int on) {
    if (!c) return fail(MOE_ERR_ARG, "null cache");
    c->up_stats = on != 0 && !c->host_only;
    return MOE_OK;
}

int moe_cache_set_decode_path(moe_cache *c, int split, int graph) {
    if (!c) return fail(MOE_ERR_ARG, "null cache");
    if (split < 0 || split > 3) return fail(MOE_ERR_ARG, "split must be 0, 1, 2 or 3");
    if ((split == 1 || split == 2) && c->sc_den > 0)
        return fail(MOE_ERR_STATE, "CPU-assisted serving runs with one expert launch (split 0 or 3); turn it off first");
    if (graph < 0 || graph > 2) return fail(MOE_ERR_ARG, "graph must be 0, 1 or 2");
    c->split = split;
    c->graph = graph;
    return MOE_OK;
}

static int pl_server_drain(moe_cache *c);

int moe_cache_set_wait_bound(moe_cache *c, double seconds) {
    if (!c) return fail(MOE_ERR_ARG, "null cache");
    if (!(seconds > 0.0) || seconds > 60.0) return fail(MOE_ERR_ARG, "wait bound %g s must be in (0, 60]", seconds);
    if (c->pls) {                       // layers queued by per-layer calls run with the old bound
        const int r = pl_server_drain(c);
        if (r != MOE_OK) return r;
    }
    if (seconds != c->fused_wait_s) drop_graphs(c);     // captured launches carry the bound
    c->fused_wait_s = seconds;
    return MOE_OK;
}

static int sc_buffers(moe_cache *c);
static bool logits_ready(const mp::SidecarPost &p, int E, int n_q8_words, uint32_t seq, int &n_lg, int &n_q8);

int moe_cache_set_sidecar(moe_cache *c, int n_threads, int num, int den) {
    if (!c) return fail(MOE_ERR_ARG, "null cache");
    if (c->host_only) return fail(MOE_ERR_STATE, "host-only cache (device < 0) cannot decode");
    if (c->pls) {                       // layers queued by per-layer calls are served first
        const int r = pl_server_drain(c);
        if (r != MOE_OK) return r;
    }
    if (n_threads <= 0) {
        if (c->sc_den) drop_graphs(c);
        c->sc_den = c->sc_num = 0;
        return MOE_OK;
    }
    if (den < 1 || num < 0 || num > den) return fail(MOE_ERR_ARG, "share %d/%d: need 0 <= num <= den, den >= 1", num, den);
    if (c->split == 1 || c->split == 2)
        return fail(MOE_ERR_STATE, "CPU-assisted serving runs with one expert launch (split 0 or 3)");
    if (c->K > 16 || (c->H / 256) * mp::Q8K_BYTES > mp::SC_Q8X_BYTES) return fail(MOE_ERR_ARG, "shape too large");
    HIPCHK(hipSetDevice(c->cfg.device));
    int r = sc_buffers(c);
    if (r != MOE_OK) return r;
    // the channel is tested before it serves (patches/0009:914-925): 10000
    // bounded round trips of a seeded pattern; a failure leaves GPU-only serving
    if (!c->sc_tested) {
        int bad = 0;
        r = moe_cache_sidecar_selftest(c, 10000, -1, c->sc_timeout_s, &bad);
        if (r != MOE_OK) {
            fprintf(stderr, "moe-cache: CPU-assisted serving DISABLED (channel self-test: %d of 10000 exchanges "
                            "failed)\n", bad);
            c->sc_den = c->sc_num = 0;
            return fail(MOE_ERR_HIP, "CPU-assisted serving disabled: channel self-test failed (%d of 10000)", bad);
        }
        c->sc_tested = true;
    }
    if (c->team && mpc::team_size(c->team) != n_threads) {
        mpc::team_destroy(c->team);
        c->team = nullptr;
    }
    if (!c->team) c->team = mpc::team_create(n_threads);
    c->sc_h.resize((size_t)c->K * c->I);
    c->sc_y.resize((size_t)c->K * c->H);
    c->sc_q8h.resize((size_t)c->K * (c->I / 256) * mp::Q8K_BYTES);
    c->sc_q8x.resize((size_t)(c->H / 256) * mp::Q8K_BYTES);
    c->sc_ids.assign((size_t)c->cfg.n_layers * c->K, -1);
    // the CPU reads the stores from now on: fault their pages in here, not
    // expert by expert in the middle of a token
    for (const Layer &ls : c->L)
        if (ls.store_host) mpc::prefault(c->team, ls.store_host, (size_t)ls.E * ls.expert_bytes);
    c->sc_num = num;
    c->sc_den = den;
    drop_graphs(c);
    return MOE_OK;
}

// the exchange blocks of CPU-assisted serving (mapped, coherent host memory)
static int sc_buffers(moe_cache *c) {
    const size_t NL = c->L.size();
    const unsigned fl = hipHostMallocMapped | hipHostMallocCoherent;
    if (!c->sc_post) {
        if (hipHostMalloc((void **)&c->sc_post, NL * sizeof(mp::SidecarPost), fl) != hipSuccess ||
            hipHostMalloc((void **)&c->sc_resp, NL * sizeof(mp::SidecarResp), fl) != hipSuccess ||
            hipHostMalloc((void **)&c->sc_rows, NL * c->K * c->H * sizeof(float), fl) != hipSuccess)
            return fail(MOE_ERR_NOMEM, "CPU-assisted serving buffers");
        // the sequence number may already exist (streaming allocates it too)
        if (!c->h_seq) {
            if (hipHostMalloc((void **)&c->h_seq, 64, hipHostMallocDefault) != hipSuccess ||
                hipMalloc(&c->d_seq, 64) != hipSuccess)
                return fail(MOE_ERR_NOMEM, "sequence number");
            HIPCHK(hipMemset(c->d_seq, 0, 64));
        }
        memset((void *)c->sc_post, 0, NL * sizeof(mp::SidecarPost));
        memset((void *)c->sc_resp, 0, NL * sizeof(mp::SidecarResp));
        HIPCHK(hipHostGetDevicePointer((void **)&c->sc_post_d, c->sc_post, 0));
        HIPCHK(hipHostGetDevicePointer((void **)&c->sc_resp_d, c->sc_resp, 0));
        HIPCHK(hipHostGetDevicePointer((void **)&c->sc_rows_d, c->sc_rows, 0));
    }
    return MOE_OK;
}

int moe_cache_sidecar_selftest(moe_cache *c, int n_rounds, int withhold_from, double timeout_s, int *n_bad) {
    if (n_bad) *n_bad = 0;
    if (!c || n_rounds < 1 || timeout_s <= 0.0) return fail(MOE_ERR_ARG, "bad arguments");
    if (c->host_only) return fail(MOE_ERR_STATE, "host-only cache has no GPU to exchange with");
    HIPCHK(hipSetDevice(c->cfg.device));
    int r = sc_buffers(c);
    if (r != MOE_OK) return r;
    // layer 0's post, answer and rows; the sequence numbers continue the
    // decode's, so no later token can mistake a test word for its own
    mp::SidecarPost &post = c->sc_post[0];
    mp::SidecarResp &resp = c->sc_resp[0];
    const int E = mp::SC_MAX_E, nq = mp::SC_Q8X_BYTES / 4, H = c->H;
    uint32_t seq0 = c->sc_seq + 1;
    if (seq0 == 0 || seq0 == mp::SC_ABORT || seq0 + (uint32_t)n_rounds < seq0 ||
        seq0 + (uint32_t)n_rounds >= mp::SC_ABORT)
        seq0 = 1;
    c->sc_seq = seq0 + (uint32_t)n_rounds - 1;
    *(volatile uint32_t *)&resp.seq = 0;
    uint32_t *bad_d = nullptr;
    uint32_t bad_h = 0;
    HIPCHK(hipMalloc((void **)&bad_d, 4));
    hipStream_t st = c->host_stream;
    mp::ScSelfTestArgs a{};
    a.post = c->sc_post_d;
    a.resp = c->sc_resp_d;
    a.rows = c->sc_rows_d;
    a.n_rounds = n_rounds;
    a.E = E;
    a.n_q8_words = nq;
    a.H = H;
    a.seq0 = seq0;
    a.timeout_ticks = (uint64_t)(timeout_s * 1e8);
    a.bad = bad_d;
    int host_bad = 0;
    hipError_t e = hipMemsetAsync(bad_d, 0, 4, st);
    if (e == hipSuccess) e = mp::launch_sc_selftest(a, st);
    if (e == hipSuccess) {
        for (int k = 0; k < n_rounds; ++k) {
            if (withhold_from >= 0 && k >= withhold_from) {     // the kernel's own bound ends the rest
                host_bad += n_rounds - k;
                break;
            }
            const uint32_t seq = seq0 + (uint32_t)k;
            const auto t0 = std::chrono::steady_clock::now();
            int n_lg = 0, n_q8 = 0;
            bool late = false;
            unsigned spins = 0;
            while (!logits_ready(post, E, nq, seq, n_lg, n_q8)) {
                _mm_pause();
                if ((++spins & 1023u) == 0 &&
                    std::chrono::duration<double>(std::chrono::steady_clock::now() - t0).count() > timeout_s) {
                    late = true;
                    break;
                }
            }
            if (late) {         // no answer: the kernel's bounded wait ends it
                host_bad += n_rounds - k;
                break;
            }
            std::atomic_thread_fence(std::memory_order_acquire);
            bool wrong = false;
            for (int i = 0; i < E; ++i) wrong |= (uint32_t)post.logit[i] != mp::sc_test_word(seq, i, 0);
            for (int i = 0; i < nq; ++i) wrong |= (uint32_t)post.q8x_words[i] != mp::sc_test_word(seq, i, 1);
            host_bad += wrong;
            for (int i = 0; i < H; ++i) {
                const uint32_t b = mp::sc_test_word(seq, i, 2) & 0x3fffffffu;
                memcpy(&c->sc_rows[i], &b, 4);
            }
            std::atomic_thread_fence(std::memory_order_release);
            *(volatile uint32_t *)&resp.seq = seq;
        }
        e = hipStreamSynchronize(st);
    }
    if (e == hipSuccess) e = hipMemcpy(&bad_h, bad_d, 4, hipMemcpyDeviceToHost);
    hipFree(bad_d);
    *(volatile uint32_t *)&resp.seq = 0;
    if (e != hipSuccess) return fail(MOE_ERR_HIP, "channel self-test: %s", hipGetErrorString(e));
    const int bad = std::max(host_bad, (int)bad_h);
    if (n_bad) *n_bad = bad;
    if (bad) return fail(MOE_ERR_HIP, "channel self-test: %d of %d exchanges failed", bad, n_rounds);
    return MOE_OK;
}

// wait (bounded) for layer l's post, compute the absent experts assigned to
// the CPU, publish their rows, answer
static bool post_ready(const mp::SidecarPost &p, int K, uint32_t seq) {
    for (int k = 0; k < K; ++k)
        if ((uint32_t)(__atomic_load_n(&p.tag[k], __ATOMIC_ACQUIRE) >> 32) != seq) return false;
    return true;
}

// the fused layer's early post: every logit and every word of Q8_K(x).  The
// words already seen valid are not read again (n_lg, n_q8 carry over between
// calls): the device's writes invalidate those lines in the host's caches, so
// each is fetched once, as it arrives, not all again at the end.
static bool logits_ready(const mp::SidecarPost &p, int E, int n_q8_words, uint32_t seq, int &n_lg, int &n_q8) {
    while (n_q8 < n_q8_words && (uint32_t)(__atomic_load_n(&p.q8x_words[n_q8], __ATOMIC_ACQUIRE) >> 32) == seq) ++n_q8;
    while (n_lg < E && (uint32_t)(__atomic_load_n(&p.logit[n_lg], __ATOMIC_ACQUIRE) >> 32) == seq) ++n_lg;
    return n_lg == E && n_q8 == n_q8_words;
}

// by_logits (the fused layer): the host routes the token itself from the
// posted logits, with the published tables' host mirrors, as soon as the
// router rows are done, instead of waiting for the selection's post
static int sidecar_serve(moe_cache *c, int l, uint32_t seq, bool by_logits) {
    const auto t0 = std::chrono::steady_clock::now();
    unsigned spins = 0;
    const mp::SidecarPost &p = c->sc_post[l];
    const int n_q8_words = (int)(c->sc_q8x.size() / 4);
    int n_lg = 0, n_q8 = 0;
    while (by_logits ? !logits_ready(p, c->E, n_q8_words, seq, n_lg, n_q8) : !post_ready(p, c->K, seq)) {
        _mm_pause();
        if ((++spins & 1023u) == 0 &&
            std::chrono::duration<double>(std::chrono::steady_clock::now() - t0).count() > c->sc_timeout_s)
            return fail(MOE_ERR_HIP, "layer %d: no post from the GPU within %.1f s", l, c->sc_timeout_s);
    }
    std::atomic_thread_fence(std::memory_order_acquire);
    const auto t1 = std::chrono::steady_clock::now();
    c->sc_wait_us += std::chrono::duration<double, std::micro>(t1 - t0).count();
    const Layer &ls = c->L[l];
    int32_t *rid = c->sc_ids.data() + (size_t)l * c->K;       // the ids the host served with, checked after the token
    if (by_logits) {
        float lg[mp::SC_MAX_E];
        for (int e = 0; e < c->E; ++e) {
            const uint32_t b = (uint32_t)p.logit[e];
            memcpy(&lg[e], &b, 4);
        }
        mpc::route_topk(lg, c->E, c->d_prior ? c->h_prior + (size_t)l * c->E : nullptr, c->cfg.prior_on_logits != 0,
                        c->K, rid);
    } else {
        for (int k = 0; k < c->K; ++k) rid[k] = (int)(p.tag[k] & 0xffff);
    }
    // the exchange block is memory the GPU reads and writes over PCIe: copy
    // x's Q8_K out of it once, compute into host scratch, publish the rows once
    if (by_logits) {
        uint32_t *q8 = (uint32_t *)c->sc_q8x.data();
        for (int i = 0; i < n_q8_words; ++i) q8[i] = (uint32_t)p.q8x_words[i];
    } else {
        memcpy(c->sc_q8x.data(), p.q8x, c->sc_q8x.size());
    }
    mpc::CpuExpert e[16];
    int kk[16];
    int n = 0, r = 0;
    for (int k = 0; k < c->K; ++k) {
        const int id = rid[k];
        const int slot = by_logits ? c->h_tbl[(size_t)l * c->E + id] : (int)((p.tag[k] >> 16) & 0xffff);
        if (id < 0 || id >= ls.E || (slot >= 0 && slot < ls.S)) continue;  // outside the store, or read from a slot
        if (r++ % c->sc_den < c->sc_num) {
            kk[n] = k;
            e[n] = {ls.store_host + (size_t)id * ls.expert_bytes, c->sc_q8x.data(), c->sc_y.data() + (size_t)n * c->H};
            ++n;
        }
    }
    if (n) c->sc_computing.store(l, std::memory_order_relaxed);
    mpc::experts(c->team, e, n, c->H, c->I, ls.down_type, c->sc_h.data(), c->sc_q8h.data());
    c->sc_computing.store(-1, std::memory_order_relaxed);
    for (int j = 0; j < n; ++j)
        memcpy(c->sc_rows + ((size_t)l * c->K + kk[j]) * c->H, c->sc_y.data() + (size_t)j * c->H, (size_t)c->H * 4);
    c->n_cpu_served += n;
    const double cpu_us = std::chrono::duration<double, std::micro>(std::chrono::steady_clock::now() - t1).count();
    c->sc_cpu_us += cpu_us;
    if (c->sc_log.size() < 3 * 65536) {
        c->sc_log.push_back((float)std::chrono::duration<double, std::micro>(t1 - t0).count());
        c->sc_log.push_back((float)cpu_us);
        c->sc_log.push_back((float)n);
    }
    std::atomic_thread_fence(std::memory_order_release);
    *(volatile uint32_t *)&c->sc_resp[l].seq = seq;
    return MOE_OK;
}

// ---- the per-layer server (see PlServer) ------------------------------------
static void pl_server_main(moe_cache *c) {
    PlServer &sv = *c->pls;
    for (;;) {
        PlServer::Job j;
        bool failed;
        {
            std::unique_lock<std::mutex> lk(sv.m);
            sv.cv.wait(lk, [&] { return sv.quit || !sv.q.empty(); });
            if (sv.q.empty()) return;
            j = sv.q.front();
            sv.q.pop_front();
            failed = sv.err != MOE_OK || sv.quit;
        }
        const int r = failed ? MOE_OK : sidecar_serve(c, j.layer, j.seq, j.fused);
        // after a failure no later layer is served: end each one's join at once
        if (failed || r != MOE_OK) *(volatile uint32_t *)&c->sc_resp[j.layer].seq = mp::SC_ABORT;
        std::lock_guard<std::mutex> lk(sv.m);
        if (r != MOE_OK && sv.err == MOE_OK) {
            sv.err = r;
            sv.msg = g_err;             // (the message was this thread's)
        }
        if (--sv.busy == 0) sv.cv_idle.notify_all();
    }
}

static void pl_server_push(moe_cache *c, int layer, uint32_t seq, bool fused) {
    if (!c->pls) {
        c->pls.reset(new PlServer);
        c->pls->th = std::thread(pl_server_main, c);
    }
    PlServer &sv = *c->pls;
    std::lock_guard<std::mutex> lk(sv.m);
    sv.q.push_back({layer, seq, fused});
    ++sv.busy;
    sv.cv.notify_one();
}

// Wait until every queued layer is served (each serve is bounded by its wait
// for the GPU's post, sc_timeout_s); the first failure, with its message.
static int pl_server_drain(moe_cache *c) {
    if (!c->pls) return MOE_OK;
    PlServer &sv = *c->pls;
    std::unique_lock<std::mutex> lk(sv.m);
    const double limit = (c->sc_timeout_s + 1.0) * std::max(1, sv.busy);
    if (!sv.cv_idle.wait_for(lk, std::chrono::duration<double>(limit), [&] { return sv.busy == 0; }))
        return fail(MOE_ERR_HIP, "the host's share of the queued layers was not served within %.1f s", limit);
    if (sv.err == MOE_OK) return MOE_OK;
    const int e = sv.err;
    const std::string msg = sv.msg;
    sv.err = MOE_OK;
    sv.msg.clear();
    return fail(e, "%s", msg.c_str());
}

static void pl_server_stop(moe_cache *c) {
    if (!c->pls) return;
    pl_server_drain(c);
    {
        std::lock_guard<std::mutex> lk(c->pls->m);
        c->pls->quit = true;
    }
    c->pls->cv.notify_all();
    if (c->pls->th.joinable()) c->pls->th.join();
    c->pls.reset();
}

int moe_cache_set_sidecar_batch(moe_cache *c, int num, int den) {
    if (!c) return fail(MOE_ERR_ARG, "null cache");
    if (num == 0 && den == 0) {
        c->sb_num = c->sb_den = 0;
        return MOE_OK;
    }
    if (den < 1 || num < 0 || num > den) return fail(MOE_ERR_ARG, "share %d/%d: need 0 <= num <= den, den >= 1", num, den);
    c->sb_num = num;
    c->sb_den = den;
    return MOE_OK;
}

int moe_cache_sidecar_log(moe_cache *c, float *out, int max_rows) {
    if (!c) return -1;
    const int rows = (int)std::min<size_t>(c->sc_log.size() / 3, (size_t)std::max(0, max_rows));
    if (out) memcpy(out, c->sc_log.data(), (size_t)rows * 3 * sizeof(float));
    c->sc_log.clear();
    return rows;
}

int moe_cache_set_staging(moe_cache *c, int on) {
    if (!c) return fail(MOE_ERR_ARG, "null cache");
    if (c->staging != (on != 0)) drop_graphs(c);      // the captured launches carry the staging pointers
    c->staging = on != 0;
    return MOE_OK;
}

int moe_cache_set_timing(moe_cache *c, int on) {
    if (!c) return fail(MOE_ERR_ARG, "null cache");
    if (c->host_only && on) return fail(MOE_ERR_STATE, "host-only cache has no kernels to time");
    c->timing = on != 0;
    c->kt = moe_kernel_times{};
    return MOE_OK;
}

int moe_cache_kernel_times(moe_cache *c, moe_kernel_times *out) {
    if (!c || !out) return fail(MOE_ERR_ARG, "bad arguments");
    *out = c->kt;
    return MOE_OK;
}

int moe_cache_sync(moe_cache *c) {
    if (!c) return fail(MOE_ERR_ARG, "null cache");
    if (c->host_only) return MOE_OK;
    HIPCHK(hipStreamSynchronize(c->up_stream));
    HIPCHK(hipStreamSynchronize(c->stg_stream));
    return MOE_OK;
}

// fused: split is 0 and streaming is off; the router, selection, experts and
// combine run as one launch.  seq_val: 0, the token's sequence number is in
// d_seq (moe_decode_token); else the call's own number, passed by value
static int decode_layer_impl(moe_cache *c, int layer, const float *x, const float *bias, float *out,
                             int32_t *ids_dev, float *w_dev, hipStream_t st, hipEvent_t *ev, bool stage,
                             bool sidecar, bool fused, uint32_t seq_val) {
    if (!c || !x || !out || layer < 0 || layer >= (int)c->L.size()) return fail(MOE_ERR_ARG, "bad arguments");
    if (c->host_only) return fail(MOE_ERR_STATE, "host-only cache (device < 0) cannot decode");
    const Layer &ls = c->L[layer];
    if (!ls.router || !ls.store_dev) return fail(MOE_ERR_STATE, "layer %d: router or host store missing", layer);
    int32_t *ids = ids_dev ? ids_dev : c->d_ids + (size_t)layer * c->K;
    float *w = w_dev ? w_dev : c->d_w + (size_t)layer * c->K;
    int32_t *slots = c->d_slots + (size_t)layer * c->K;
    moe_route_desc rd{};
    rd.W = ls.router; rd.x = x; rd.bias = bias;
    rd.prior = c->d_prior ? c->d_prior + (size_t)layer * c->E : nullptr;
    rd.table = c->d_tbl + (size_t)layer * c->E;
    rd.dummy = ls.S;
    rd.prior_on_logits = c->cfg.prior_on_logits;
    rd.E = c->E; rd.H = c->H; rd.K = c->K; rd.n_tok = 1;
    rd.ids = ids; rd.w = w; rd.slots = slots; rd.probs = nullptr; rd.q8x = c->d_q8x;
    rd.workspace = c->route_ws;
    // ev (timing mode), 12 per layer, stamped by the dispatches themselves:
    // [0,1] route_logits [2,3] route_select [4,5] gate/up (resident or all)
    // [6,7] down (resident or all) [8,9] gate/up absent [10,11] down absent
    // just-in-time streaming: this layer's router launch also scores the next
    // layers' routers and posts the record the mover thread works from
    mp::RouteLaunch look{};
    const Streamer *stm = c->st && c->st->live ? c->st : nullptr;
    if (stm) {
        const auto &tg = stm->targets[(size_t)layer];
        for (int t = 0; t < 2; ++t) {
            if (tg[t] < 0) continue;
            const int i = look.an++;
            look.aW[i] = c->L[(size_t)tg[t]].router;
            look.ar[i] = stm->ratio + ((size_t)layer * 2 + t) * c->H;
            look.atbl[i] = c->d_tbl + (size_t)tg[t] * c->E;
            look.adummy[i] = c->L[(size_t)tg[t]].S;
            look.atarget[i] = tg[t];
        }
        look.ak = stm->top_k;
        look.alayer = layer;
        look.alog = stm->alog;
        look.apost = stm->post_d + layer;
        look.fresh = stm->fresh + layer;
    }
    moe_experts_desc ed{};
    ed.ids = ids; ed.slots = slots; ed.w = w;
    ed.slot_pool = ls.pool; ed.slot_bytes = ls.slot_bytes; ed.n_slots = ls.S;
    ed.host_store = ls.store_dev; ed.expert_bytes = ls.expert_bytes; ed.n_experts = c->E;
    ed.q8x = c->d_q8x; ed.out = out; ed.accumulate = 0;
    ed.H = c->H; ed.I = c->I; ed.K = c->K; ed.down_type = ls.down_type;
    ed.workspace = c->exp_ws;
    mp::ExpertArgs a{};
    a.ids = ed.ids; a.slots = ed.slots; a.w = ed.w;
    a.slot_pool = ed.slot_pool; a.slot_bytes = ed.slot_bytes; a.n_slots = ed.n_slots;
    a.host_store = ed.host_store; a.expert_bytes = ed.expert_bytes; a.n_experts = ed.n_experts;
    a.q8x = ed.q8x; a.out = ed.out;
    a.H = ed.H; a.I = ed.I; a.K = ed.K; a.down_type = ed.down_type;
    a.shared = ls.shared; a.n_shared = ls.shared ? 1 : 0;
    if (stage && c->stage) {
        a.stage = c->stage + (size_t)layer * c->K * c->stage_stride;
        a.stage_stride = c->stage_stride;
    }
    if (sidecar) {
        a.cpu_num = c->sc_num;
        a.cpu_den = c->sc_den;
    }
    if (stm) a.fresh = stm->fresh + layer;
    uint8_t *ws = (uint8_t *)ed.workspace;
    a.h = (float *)ws;
    size_t o = align_up((size_t)(ed.K + 1) * ed.I * 4, 256);
    a.q8h = ws + o;
    o += align_up((size_t)(ed.K + 1) * (ed.I / 256) * mp::Q8K_BYTES, 256);
    a.counter = (uint32_t *)(ws + o);
    auto E_ = [ev](int i) -> hipEvent_t { return ev ? ev[i] : nullptr; };
    a.accumulate = 0;
    // split: the first down launch keeps every expert's rows, the second
    // reads the ones it did not compute and writes sum_k w_k y_k in k order
    // (the order of one launch over all experts)
    a.ypart = c->ypart;
    mp::ExpertArgs ah = a;
    ah.join = 1;
    if (fused) {
        mp::FusedArgs f{};
        mp::RouteLaunch &rl = f.r;
        rl.W = rd.W; rl.x = rd.x; rl.bias = rd.bias; rl.prior = rd.prior; rl.table = rd.table; rl.dummy = rd.dummy;
        rl.prior_on_logits = rd.prior_on_logits;
        rl.E = rd.E; rl.H = rd.H; rl.K = rd.K; rl.n_tok = 1;
        rl.ids = ids; rl.w = w; rl.slots = slots;
        rl.post = sidecar ? c->sc_post_d + layer : nullptr;
        rl.seq = seq_val ? nullptr : c->d_seq;
        rl.seq_val = seq_val;
        f.x = a;
        f.x.ypart = sidecar ? c->ypart : nullptr;       // the join kernel combines with the host's rows
        f.xlog = c->fx + (size_t)layer * c->fx_words;
        f.rec = f.xlog + (size_t)mp::FUSED_LOG_COPIES * 256;
        f.hx = f.rec + (size_t)mp::FUSED_COPIES * mp::FUSED_REC;
        f.yx = f.hx + (size_t)(c->K + 1) * c->I;
        f.err = (uint32_t *)(c->d_ids + c->L.size() * (size_t)c->K);
        f.wait_ticks = (uint64_t)(c->fused_wait_s * 1e8);
        if (c->pub_on && !sidecar) {
            f.pub = c->h_pub_d;
            f.pub_ctr = c->d_pub_ctr + layer;
            f.pub_layer = layer;
            f.pub_L = (int)c->L.size();
            f.pub_done = layer + 1 == (int)c->L.size();
        }
        HIPCHK(mp::launch_fused(f, st, E_(0), E_(1)));
    } else {
        const int r = run_route(&rd, st, ev, sidecar ? c->sc_post_d + layer : nullptr, seq_val ? nullptr : c->d_seq,
                                stm ? &look : nullptr, seq_val);
        if (r != MOE_OK) return r;
    }
    if (c->split == 0 || c->split == 3) {
        if (!fused) {
            HIPCHK(mp::launch_gateup(a, 0, st, E_(4), E_(5)));
            HIPCHK(mp::launch_down(a, 0, st, E_(6), E_(7)));
        }
        if (sidecar) {
            mp::JoinArgs j{};
            j.ids = a.ids; j.slots = a.slots; j.w = a.w;
            j.slot_pool = a.slot_pool; j.n_slots = a.n_slots;
            j.host_store = a.host_store; j.n_experts = a.n_experts;
            j.K = a.K; j.H = a.H; j.n_shared = a.n_shared; j.cpu_num = a.cpu_num; j.cpu_den = a.cpu_den;
            j.ypart = c->ypart;
            j.hrows = c->sc_rows_d + (size_t)layer * c->K * c->H;
            j.resp = c->sc_resp_d + layer;
            j.seq = seq_val ? nullptr : c->d_seq;
            j.seq_val = seq_val;
            j.timeout_ticks = (uint64_t)(c->sc_timeout_s * 1e8);     // 100 MHz wall clock
            j.out = a.out;
            HIPCHK(mp::launch_join(j, st));
        }
        return MOE_OK;
    }
    if (c->split == 2) {
        HIPCHK(mp::launch_gateup(a, 1, st, E_(4), E_(5)));
        HIPCHK(mp::launch_down(a, 1, st, E_(6), E_(7)));
        HIPCHK(mp::launch_gateup(ah, 2, st, E_(8), E_(9)));
        HIPCHK(mp::launch_down(ah, 2, st, E_(10), E_(11)));
        return MOE_OK;
    }
    // fork: resident experts on st, absent ones on the host stream; the host
    // stream's down launch adds onto what the resident one wrote; join.
    hipStream_t hs = c->host_stream;
    HIPCHK(hipEventRecord(c->ev_route, st));
    HIPCHK(hipStreamWaitEvent(hs, c->ev_route, 0));
    HIPCHK(mp::launch_gateup(ah, 2, hs, E_(8), E_(9)));
    HIPCHK(mp::launch_gateup(a, 1, st, E_(4), E_(5)));
    HIPCHK(mp::launch_down(a, 1, st, E_(6), E_(7)));
    HIPCHK(hipEventRecord(c->ev_hbm, st));
    HIPCHK(hipStreamWaitEvent(hs, c->ev_hbm, 0));
    HIPCHK(mp::launch_down(ah, 2, hs, E_(10), E_(11)));
    HIPCHK(hipEventRecord(c->ev_host, hs));
    HIPCHK(hipStreamWaitEvent(st, c->ev_host, 0));
    return MOE_OK;
}

// a fresh sequence number for a token or a layer call (never 0 nor SC_ABORT)
static uint32_t next_seq(moe_cache *c) {
    uint32_t seq = ++c->sc_seq;
    if (seq == 0 || seq == mp::SC_ABORT) seq = c->sc_seq = 1;
    return seq;
}

// timing mode: 12 events per layer, stamped by the launches' dispatches
static int ensure_tev(moe_cache *c) {
    const size_t n = c->L.size() * 12;
    if (!c->timing || c->tev.size() == n) return MOE_OK;
    for (hipEvent_t e : c->tev) hipEventDestroy(e);
    c->tev.assign(n, nullptr);
    for (auto &e : c->tev) HIPCHK(hipEventCreate(&e));
    return MOE_OK;
}

// the staging area, [L][K] experts of the largest slot size, at first use
static int ensure_stage(moe_cache *c) {
    if (!c->staging || c->stage) return MOE_OK;
    size_t sb = 0;
    for (const Layer &ls : c->L) sb = std::max(sb, (size_t)ls.slot_bytes);
    const size_t n = c->L.size() * (size_t)c->K * sb;
    if (hipMalloc(&c->stage, n) != hipSuccess) {
        c->stage = nullptr;
        return fail(MOE_ERR_NOMEM, "staging area of %zu bytes", n);
    }
    c->stage_stride = sb;
    drop_graphs(c);             // captured launches carry the staging pointers
    return MOE_OK;
}

// layer l's routed experts the kernels read from the pinned store (and so
// staged), from the token's ids and the slots the GPU read (h_ids, h_slots):
// absent experts the host served were not read by the kernels
static void set_staged(moe_cache *c, int l, bool sc, bool stage) {
    Layer &ls = c->L[l];
    int r = 0;
    for (int k = 0; k < c->K; ++k) {
        const int id = c->h_ids[(size_t)l * c->K + k], gs = c->h_slots[(size_t)l * c->K + k];
        const bool absent = id >= 0 && id < ls.E && !(gs >= 0 && gs < ls.S);
        const bool cpu = absent && sc && r % c->sc_den < c->sc_num;
        r += absent;
        ls.staged[k] = stage && absent && !cpu ? id : -1;
    }
}

// timing mode: layer l's kernel times (its events) and the expert bytes its
// launches read by source, from h_ids / h_slots when have_ids
static int account_times(moe_cache *c, int l, bool fused, bool sc, bool have_ids) {
    const uint64_t gu_b = 2ull * c->I * (c->H / 256) * mp::Q4K_BYTES;
    float t[6] = {0, 0, 0, 0, 0, 0};
    hipEvent_t *e = c->tev.data() + (size_t)l * 12;
    const Layer &ls = c->L[l];
    if (fused) {            // [0,1] the fused layer
        HIPCHK(hipEventElapsedTime(&t[0], e[0], e[1]));
        c->kt.layer_ms += t[0];
        c->kt.layer_hbm_bytes += (uint64_t)c->E * c->H * 4;       // the router rows
    } else {
        for (int i = 0; i < 6; ++i) {
            if ((c->split == 0 || c->split == 3) && i >= 4) break;   // no separate absent-expert launches
            HIPCHK(hipEventElapsedTime(&t[i], e[2 * i], e[2 * i + 1]));
        }
        c->kt.route_ms += t[0] + t[1];
        c->kt.gateup_hbm_ms += t[2];
        c->kt.down_hbm_ms += t[3];
        c->kt.gateup_host_ms += t[4];
        c->kt.down_host_ms += t[5];
    }
    c->kt.n_layers++;
    if (!have_ids) return MOE_OK;
    int r_abs = 0;          // rank among the absent experts: the host's share is not read by the GPU
    for (int k = 0; k < c->K; ++k) {
        const int gs = c->h_slots[(size_t)l * c->K + k];
        const int id = c->h_ids[(size_t)l * c->K + k];
        const bool res = gs >= 0 && gs < ls.S;
        const bool absent = !res && id >= 0 && id < ls.E;
        const bool cpu = absent && sc && r_abs % c->sc_den < c->sc_num;
        r_abs += absent;
        if (cpu) continue;
        (res ? c->kt.gateup_hbm_bytes : c->kt.gateup_host_bytes) += gu_b;
        (res ? c->kt.down_hbm_bytes : c->kt.down_host_bytes) += ls.expert_bytes - gu_b;
        if (fused) (res ? c->kt.layer_hbm_bytes : c->kt.layer_host_bytes) += ls.expert_bytes;
    }
    if (ls.shared) {
        c->kt.gateup_hbm_bytes += gu_b;
        c->kt.down_hbm_bytes += ls.expert_bytes - gu_b;
        if (fused) c->kt.layer_hbm_bytes += ls.expert_bytes;
    }
    return MOE_OK;
}

// ---- one layer per call ---------------------------------------------------------
static int pl_sync(moe_cache *c) {
    if (c->pl_synced) return MOE_OK;
    const int r = pl_server_drain(c);          // the host's share of every queued layer
    for (hipStream_t s : c->pl_streams) HIPCHK(hipStreamSynchronize(s));
    if (r != MOE_OK) return r;
    c->pl_synced = true;
    return MOE_OK;
}

static void pl_clear(moe_cache *c) {
    std::fill(c->pl_flags.begin(), c->pl_flags.end(), (uint8_t)0);
    c->pl_streams.clear();
    c->pl_synced = false;
    if (c->pl_hot && c->team) mpc::team_hot(c->team, false);
    c->pl_hot = false;
}

// observe of a layer decoded by moe_decode_layer: its ids and the slots the
// GPU read (the published table, which changes only at the step) become the
// token's record; with CPU-assisted serving the host's routing must equal
// the ids observed; with staging, the experts the kernels read from the
// store are staged for the uploads observe (early issue) or the step start
static int pl_observe(moe_cache *c, int l, const int32_t *ids) {
    const int r = pl_sync(c);
    if (r != MOE_OK) return r;
    const uint8_t f = c->pl_flags[(size_t)l];
    const Layer &ls = c->L[(size_t)l];
    for (int k = 0; k < c->K; ++k) {
        const int id = ids[k];
        c->h_ids[(size_t)l * c->K + k] = id;
        c->h_slots[(size_t)l * c->K + k] = id >= 0 && id < ls.E ? c->h_tbl[(size_t)l * c->E + id] : ls.S;
    }
    const bool once = !(f & PL_AGAIN);
    if ((f & PL_SIDECAR) && once && memcmp(c->sc_ids.data() + (size_t)l * c->K, ids, (size_t)c->K * 4) != 0)
        return fail(MOE_ERR_STATE, "layer %d: the host's routing differs from the ids observed", l);
    set_staged(c, l, (f & PL_SIDECAR) != 0, (f & PL_STAGE) && once);
    c->pl_flags[(size_t)l] |= PL_OBSERVED;
    return MOE_OK;
}

// the step after per-layer calls: their kernels have finished; a bounded
// wait that ran out (fused late word, a join's error word) fails the token
static int pl_step(moe_cache *c) {
    int r = pl_sync(c);
    uint32_t late_seq = 0;
    const size_t NL = c->L.size();
    if (r == MOE_OK && hipMemcpy(&late_seq, c->d_ids + NL * c->K, 4, hipMemcpyDeviceToHost) != hipSuccess)
        r = fail(MOE_ERR_HIP, "late-wait word read back");
    bool late = false, late_join = false, staged = false;
    for (size_t l = 0; l < NL && r == MOE_OK; ++l) {
        const uint8_t f = c->pl_flags[l];
        if (!(f & PL_DECODED)) continue;
        late |= (f & PL_FUSED) && late_seq == c->pl_seq[l];
        if (f & PL_SIDECAR) {
            late_join |= c->sc_resp[l].err != 0;
            c->sc_resp[l].err = 0;
        }
        staged |= (f & PL_STAGE) && (f & PL_OBSERVED) && !(f & PL_AGAIN);
        if (c->timing) r = account_times(c, (int)l, (f & PL_FUSED) != 0, (f & PL_SIDECAR) != 0, (f & PL_OBSERVED) != 0);
    }
    pl_clear(c);
    if (r != MOE_OK) return r;
    if (late) return fail(MOE_ERR_HIP, "a fused layer's workgroup gave up waiting for another (%.1f s)", c->fused_wait_s);
    if (late_join) return fail(MOE_ERR_HIP, "a join kernel gave up waiting for the host (%.1f s)", c->sc_timeout_s);
    c->stage_valid = staged;
    r = cache_step(c);
    c->stage_valid = false;
    if (c->stg_pending) HIPCHK(hipEventRecord(c->ev_stg, c->stg_stream));
    return r;
}

// One decode layer at batch 1 on its own: the reference's per-layer graph op
// (the cached chain, and with the sidecar its post and join, P9:659-705).
// The fused launch by default (split 0); split 3's launches otherwise.  With
// CPU-assisted serving the calling thread serves the host's share of the
// layer's absent experts before it returns, and the GPU's join waits for it.
int moe_decode_layer(moe_cache *c, int layer, const float *x, const float *bias, float *out, int32_t *ids_dev,
                     float *w_dev, void *stream) {
    if (!c || !x || !out || layer < 0 || layer >= (int)c->L.size()) return fail(MOE_ERR_ARG, "bad arguments");
    if (c->host_only) return fail(MOE_ERR_STATE, "host-only cache (device < 0) cannot decode");
    if (c->st && c->st->live) return fail(MOE_ERR_STATE, "just-in-time streaming decodes whole tokens (moe_decode_token)");
    const hipStream_t st = (hipStream_t)stream;
    const size_t NL = c->L.size();
    int r = ensure_stage(c);
    if (r == MOE_OK) r = ensure_tev(c);
    if (r != MOE_OK) return r;
    if (c->pl_flags.size() != NL) {
        c->pl_flags.assign(NL, 0);
        c->pl_seq.assign(NL, 0);
    }
    if (c->pl_streams.empty())          // the first call since the step: nothing is staged yet
        for (Layer &ls : c->L) std::fill(ls.staged.begin(), ls.staged.end(), -1);
    std::fill(c->L[(size_t)layer].staged.begin(), c->L[(size_t)layer].staged.end(), -1);
    // uploads copied from the staging area so far must be done before this
    // layer's kernels overwrite it
    if (c->stg_pending) {
        HIPCHK(hipEventRecord(c->ev_stg, c->stg_stream));
        HIPCHK(hipStreamWaitEvent(st, c->ev_stg, 0));
        c->stg_pending = false;
    }
    const bool stage = c->staging && c->stage;
    const bool sc = c->sc_den > 0;
    const bool fused = c->split == 0;
    // a failed token may have left SC_ABORT in this layer's answer word; every
    // kernel of that token has finished (the failure synchronised its stream)
    if (sc && c->sc_resp[layer].seq == mp::SC_ABORT) {
        *(volatile uint32_t *)&c->sc_resp[layer].seq = 0;
        *(volatile uint32_t *)&c->sc_resp[layer].err = 0;
    }
    // an earlier layer's serving failed: report it before launching more
    if (c->pls) {
        bool failed;
        {
            std::lock_guard<std::mutex> lk(c->pls->m);
            failed = c->pls->err != MOE_OK;
        }
        if (failed) {
            r = pl_server_drain(c);
            for (hipStream_t s : c->pl_streams) hipStreamSynchronize(s);
            return r;
        }
    }
    const uint32_t seq = next_seq(c);
    r = decode_layer_impl(c, layer, x, bias, out, ids_dev, w_dev, st,
                          c->timing ? c->tev.data() + (size_t)layer * 12 : nullptr, stage, sc, fused, seq);
    if (r != MOE_OK) {
        hipStreamSynchronize(st);
        return r;
    }
    if (sc) {                           // the host's share: served by the server thread, in call order
        if (!c->pl_hot) {
            mpc::team_hot(c->team, true);
            c->pl_hot = true;
        }
        pl_server_push(c, layer, seq, fused);
    }
    uint8_t &f = c->pl_flags[(size_t)layer];
    f = (uint8_t)((f & PL_DECODED ? PL_AGAIN : 0) | PL_DECODED | (fused ? PL_FUSED : 0) | (sc ? PL_SIDECAR : 0) |
                  (stage ? PL_STAGE : 0));
    c->pl_seq[(size_t)layer] = seq;
    if (std::find(c->pl_streams.begin(), c->pl_streams.end(), st) == c->pl_streams.end()) c->pl_streams.push_back(st);
    c->pl_synced = false;
    return MOE_OK;
}

// tokens of at most this many layers launch directly in graph mode (see below)
constexpr int DIRECT_MAX_LAYERS = 8;

// every word the fused launches publish (h_pub) carries this token's number:
// bounded spin (a legitimate token takes microseconds; past the bound the
// caller copies back and synchronises, which also reports a failed launch),
// then the ids, slots and late word go where the copy back would put them
static bool wait_published(moe_cache *c, int NL, uint32_t seq) {
    const size_t n = (size_t)NL * c->K + 1;
    const auto t0 = std::chrono::steady_clock::now();
    const auto bound = std::chrono::duration<double>(4 * c->fused_wait_s + 0.5);
    size_t i = 0;                       // words before i carry seq
    for (uint64_t spin = 0; i < n; ++spin) {
        while (i < n && (uint32_t)(__atomic_load_n(c->h_pub + i, __ATOMIC_ACQUIRE) >> 32) == seq) ++i;
        if (i == n) break;
        if ((spin & 255) == 0 && std::chrono::steady_clock::now() - t0 > bound) return false;
#if defined(__x86_64__)
        __builtin_ia32_pause();
#endif
    }
    for (size_t j = 0; j + 1 < n; ++j) {
        const uint64_t w = c->h_pub[j];
        c->h_ids[j] = (int32_t)(w & 0xffffu);
        c->h_slots[j] = (int32_t)((w >> 16) & 0xffffu);
    }
    c->h_ids[n - 1] = (int32_t)(uint32_t)c->h_pub[n - 1];     // the late word
    return true;
}

int moe_decode_token(moe_cache *c, const float *x, const float *bias, float *out, int32_t *ids_host, void *stream) {
    if (!c || !x || !out) return fail(MOE_ERR_ARG, "bad arguments");
    if (c->host_only) return fail(MOE_ERR_STATE, "host-only cache (device < 0) cannot decode");
    hipStream_t st = (hipStream_t)stream;
    const int NL = (int)c->L.size();
    int er = ensure_tev(c);
    if (er == MOE_OK) er = ensure_stage(c);
    if (er != MOE_OK) return er;
    // layers decoded one by one and not stepped: their kernels finish first,
    // and this token's record replaces theirs
    if (!c->pl_streams.empty()) {
        er = pl_sync(c);
        pl_clear(c);
        if (er != MOE_OK) return er;
    }
    const bool stage = c->staging && c->stage;
    // the last step's device-to-device uploads read the staging area this
    // token's kernels are about to overwrite
    if (c->stg_pending) {
        HIPCHK(hipStreamWaitEvent(st, c->ev_stg, 0));
        c->stg_pending = false;
    }
    // CPU-assisted serving: this token's sequence number, for the posts and
    // the answers of every layer
    const bool sc = c->sc_den > 0;
    Streamer *stm = c->st && c->st->live ? c->st : nullptr;
    // (the fused layers' exchange words are tagged with it too).  The copy
    // reads h_seq when the stream reaches it; the previous token synchronised
    // the stream before returning, so no copy of an older number is pending.
    const uint32_t seq = next_seq(c);
    // A captured graph's launch costs ~30 us of latency here (ROCm 7 on
    // MI355X) against ~11 us for a kernel launch, and launching ~15 us layers
    // one by one measured faster at every layer count (1 layer: 26 against
    // 35 us a step; 48 layers within 1 %).  The graph frees the host sooner,
    // which CPU-assisted serving and streaming need (the host serves a layer
    // while the GPU runs the next), and it costs less host time for many
    // layers.  So a token of at most DIRECT_MAX_LAYERS layers without them
    // launches its layers directly, with the sequence number by value and the
    // caller's x and out: no copies.  (graph 2 keeps the graph for any token.)
    const bool use_graph = c->graph && !c->timing && (c->graph == 2 || NL > DIRECT_MAX_LAYERS || sc || stm);
    if (use_graph) {
        *c->h_seq = seq;
        HIPCHK(hipMemcpyAsync(c->d_seq, c->h_seq, 4, hipMemcpyHostToDevice, st));
    }
    const bool fused = c->split == 0 && !stm;
    // An earlier token that failed may have left SC_ABORT in the answers; a
    // join of this token must wait for this token's answer, not end on that.
    // Nothing of this token runs yet, so plain stores suffice.
    if (sc)
        for (int l = 0; l < NL; ++l) {
            *(volatile uint32_t *)&c->sc_resp[l].seq = 0;
            *(volatile uint32_t *)&c->sc_resp[l].err = 0;
        }
    // streaming: the mover serves this token's lookahead records
    bool mover_on = false;
    if (stm && !stm->failed) {
        stm->seq = seq;
        stm->stop.store(false, std::memory_order_relaxed);
        {
            std::lock_guard<std::mutex> lk(stm->m);
            stm->gen++;
        }
        stm->cv.notify_one();
        mover_on = true;
    }
    // the mover is told the token's GPU work is over and hands the
    // bookkeeping back (it waits for the copies it queued); bounded
    auto mover_drain = [&]() -> int {
        if (!mover_on) return MOE_OK;
        mover_on = false;
        stm->stop.store(true, std::memory_order_release);
        std::unique_lock<std::mutex> lk(stm->m);
        if (!stm->cv_done.wait_for(lk, std::chrono::seconds(2), [&] { return stm->gen_done == stm->gen; }))
            return fail(MOE_ERR_HIP, "stream mover did not finish within 2 s");
        return MOE_OK;
    };
    auto abort_joins = [&] {        // end every join kernel still waiting
        if (sc)
            for (int l = 0; l < NL; ++l) *(volatile uint32_t *)&c->sc_resp[l].seq = mp::SC_ABORT;
    };
    // Launched directly, GPU only, the fused layers publish the token's ids,
    // slots and late word into h_ids themselves and then a done word: the host
    // spins on that word instead of a copy back and a stream synchronisation
    // (a kernel's completion reaches a waiting host ~4.7 us later than a word
    // it writes; the copy costs 1.7 us more).  The wait is bounded; past it
    // (a workgroup gave up, no done word) the copy and the synchronisation
    // run as on the other paths.
    const bool publish = !use_graph && fused && !sc && !stm && !c->timing;
    c->pub_on = publish;
    // per-kernel HIP-event timing needs eager launches: hipEventElapsedTime
    // does not accept events recorded as nodes of a graph
    if (!use_graph) {
        for (int l = 0; l < NL; ++l) {
            const int r = decode_layer_impl(c, l, x + (size_t)l * c->H, bias ? bias + (size_t)l * c->E : nullptr,
                                            out + (size_t)l * c->H, nullptr, nullptr, st,
                                            c->timing ? c->tev.data() + (size_t)l * 12 : nullptr, stage, sc, fused,
                                            seq);
            if (r != MOE_OK) {
                c->pub_on = false;
                abort_joins();
                hipStreamSynchronize(st);
                mover_drain();
                return r;
            }
        }
        c->pub_on = false;

    } else {
        const int key = bias ? 1 : 0;        const int mode = c->split + (fused ? 10 : 0);
        if (!c->gx[key] || c->g_mode[key] != mode) {
            if (c->gx[key]) { hipGraphExecDestroy(c->gx[key]); c->gx[key] = nullptr; }
            if (c->g[key]) { hipGraphDestroy(c->g[key]); c->g[key] = nullptr; }
            HIPCHK(hipStreamBeginCapture(c->cap_stream, hipStreamCaptureModeThreadLocal));
            int r = MOE_OK;
            for (int l = 0; l < NL && r == MOE_OK; ++l)
                r = decode_layer_impl(c, l, c->x_buf + (size_t)l * c->H, key ? c->bias_buf + (size_t)l * c->E : nullptr,
                                      c->out_buf + (size_t)l * c->H, nullptr, nullptr, c->cap_stream, nullptr, stage,
                                      sc, fused, 0);

            hipGraph_t g = nullptr;
            const hipError_t ec = hipStreamEndCapture(c->cap_stream, &g);
            if (r != MOE_OK || ec != hipSuccess) {
                if (g) hipGraphDestroy(g);
                mover_drain();
                return r != MOE_OK ? r : fail(MOE_ERR_HIP, "hipStreamEndCapture: %s", hipGetErrorString(ec));
            }
            c->g[key] = g;
            HIPCHK(hipGraphInstantiate(&c->gx[key], g, nullptr, nullptr, 0));
            c->g_mode[key] = mode;
        }
        HIPCHK(hipMemcpyAsync(c->x_buf, x, (size_t)NL * c->H * 4, hipMemcpyDeviceToDevice, st));
        if (bias) HIPCHK(hipMemcpyAsync(c->bias_buf, bias, (size_t)NL * c->E * 4, hipMemcpyDeviceToDevice, st));
        HIPCHK(hipGraphLaunch(c->gx[key], st));
        HIPCHK(hipMemcpyAsync(out, c->out_buf, (size_t)NL * c->H * 4, hipMemcpyDeviceToDevice, st));
    }
    int serve_err = MOE_OK;
    if (sc) {               // serve the layers as the GPU reaches them
        mpc::team_hot(c->team, true);
        for (int l = 0; l < NL && serve_err == MOE_OK; ++l) serve_err = sidecar_serve(c, l, seq, fused);
        mpc::team_hot(c->team, false);
        if (serve_err != MOE_OK) abort_joins();
    }
    // the routed ids and, after them, the fused layers' late-wait word
    hipError_t sync_err = hipSuccess;
    // (the token's staged copies, issued by observe or the step below, are the
    // only readers of what the launches wrote that run on another stream)
    struct DecClose {
        moe_cache *c;
        ~DecClose() { c->dec_open = nullptr; }
    } dec_close{c};
    if (publish && wait_published(c, NL, seq)) {
        c->dec_open = st;
    } else {
        HIPCHK(hipMemcpyAsync(c->h_ids, c->d_ids, (2 * (size_t)NL * c->K + 64) * 4, hipMemcpyDeviceToHost, st));
        sync_err = hipStreamSynchronize(st);
    }
    const auto t_sync = std::chrono::steady_clock::now();
    const int drain_err = mover_drain();
    if (sync_err != hipSuccess) return fail(MOE_ERR_HIP, "decode: %s", hipGetErrorString(sync_err));
    if (drain_err != MOE_OK) return drain_err;
    if (fused && (uint32_t)c->h_ids[(size_t)NL * c->K] == seq)
        return fail(MOE_ERR_HIP, "a fused layer's workgroup gave up waiting for another (%.1f s)", c->fused_wait_s);
    if (stm && stm->failed) return fail(MOE_ERR_HIP, "streaming stopped on a copy queue error");
    if (sc) {
        bool late = false;
        for (int l = 0; l < NL; ++l) {
            late |= c->sc_resp[l].err != 0;
            c->sc_resp[l].err = 0;
        }
        if (serve_err != MOE_OK) return serve_err;
        if (late) return fail(MOE_ERR_HIP, "a join kernel gave up waiting for the host (%.1f s)", c->sc_timeout_s);
        // the host's routing must have been the GPU's (it chose which experts it computed)
        if (memcmp(c->sc_ids.data(), c->h_ids, (size_t)NL * c->K * 4) != 0)
            return fail(MOE_ERR_STATE, "the host's routing of a layer differs from the GPU's");
    }
    if (c->timing)
        for (int l = 0; l < NL; ++l) {
            const int tr = account_times(c, l, fused, sc, true);
            if (tr != MOE_OK) return tr;
        }
    // which routed experts the kernels read from the store (and staged): the
    // slots the GPU read say which were absent
    if (stage)
        for (int l = 0; l < NL; ++l) set_staged(c, l, sc, true);
    // (early issue starts uploads inside observe: staged copies apply there too)
    c->stage_valid = stage;
    int r = MOE_OK;
    for (int l = 0; l < NL && r == MOE_OK; ++l)
        r = cache_observe(c, l, c->h_ids + (size_t)l * c->K, c->K, 1, stm ? c->h_slots + (size_t)l * c->K : nullptr);
    if (r == MOE_OK) {
        if (ids_host) memcpy(ids_host, c->h_ids, (size_t)NL * c->K * 4);
        r = cache_step(c);
    }
    c->stage_valid = false;
    if (c->stg_pending) HIPCHK(hipEventRecord(c->ev_stg, c->stg_stream));
    c->boundary_us += std::chrono::duration<double, std::micro>(std::chrono::steady_clock::now() - t_sync).count();
    return r;
}

// ---- batched path -------------------------------------------------------------
int moe_dispatch(const int32_t *ids, int n_tok, int K, int E, int32_t *counts, int32_t *offsets, int32_t *perm,
                 void *stream) {
    if (!ids || !counts || !offsets || !perm) return fail(MOE_ERR_ARG, "moe_dispatch: null argument");
    if (E < 1 || E > mp::MAX_E) return fail(MOE_ERR_ARG, "moe_dispatch: n_experts %d must be 1..%d", E, mp::MAX_E);
    if (n_tok < 0 || K < 1 || (int64_t)n_tok * K > 65535)
        return fail(MOE_ERR_ARG, "moe_dispatch: n_tok * K must be <= 65535 (n_tok %d, K %d)", n_tok, K);
    HIPCHK(mp::launch_dispatch(ids, n_tok * K, E, counts, offsets, perm, (hipStream_t)stream));
    return MOE_OK;
}

int moe_quant_rows(const void *src, int src_type, int n_rows, int n, uint16_t *q16, float *d, uint16_t *bsum16,
                   void *stream) {
    if (!src || !q16 || !d || !bsum16) return fail(MOE_ERR_ARG, "moe_quant_rows: null argument");
    if (src_type != MOE_DTYPE_F32 && src_type != MOE_DTYPE_BF16)
        return fail(MOE_ERR_ARG, "moe_quant_rows: src_type %d unsupported", src_type);
    if (n_rows < 0 || n <= 0 || n % 256) return fail(MOE_ERR_ARG, "moe_quant_rows: n %d must be a multiple of 256", n);
    if (((uintptr_t)src | (uintptr_t)q16) % 16) return fail(MOE_ERR_ARG, "moe_quant_rows: src and q16 must be 16-byte aligned");
    HIPCHK(mp::launch_quant_rows(src, src_type == MOE_DTYPE_BF16, n_rows, n, q16, d, bsum16, (hipStream_t)stream));
    return MOE_OK;
}

size_t moe_grouped_workspace_bytes(int n_tok, int K, int H, int I) {
    if (n_tok < 0 || K < 1 || H < 256 || I < 256) return 0;
    return grouped_ws(n_tok, K, H, I).total;
}

int moe_combine(const float *pair_rows, int n_tok, int K, int H, float *out, int accumulate, void *stream) {
    if (!pair_rows || !out) return fail(MOE_ERR_ARG, "moe_combine: null argument");
    if (n_tok < 0 || K < 1 || H <= 0 || H % 4) return fail(MOE_ERR_ARG, "moe_combine: bad shape");
    if (((uintptr_t)pair_rows | (uintptr_t)out) % 16) return fail(MOE_ERR_ARG, "moe_combine: 16-byte alignment");
    HIPCHK(mp::launch_combine(pair_rows, n_tok, K, H, out, accumulate, (hipStream_t)stream));
    return MOE_OK;
}

// shape and pointer checks shared by both grouped entry points
static int grouped_check(const moe_grouped_desc *d) {
    if (!d || !d->offsets || !d->perm || !d->w || !d->x || !d->out)
        return fail(MOE_ERR_ARG, "moe_grouped_experts: null argument");
    if (d->H != 2048) return fail(MOE_ERR_ARG, "hidden size %d unsupported (the kernels are built for 2048)", d->H);
    if (d->I % 256 || d->I < 256 || d->I > 768) return fail(MOE_ERR_ARG, "intermediate %d must be 256, 512 or 768", d->I);
    if (d->E < 1 || d->E > mp::MAX_E) return fail(MOE_ERR_ARG, "n_experts %d must be 1..%d", d->E, mp::MAX_E);
    if (d->K < 1 || d->n_tok < 1 || (int64_t)d->n_tok * d->K > 65535)
        return fail(MOE_ERR_ARG, "n_tok %d x K %d out of range", d->n_tok, d->K);
    if (d->x_type != MOE_DTYPE_F32 && d->x_type != MOE_DTYPE_BF16)
        return fail(MOE_ERR_ARG, "x_type %d unsupported", d->x_type);
    if (d->down_type != MOE_TYPE_Q4K && d->down_type != MOE_TYPE_Q6K)
        return fail(MOE_ERR_ARG, "down type %d unsupported", d->down_type);
    if (!d->store && !d->slot_pool) return fail(MOE_ERR_ARG, "no weights");
    if (d->expert_bytes != mp::expert_bytes(d->H, d->I, d->down_type))
        return fail(MOE_ERR_ARG, "expert_bytes %llu does not match the shape", (unsigned long long)d->expert_bytes);
    if (d->slot_pool && (d->slot_bytes < d->expert_bytes || d->slot_bytes % 16))
        return fail(MOE_ERR_ARG, "slot_bytes must be >= expert_bytes and a multiple of 16");
    if (((uintptr_t)d->slot_pool | (uintptr_t)d->store | (uintptr_t)d->x | (uintptr_t)d->out |
         (uintptr_t)d->workspace | (uintptr_t)d->pair_out | (uintptr_t)d->h_out) % 16)
        return fail(MOE_ERR_ARG, "weights, activations and outputs must be 16-byte aligned");
    int r = check_weight_ptrs("moe_grouped_experts", d->slot_pool, d->store);
    if (r != MOE_OK) return r;
    if (d->shared && (r = check_weight_ptrs("moe_grouped_experts", d->shared, nullptr)) != MOE_OK) return r;
    if ((uintptr_t)d->shared % 16) return fail(MOE_ERR_ARG, "shared expert must be 16-byte aligned");
    return MOE_OK;
}

// the grouped expert chain over a checked descriptor, with ws as its workspace.
// CPU-assisted batched decode runs it in two parts: the expert products with
// the host's experts masked out (host_mask, device view of [E] flags), then,
// once the host's rows are written, the combine taking flagged pairs' rows
// from hrows (hflag [P]) and the shared expert.
constexpr int GR_EXPERTS = 1, GR_COMBINE = 2;
static int grouped_run(const moe_grouped_desc *d, uint8_t *ws, hipStream_t st, int parts = GR_EXPERTS | GR_COMBINE,
                       const uint8_t *host_mask = nullptr, const float *hrows = nullptr,
                       const uint8_t *hflag = nullptr) {
    const GroupedWs w = grouped_ws(d->n_tok, d->K, d->H, d->I);
    mp::GroupedArgs a{};
    a.offsets = d->offsets; a.perm = d->perm; a.w = d->w;
    a.table = d->table; a.slot_pool = d->slot_pool; a.slot_bytes = d->slot_bytes; a.n_slots = d->n_slots;
    a.store = d->store; a.expert_bytes = d->expert_bytes; a.n_store = d->n_store;
    a.E = d->E; a.K = d->K; a.H = d->H; a.I = d->I; a.down_type = d->down_type;
    a.xa = (const uint16_t *)(ws + w.xa); a.xdx = (const float *)(ws + w.xdx); a.xbs = (const uint16_t *)(ws + w.xbs);
    a.y2 = (float *)(ws + w.h);
    a.ha = (const uint16_t *)(ws + w.ha); a.hdx = (const float *)(ws + w.hdx); a.hbs = (const uint16_t *)(ws + w.hbs);
    a.ypair = d->pair_out ? d->pair_out : (float *)(ws + w.ypair);
    a.host_mask = host_mask;
    const int P = d->n_tok * d->K;
    a.P = P;
    hipEvent_t ev[4] = {};
    const bool timed = d->kernel_ms != nullptr;
    if (timed)
        for (auto &e : ev) HIPCHK(hipEventCreate(&e));
    auto run = [&]() -> int {
        if (parts & GR_EXPERTS) {
            HIPCHK(mp::launch_quant_rows(d->x, d->x_type == MOE_DTYPE_BF16, d->n_tok, d->H, (uint16_t *)a.xa,
                                         (float *)a.xdx, (uint16_t *)a.xbs, st));
            HIPCHK(mp::launch_gateup_grouped(a, st, ev[0], ev[1]));
            HIPCHK(mp::launch_swiglu_quant(a.y2, P, d->I, d->h_out, (uint16_t *)a.ha, (float *)a.hdx,
                                           (uint16_t *)a.hbs, st));
            HIPCHK(mp::launch_down_grouped(a, st, ev[2], ev[3]));
        }
        if (!(parts & GR_COMBINE)) return MOE_OK;
        if (hflag)
            HIPCHK(mp::launch_combine_host(a.ypair, hrows, hflag, d->n_tok, d->K, d->H, d->out, d->accumulate, st));
        else
            HIPCHK(mp::launch_combine(a.ypair, d->n_tok, d->K, d->H, d->out, d->accumulate, st));
        if (d->shared) {
            // the shared expert as a one-expert dispatch of every token, added after the routed sum
            mp::GroupedArgs sa = a;
            sa.host_mask = nullptr;
            sa.offsets = (const int32_t *)(ws + w.sh_offs);
            sa.perm = (const int32_t *)(ws + w.sh_perm);
            sa.w = (const float *)(ws + w.sh_ones);
            sa.table = nullptr; sa.slot_pool = nullptr; sa.n_slots = 0;
            sa.store = d->shared; sa.n_store = 1; sa.E = 1; sa.K = 1; sa.P = d->n_tok;
            HIPCHK(mp::launch_iota(d->n_tok, (int32_t *)sa.offsets, (int32_t *)sa.perm, (float *)sa.w, st));
            HIPCHK(mp::launch_gateup_grouped(sa, st, nullptr, nullptr));
            HIPCHK(mp::launch_swiglu_quant(sa.y2, d->n_tok, d->I, nullptr, (uint16_t *)sa.ha, (float *)sa.hdx,
                                           (uint16_t *)sa.hbs, st));
            HIPCHK(mp::launch_down_grouped(sa, st, nullptr, nullptr));
            HIPCHK(mp::launch_combine(sa.ypair, d->n_tok, 1, d->H, d->out, 1, st));
        }
        return MOE_OK;
    };
    int rc = run();
    if (timed) {
        if (rc == MOE_OK && (parts & GR_EXPERTS) && hipEventSynchronize(ev[3]) == hipSuccess) {
            float ms = 0.0f;
            hipEventElapsedTime(&ms, ev[0], ev[1]);
            d->kernel_ms[0] = ms;
            hipEventElapsedTime(&ms, ev[2], ev[3]);
            d->kernel_ms[1] = ms;
        }
        for (auto e : ev) hipEventDestroy(e);
    }
    return rc;
}

int moe_grouped_experts(const moe_grouped_desc *d, void *stream) {
    int r = grouped_check(d);
    if (r != MOE_OK) return r;
    if (!d->workspace) return fail(MOE_ERR_ARG, "moe_grouped_experts: null workspace");
    return grouped_run(d, (uint8_t *)d->workspace, (hipStream_t)stream);
}

int moe_grouped_experts_static(const moe_grouped_desc *d, void *stream) {
    int r = grouped_check(d);
    if (r != MOE_OK) return r;
    if (d->workspace) return fail(MOE_ERR_ARG, "moe_grouped_experts_static: workspace must be NULL (it uses its own)");
    if (d->kernel_ms) return fail(MOE_ERR_ARG, "moe_grouped_experts_static: kernel_ms must be NULL (timing creates events)");
    const size_t need = grouped_ws(d->n_tok, d->K, d->H, d->I).total;
    static_assert(mp::STATIC_SCRATCH_BYTES == MOE_GROUPED_STATIC_SCRATCH_BYTES, "header and library disagree");
    if (need > mp::STATIC_SCRATCH_BYTES)
        return fail(MOE_ERR_ARG, "moe_grouped_experts_static: n_tok %d x K %d at I %d needs %zu bytes of scratch, "
                    "more than the %zu it holds", d->n_tok, d->K, d->I, need, (size_t)mp::STATIC_SCRATCH_BYTES);
    void *ws = nullptr;
    const hipError_t e = mp::static_scratch(&ws);
    if (e != hipSuccess) return fail(MOE_ERR_HIP, "static scratch: %s", hipGetErrorString(e));
    return grouped_run(d, (uint8_t *)ws, (hipStream_t)stream);
}

// ---- batched decode through the cache ------------------------------------------
static int batch_buffers(moe_cache *c, int n_tok) {
    if (n_tok <= c->b_cap) return MOE_OK;
    for (void *p : {(void *)c->b_ids, (void *)c->b_slots, (void *)c->b_counts, (void *)c->b_offs, (void *)c->b_perm,
                    (void *)c->b_w, (void *)c->b_q8x, c->b_route_ws, c->b_ws})
        hipFree(p);
    if (c->bh_ids) hipHostFree(c->bh_ids);
    c->b_ids = c->b_slots = c->b_counts = c->b_offs = c->b_perm = c->bh_ids = nullptr;
    c->b_w = nullptr;
    c->b_q8x = nullptr;
    c->b_route_ws = c->b_ws = nullptr;
    c->b_cap = 0;
    const size_t NL = c->L.size(), TK = (size_t)n_tok * c->K;
    const size_t rws = route_ws_bytes(c->E, n_tok), gws = grouped_ws(n_tok, c->K, c->H, c->I).total;
    bool ok = hipMalloc(&c->b_ids, NL * TK * 4) == hipSuccess && hipMalloc(&c->b_slots, TK * 4) == hipSuccess &&
              hipMalloc(&c->b_w, TK * 4) == hipSuccess && hipMalloc(&c->b_counts, (size_t)c->E * 4) == hipSuccess &&
              hipMalloc(&c->b_offs, ((size_t)c->E + 1) * 4) == hipSuccess && hipMalloc(&c->b_perm, TK * 4) == hipSuccess &&
              hipMalloc(&c->b_q8x, (size_t)n_tok * (c->H / 256) * mp::Q8K_BYTES) == hipSuccess &&
              hipMalloc(&c->b_route_ws, rws) == hipSuccess && hipMalloc(&c->b_ws, gws) == hipSuccess &&
              hipHostMalloc((void **)&c->bh_ids, NL * TK * 4, hipHostMallocDefault) == hipSuccess;
    if (!ok || hipMemset(c->b_route_ws, 0, rws) != hipSuccess) return fail(MOE_ERR_NOMEM, "batch buffers for %d tokens", n_tok);
    c->b_cap = n_tok;
    return MOE_OK;
}

// exchange buffers of CPU-assisted batched decode for up to n_tok tokens
static int batch_sidecar_buffers(moe_cache *c, int n_tok) {
    if (n_tok <= c->bs_cap) return MOE_OK;
    for (void *p : {(void *)c->bs_w, (void *)c->bs_q8, (void *)c->bs_mask, (void *)c->bs_flag, (void *)c->bs_rows})
        if (p) hipHostFree(p);
    c->bs_w = nullptr;
    c->bs_q8 = c->bs_mask = c->bs_flag = nullptr;
    c->bs_rows = nullptr;
    c->bs_cap = 0;
    const size_t TK = (size_t)n_tok * c->K;
    const unsigned fl = hipHostMallocMapped | hipHostMallocCoherent;
    bool ok = hipHostMalloc((void **)&c->bs_w, TK * 4, hipHostMallocDefault) == hipSuccess &&
              hipHostMalloc((void **)&c->bs_q8, (size_t)n_tok * (c->H / 256) * mp::Q8K_BYTES, hipHostMallocDefault) ==
                  hipSuccess &&
              hipHostMalloc((void **)&c->bs_mask, 2 * (size_t)c->E, fl) == hipSuccess &&
              hipHostMalloc((void **)&c->bs_flag, 2 * TK, fl) == hipSuccess &&
              hipHostMalloc((void **)&c->bs_rows, 2 * TK * c->H * 4, fl) == hipSuccess;
    if (!ok) return fail(MOE_ERR_NOMEM, "CPU-assisted batch buffers for %d tokens", n_tok);
    HIPCHK(hipHostGetDevicePointer((void **)&c->bs_mask_d, c->bs_mask, 0));
    HIPCHK(hipHostGetDevicePointer((void **)&c->bs_flag_d, c->bs_flag, 0));
    HIPCHK(hipHostGetDevicePointer((void **)&c->bs_rows_d, c->bs_rows, 0));
    if (!c->bs_ev) HIPCHK(hipEventCreateWithFlags(&c->bs_ev, hipEventDisableTiming));
    c->bs_cap = n_tok;
    return MOE_OK;
}

// CPU-assisted serving of one layer of a batch, after its routing was copied
// back: the host takes the absent experts whose rank r among the layer's
// absent experts (ascending id) has r % den < num, masks them out of the
// grouped products it then enqueues, computes their pairs from the pinned
// store while the GPU runs the rest, and writes each pair's weighted row
// (w * y, the kernels' one multiplication) for the combine.
static int batch_sidecar_layer(moe_cache *c, int l, int n_tok, const moe_grouped_desc *gd, hipStream_t st) {
    const Layer &ls = c->L[l];
    const int TK = n_tok * c->K, par = l & 1;
    const auto t0 = std::chrono::steady_clock::now();
    HIPCHK(hipEventSynchronize(c->bs_ev));
    const auto t1 = std::chrono::steady_clock::now();
    c->sc_wait_us += std::chrono::duration<double, std::micro>(t1 - t0).count();
    uint8_t *mask = c->bs_mask + (size_t)par * c->E, *flag = c->bs_flag + (size_t)par * TK;
    float *rows = c->bs_rows + (size_t)par * TK * c->H;
    const int32_t *ids = c->bh_ids + (size_t)l * TK;
    std::vector<uint8_t> absent((size_t)c->E, 0);
    for (int i = 0; i < TK; ++i) {
        const int id = ids[i];
        if (id < 0 || id >= ls.E) continue;
        const int slot = c->h_tbl[(size_t)l * c->E + id];
        if (!(slot >= 0 && slot < ls.S)) absent[id] = 1;
    }
    const int num = c->sb_den ? c->sb_num : c->sc_num, den = c->sb_den ? c->sb_den : c->sc_den;
    for (int e = 0, r = 0; e < c->E; ++e) {
        mask[e] = absent[e] && r % den < num;
        r += absent[e];
    }
    // the host's pairs grouped by expert (ascending id, pairs in order): each
    // expert's rows are read from memory once for all of its tokens
    std::vector<int> first((size_t)c->E + 1, 0);
    for (int i = 0; i < TK; ++i) {
        const int id = ids[i];
        flag[i] = id >= 0 && id < ls.E && mask[id];
        if (flag[i]) ++first[(size_t)id + 1];
    }
    for (int e = 0; e < c->E; ++e) first[(size_t)e + 1] += first[e];
    const int n = first[c->E];
    std::vector<int> pair((size_t)n), fill(first.begin(), first.end() - 1);
    for (int i = 0; i < TK; ++i)
        if (flag[i]) pair[(size_t)fill[ids[i]]++] = i;
    std::vector<mpc::CpuGroup> grp;
    for (int e = 0; e < c->E; ++e)
        if (first[(size_t)e + 1] > first[e])
            grp.push_back({ls.store_host + (size_t)e * ls.expert_bytes, first[e], first[(size_t)e + 1] - first[e]});
    const size_t q8row = (size_t)(c->H / 256) * mp::Q8K_BYTES;
    if (c->bs_y.size() < (size_t)TK * c->H) {
        c->bs_y.resize((size_t)TK * c->H);
        c->bs_h.resize((size_t)TK * c->I);
        c->bs_q8h.resize((size_t)TK * (c->I / 256) * mp::Q8K_BYTES);
    }
    std::vector<const uint8_t *> q8p((size_t)n);
    std::vector<float *> yp((size_t)n);
    for (int j = 0; j < n; ++j) {
        q8p[(size_t)j] = c->bs_q8 + (size_t)(pair[(size_t)j] / c->K) * q8row;
        yp[(size_t)j] = c->bs_y.data() + (size_t)j * c->H;
    }
    std::atomic_thread_fence(std::memory_order_release);
    int r = grouped_run(gd, (uint8_t *)c->b_ws, st, GR_EXPERTS, c->bs_mask_d + (size_t)par * c->E);
    if (r != MOE_OK) return r;
    if (n) {
        c->sc_computing.store(l, std::memory_order_relaxed);
        mpc::experts_grouped(c->team, grp.data(), (int)grp.size(), q8p.data(), yp.data(), c->H, c->I, ls.down_type,
                             c->bs_h.data(), c->bs_q8h.data());
        c->sc_computing.store(-1, std::memory_order_relaxed);
        for (int j = 0; j < n; ++j) {
            const float w = c->bs_w[pair[j]];
            const float *y = c->bs_y.data() + (size_t)j * c->H;
            float *o = rows + (size_t)pair[j] * c->H;
            for (int h = 0; h < c->H; ++h) o[h] = w * y[h];
        }
    }
    c->n_cpu_served += n;
    c->sc_cpu_us += std::chrono::duration<double, std::micro>(std::chrono::steady_clock::now() - t1).count();
    std::atomic_thread_fence(std::memory_order_release);
    return grouped_run(gd, (uint8_t *)c->b_ws, st, GR_COMBINE, nullptr, c->bs_rows_d + (size_t)par * TK * c->H,
                       c->bs_flag_d + (size_t)par * TK);
}

int moe_decode_batch(moe_cache *c, const float *x, const float *bias, float *out, int n_tok, int32_t *ids_host,
                     void *stream) {
    if (!c || !x || !out) return fail(MOE_ERR_ARG, "bad arguments");
    if (c->host_only) return fail(MOE_ERR_STATE, "host-only cache (device < 0) cannot decode");
    if (n_tok < 1 || n_tok > 4096) return fail(MOE_ERR_ARG, "n_tok %d out of range 1..4096", n_tok);
    if (((uintptr_t)x | (uintptr_t)out) % 16) return fail(MOE_ERR_ARG, "x and out must be 16-byte aligned");
    HIPCHK(hipSetDevice(c->cfg.device));
    int r = batch_buffers(c, n_tok);
    if (r != MOE_OK) return r;
    const hipStream_t st = (hipStream_t)stream;
    const int NL = (int)c->L.size(), TK = n_tok * c->K;
    // the host's share applies to decode-sized batches; a prefill-sized batch
    // would serialise every layer on the CPU and pin 2 n_tok K H floats
    const int sh_num = c->sb_den ? c->sb_num : c->sc_num, sh_den = c->sb_den ? c->sb_den : c->sc_den;
    const bool sc = c->sc_den > 0 && sh_num > 0 && n_tok <= MOE_BATCH_HOST_MAX_TOKENS;
    if (c->pls && (r = pl_server_drain(c)) != MOE_OK) return r;     // the team is the server's until then
    if (sc && (r = batch_sidecar_buffers(c, n_tok)) != MOE_OK) return r;
    float gms[2] = {0.0f, 0.0f};
    if (sc) mpc::team_hot(c->team, true);
    struct Cold {
        moe_cache *c;
        bool on;
        ~Cold() { if (on) mpc::team_hot(c->team, false); }
    } cold{c, sc};
    // (the last step published only finished copies: its tables are safe to read)
    for (int l = 0; l < NL; ++l) {
        const Layer &ls = c->L[l];
        if (!ls.router || !ls.store_dev) return fail(MOE_ERR_STATE, "layer %d: router or host store missing", l);
        const float *xl = x + (size_t)l * n_tok * c->H;
        moe_route_desc rd{};
        rd.W = ls.router; rd.x = xl; rd.bias = bias ? bias + (size_t)l * n_tok * c->E : nullptr;
        // the cache prior biases single-token selection only (patches/0007:114)
        rd.prior = c->d_prior && n_tok == 1 ? c->d_prior + (size_t)l * c->E : nullptr;
        rd.table = c->d_tbl + (size_t)l * c->E;
        rd.dummy = ls.S;
        rd.prior_on_logits = c->cfg.prior_on_logits;
        rd.E = c->E; rd.H = c->H; rd.K = c->K; rd.n_tok = n_tok;
        rd.ids = c->b_ids + (size_t)l * TK; rd.w = c->b_w; rd.slots = c->b_slots; rd.q8x = c->b_q8x;
        rd.workspace = c->b_route_ws;
        if ((r = run_route(&rd, st)) != MOE_OK) return r;
        if (sc) {                       // the routing back to the host for its share
            HIPCHK(hipMemcpyAsync(c->bh_ids + (size_t)l * TK, rd.ids, (size_t)TK * 4, hipMemcpyDeviceToHost, st));
            HIPCHK(hipMemcpyAsync(c->bs_w, c->b_w, (size_t)TK * 4, hipMemcpyDeviceToHost, st));
            HIPCHK(hipMemcpyAsync(c->bs_q8, c->b_q8x, (size_t)n_tok * (c->H / 256) * mp::Q8K_BYTES,
                                  hipMemcpyDeviceToHost, st));
            HIPCHK(hipEventRecord(c->bs_ev, st));
        }
        HIPCHK(mp::launch_dispatch(rd.ids, TK, c->E, c->b_counts, c->b_offs, c->b_perm, st));
        moe_grouped_desc gd{};
        gd.offsets = c->b_offs; gd.perm = c->b_perm; gd.w = c->b_w;
        gd.x = xl; gd.x_type = MOE_DTYPE_F32;
        gd.n_tok = n_tok; gd.K = c->K; gd.E = c->E; gd.H = c->H; gd.I = c->I; gd.down_type = ls.down_type;
        gd.table = c->d_tbl + (size_t)l * c->E;
        gd.slot_pool = ls.pool; gd.slot_bytes = ls.slot_bytes; gd.n_slots = ls.S;
        gd.store = ls.store_dev; gd.expert_bytes = ls.expert_bytes; gd.n_store = c->E;
        gd.out = out + (size_t)l * n_tok * c->H; gd.accumulate = 0;
        gd.workspace = c->b_ws; gd.shared = ls.shared;
        gd.kernel_ms = c->timing ? gms : nullptr;
        if (!sc) {
            if ((r = moe_grouped_experts(&gd, stream)) != MOE_OK) return r;
        } else {
            if ((r = grouped_check(&gd)) != MOE_OK) return r;
            if (!ls.store_host) return fail(MOE_ERR_STATE, "layer %d: CPU-assisted serving needs the host store", l);
            if ((r = batch_sidecar_layer(c, l, n_tok, &gd, st)) != MOE_OK) return r;
        }
        if (c->timing) {
            c->kt.grouped_gateup_ms += gms[0];
            c->kt.grouped_down_ms += gms[1];
            c->kt.grouped_launches++;
        }
    }
    HIPCHK(hipMemcpyAsync(c->bh_ids, c->b_ids, (size_t)NL * TK * 4, hipMemcpyDeviceToHost, st));
    HIPCHK(hipStreamSynchronize(st));
    if (c->timing)          // the weights the grouped launches read: each GPU expert's once, by source
        for (int l = 0; l < NL; ++l) {
            const Layer &ls = c->L[l];
            const int32_t *ids = c->bh_ids + (size_t)l * TK;
            std::vector<uint8_t> used((size_t)c->E, 0);
            for (int i = 0; i < TK; ++i)
                if (ids[i] >= 0 && ids[i] < ls.E) used[(size_t)ids[i]] = 1;
            const uint64_t gu_b = 2ull * c->I * (c->H / 256) * mp::Q4K_BYTES, dn_b = ls.expert_bytes - gu_b;
            std::vector<uint8_t> host((size_t)c->E, 0);
            for (int e = 0, rk = 0; e < c->E; ++e) {        // the host's experts: batch_sidecar_layer's rule
                const int slot = c->h_tbl[(size_t)l * c->E + e];
                const bool absent = used[(size_t)e] && !(slot >= 0 && slot < ls.S);
                host[(size_t)e] = sc && absent && rk % sh_den < sh_num;
                rk += absent;
                if (!used[(size_t)e] || host[(size_t)e]) continue;
                const bool res = slot >= 0 && slot < ls.S;
                (res ? c->kt.grouped_gateup_hbm_bytes : c->kt.grouped_gateup_host_bytes) += gu_b;
                (res ? c->kt.grouped_down_hbm_bytes : c->kt.grouped_down_host_bytes) += dn_b;
            }
            for (int i = 0; i < TK; ++i) c->kt.grouped_pairs += ids[i] >= 0 && ids[i] < ls.E && !host[(size_t)ids[i]];
        }
    for (int l = 0; l < NL; ++l) {
        if ((r = cache_observe(c, l, c->bh_ids + (size_t)l * TK, c->K, n_tok)) != MOE_OK) return r;
    }
    if (ids_host) memcpy(ids_host, c->bh_ids, (size_t)NL * TK * 4);
    return cache_step(c);
}

// ---- slab pool --------------------------------------------------------------
int moe_pool_create(int n_layers, int capacity, size_t bytes_per_expert, int device, moe_pool **out) {
    if (!out || n_layers <= 0 || capacity <= 0 || bytes_per_expert == 0) return fail(MOE_ERR_ARG, "bad arguments");
    *out = nullptr;
    moe_pool *p = new moe_pool();
    p->n_layers = n_layers;
    p->capacity = capacity;
    p->bytes = align_up(bytes_per_expert, 256);
    p->device = device;
    auto bail = [&](int code) {
        if (p->base) hipFree(p->base);
        for (hipEvent_t e : p->ev) if (e) hipEventDestroy(e);
        if (p->stream) hipStreamDestroy(p->stream);
        delete p;
        return code;
    };
    if (hipSetDevice(device) != hipSuccess) return bail(fail(MOE_ERR_HIP, "hipSetDevice"));
    if (hipMalloc(&p->base, p->bytes * (size_t)n_layers * capacity) != hipSuccess)
        return bail(fail(MOE_ERR_NOMEM, "pool of %zu bytes", p->bytes * (size_t)n_layers * capacity));
    if (hipStreamCreateWithFlags(&p->stream, hipStreamNonBlocking) != hipSuccess)
        return bail(fail(MOE_ERR_HIP, "stream"));
    p->ev.assign((size_t)n_layers * capacity, nullptr);
    p->armed.assign((size_t)n_layers * capacity, 0);
    for (auto &e : p->ev)
        if (hipEventCreateWithFlags(&e, hipEventDisableTiming) != hipSuccess) return bail(fail(MOE_ERR_HIP, "events"));
    *out = p;
    return MOE_OK;
}

int moe_pool_destroy(moe_pool *p) {
    if (!p) return MOE_OK;
    hipStreamSynchronize(p->stream);
    for (hipEvent_t e : p->ev) hipEventDestroy(e);
    hipStreamDestroy(p->stream);
    hipFree(p->base);
    delete p;
    return MOE_OK;
}

int moe_pool_copy(moe_pool *p, int layer, int slot, const void *src_host, size_t bytes) {
    if (!p || layer < 0 || layer >= p->n_layers || slot < 0 || slot >= p->capacity || !src_host || bytes > p->bytes)
        return fail(MOE_ERR_ARG, "bad arguments");
    const size_t i = (size_t)layer * p->capacity + slot;
    HIPCHK(hipMemcpyAsync(p->base + i * p->bytes, src_host, bytes, hipMemcpyHostToDevice, p->stream));
    HIPCHK(hipEventRecord(p->ev[i], p->stream));
    p->armed[i] = 1;
    return MOE_OK;
}

int moe_pool_ready(moe_pool *p, int layer, int slot) {
    if (!p || layer < 0 || layer >= p->n_layers || slot < 0 || slot >= p->capacity)
        return fail(MOE_ERR_ARG, "bad arguments");
    const size_t i = (size_t)layer * p->capacity + slot;
    if (!p->armed[i]) return 1;
    const hipError_t q = hipEventQuery(p->ev[i]);
    if (q == hipSuccess) return 1;
    if (q == hipErrorNotReady) return 0;
    return fail(MOE_ERR_HIP, "hipEventQuery: %s", hipGetErrorString(q));
}

int moe_pool_sync(moe_pool *p) {
    if (!p) return fail(MOE_ERR_ARG, "null pool");
    HIPCHK(hipStreamSynchronize(p->stream));
    return MOE_OK;
}

void *moe_pool_slot_ptr(moe_pool *p, int layer, int slot) {
    if (!p || layer < 0 || layer >= p->n_layers || slot < 0 || slot >= p->capacity) return nullptr;
    return p->base + ((size_t)layer * p->capacity + slot) * p->bytes;
}

}  // extern "C"
