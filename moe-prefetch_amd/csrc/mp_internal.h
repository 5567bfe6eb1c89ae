// mp_internal.h -- kernel argument blocks and launchers shared by the kernels
// (mp_kernels.hip) and the host runtime (mp_runtime.cpp).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace mp {

// CPU-assisted serving of absent experts: per-layer exchange blocks in
// mapped, fine-grained host memory.  The GPU posts the Q8_K of x and the
// routed ids, each id tagged with the token's sequence number; the host
// computes the experts assigned to it, writes their rows and answers with
// the sequence number (or SC_ABORT).
constexpr int SC_Q8X_BYTES = 8 * 292;          // Q8_K of x at H = 2048
// One word per routed expert k: (token sequence number << 32) | (slot << 16) |
// id, where slot is the one the GPU read (n_slots = absent).  Each word is one
// aligned 8-byte store (one write on PCIe, read by the host in one 8-byte
// load), so the host takes the layer once every word of it carries the token's
// number: no word has to land before another.  q8x (the Q8_K of x) is
// written, and waited for, by an earlier kernel of the layer.
constexpr int SC_MAX_E = 256;
struct alignas(256) SidecarPost {
    uint64_t tag[16];
    uint8_t pad0[128];
    uint8_t q8x[SC_Q8X_BYTES];
    // the fused layer also posts what the host needs to route the token and
    // compute its experts as soon as each part exists, as tagged words
    // (seq << 32) | payload: every logit (bias added) and the 32-bit words
    // of Q8_K(x) (q8x's bytes, word by word)
    uint64_t logit[SC_MAX_E];
    uint64_t q8x_words[SC_Q8X_BYTES / 4];
};
__host__ __device__ inline uint64_t sc_tag(uint32_t seq, int32_t slot, int32_t id) {
    return ((uint64_t)seq << 32) | ((uint64_t)(uint16_t)slot << 16) | (uint64_t)(uint16_t)id;
}
struct alignas(128) SidecarResp {
    uint32_t seq;                              // host -> GPU
    uint32_t pad0[15];
    uint32_t err;                              // GPU -> host: the join gave up waiting
    uint32_t pad1[15];
};
constexpr uint32_t SC_ABORT = 0xffffffffu;

// Just-in-time streaming.  A table word written in the middle of a token
// carries STREAM_BIT next to the slot: the expert's bytes were copied into
// the slot by the host's copy stream while the token ran, and kernels that
// read that slot first invalidate their caches (agent-scope acquire).  The
// boundary's table flush rewrites every such word without the bit.
constexpr int32_t STREAM_BIT = 0x40000000;
constexpr int32_t SLOT_MASK = 0x0fffffff;
constexpr int AHEAD_K = 8;                     // candidates per target layer at most

// Router lookahead record: layer L's router launch scores the routers of
// layers L+1 and L+2 on L's input (x * g_T / g_L) and posts, per target, the
// experts of its top-k whose table word is the dummy, best first: every word
// written through to host memory, the wave waits for them, seq last.  t: the
// GPU's 100 MHz wall clock at the post.
struct alignas(256) AheadPost {
    uint32_t seq;
    uint32_t layer;
    uint32_t t_lo, t_hi;
    int32_t target[2];                         // -1: none
    int32_t n[2];
    int32_t ids[2][AHEAD_K];
};

struct RouteLaunch {
    const float *W;        // [E][H] f32
    const float *x;        // [n_tok][H] f32
    const float *bias;     // [n_tok][E] or null (synthetic steering)
    const float *prior;    // [E] or null (cache prior: delta on resident experts)
    const int32_t *table;  // [E] or null (expert -> slot, n_slots = absent)
    int32_t dummy;
    int prior_on_logits;   // 1: the prior is added to the logits (selection only)
    int E, H, K, n_tok;
    const float *logits_in; // [n_tok][E] given logits (no router GEMV) or null
    float *logits;         // scratch [n_tok][E]
    uint32_t *counter;     // scratch [n_tok], zero
    int32_t *ids;          // out [n_tok][K]
    float *w;              // out [n_tok][K]
    int32_t *slots;        // out [n_tok][K]
    float *probs;          // out [n_tok][E] or null
    uint8_t *q8x;          // out [n_tok][H/256][292]
    SidecarPost *post;     // batch-1 decode with CPU-assisted serving: post ids + Q8_K(x), or null
    const uint32_t *seq;   // device: the token's sequence number, or null: seq_val (one layer decoded on
    uint32_t seq_val;      // its own carries the call's number by value; 0 reads as 1)
    // router lookahead (batch 1, router GEMV path): an > 0 target layers
    int an, ak;            // targets (0..2), candidates kept per target (<= AHEAD_K)
    const float *aW[2];    // [E][H] f32 routers of the targets
    const float *ar[2];    // [H] g_target / g_this
    const int32_t *atbl[2];
    int32_t adummy[2];
    int32_t atarget[2];
    int32_t alayer;
    float *alog;           // scratch [2][E]
    AheadPost *apost;      // the record (mapped host memory, or device memory for a test)
    uint32_t *fresh;       // non-null: read the table at system scope (words may flip in the middle
                           // of the token) and set *fresh when a word carries STREAM_BIT
};

struct ExpertArgs {
    const int32_t *ids;       // [K]
    const int32_t *slots;     // [K]
    const float *w;           // [K]
    const uint8_t *slot_pool; // [n_slots][slot_bytes] in HBM
    uint64_t slot_bytes;
    int n_slots;
    const uint8_t *host_store;  // [n_experts][expert_bytes], device view of pinned host memory
    uint64_t expert_bytes;
    int n_experts;
    const uint8_t *q8x;       // [H/256][292]
    float *h;                 // scratch [K + n_shared][I]
    uint8_t *q8h;             // scratch [K + n_shared][I/256][292]
    uint32_t *counter;        // scratch [K], zero
    float *out;               // [H]
    int accumulate;           // 1: out += result
    float *ypart;             // scratch [K + n_shared][H] or null: each expert's down rows, kept by the
                              // first launch of a resident/absent pair for the second
    int join;                 // 1: second launch of a pair; rows of the experts the first launch
                              // served come from ypart and out is the whole k-order sum
    uint8_t *stage;           // [K][stage_stride] in HBM or null: an expert read from the pinned
                              // store is also written here, byte for byte, so that an upload of it
                              // can be a device-to-device copy
    uint64_t stage_stride;
    int H, I, K, down_type;
    const uint8_t *shared;    // always-on shared expert in HBM (weight 1, combined after the K routed
                              // ones) or null; it is expert K of the launch
    int n_shared;             // 1 with a shared expert
    int cpu_num, cpu_den;     // CPU-assisted serving (den > 0): the CPU computes absent expert k when
                              // its rank among the absent ones (k order) r has r % den < num
    const uint32_t *fresh;    // non-null and set: a slot of this layer was filled by the copy stream
                              // during the token; invalidate caches before reading weights
};

// batch-1 combine after CPU-assisted serving: waits (bounded) for the host's
// answer, then out = sum_k w_k y_k in k order (rows from the host or from
// ypart) + the shared expert's row
struct JoinArgs {
    const int32_t *ids, *slots;
    const float *w;
    const uint8_t *slot_pool;
    int n_slots;
    const uint8_t *host_store;
    int n_experts, K, H, n_shared, cpu_num, cpu_den;
    const float *ypart;       // dev [K + n_shared][H]
    const float *hrows;       // mapped host [K][H]
    SidecarResp *resp;        // mapped host
    const uint32_t *seq;      // dev, or null: seq_val is the call's sequence number
    uint32_t seq_val;
    uint64_t timeout_ticks;   // of the 100 MHz wall clock
    float *out;               // dev [H]
};

// Self-test of the CPU-assisted serving channel, over the words the decode
// uses (one layer's post, answer and rows): in round r the kernel posts every
// logit word and every Q8_K(x) word of the post as (seq0 + r) << 32 | a seeded
// pattern, waits (bounded by the 100 MHz wall clock) for the host's answer,
// then checks the H rows the host wrote.  A timeout ends the kernel: the
// rounds left count as failed.
struct ScSelfTestArgs {
    SidecarPost *post;        // mapped host
    const SidecarResp *resp;  // mapped host
    const float *rows;        // mapped host [H]
    int n_rounds, E, n_q8_words, H;
    uint32_t seq0;
    uint64_t timeout_ticks;
    uint32_t *bad;            // dev: failed exchanges (zeroed by the caller)
};
// the seeded words of round r (splitmix64 finaliser of (round, index, stream))
__host__ __device__ inline uint32_t sc_test_word(uint32_t r, uint32_t i, uint32_t stream) {
    uint64_t z = ((uint64_t)r << 32 | i) + 0x9e3779b97f4a7c15ull * (stream + 1);
    z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
    z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
    return (uint32_t)(z ^ (z >> 31));
}
hipError_t launch_sc_selftest(const ScSelfTestArgs &a, hipStream_t st);

// A batch-1 decode layer in one launch: the router GEMV, the selection, every
// routed expert's gate/up rows, its down rows and the weighted combine.
// Inside the launch the phases pass tagged 8-byte words, (token sequence
// number << 32) | payload, each written and read whole at agent scope; a word
// is valid once its tag is the token's number, so nothing is reset between
// tokens.  Workgroups in index order: with CPU-assisted serving first H/256
// that post x's Q8_K blocks to the host, then [0, E) router rows (each also
// posting its logit to the host when serving), the selection, gate/up row
// tiles, down row tiles, combine tiles; a workgroup waits only
// for words of workgroups with a lower index.  The gate/up workgroups route
// the token themselves from the posted logits (the selection's code, so the
// same ids), which spares them the wait for the selection's record; the
// down and combine workgroups read the record.
constexpr int FUSED_LOG_COPIES = 8; // copies of the posted logits (fewer readers per line)
constexpr int FUSED_COPIES = 16;    // copies of the routing record (fewer readers per line)
constexpr int FUSED_REC = 32;       // words per copy: [k] sc_tag(seq, slot, id) of routed expert k,
                                    // [16 + k] (seq << 32) | bits of its gate weight
constexpr int FUSED_GU_TILE = 16;   // gate/up rows per workgroup (4 per wave)
constexpr int FUSED_DN_TILE = 32;   // down rows per workgroup (8 per wave)
struct FusedArgs {
    RouteLaunch r;            // router and selection (seq, table, prior, bias, post; no lookahead)
    ExpertArgs x;             // the experts; x.ids/slots/w receive the selection.  x.ypart set: the down
                              // rows go there for the join kernel (CPU-assisted serving) and there is
                              // no combine; else combine workgroups write x.out
    uint64_t *xlog;           // [FUSED_LOG_COPIES][256] tagged logits (bias added)
    uint64_t *rec;            // [FUSED_COPIES][FUSED_REC] tagged routing words
    uint64_t *hx;             // [K + 1][I] tagged SwiGLU activations
    uint64_t *yx;             // [K + 1][H] tagged down rows
    uint32_t *err;            // a bounded wait ran out: the token's sequence number is written here
    uint64_t wait_ticks;      // bound of every wait, 100 MHz wall clock
    // Publishing to the host (or pub null): tagged words in mapped host memory,
    // [l * K + k] = (seq << 32) | (slot & 0xffff) << 16 | id of layer l's routed
    // expert k, [L * K] = (seq << 32) | the late word.  The layer's last combine
    // workgroup writes the layer's words after every combine workgroup has
    // written its output rows (through to memory), and with pub_done the late
    // word: when every word carries the token's number its outputs are complete.
    uint64_t *pub;
    uint64_t *pub_ctr;        // (seq << 32) | the layer's combine workgroups finished
    int pub_layer, pub_L;
    int pub_done;
};
// exchange words per layer of the fused decode
inline size_t fused_words(int K, int I, int H) {
    return (size_t)FUSED_LOG_COPIES * 256 + (size_t)FUSED_COPIES * FUSED_REC + (size_t)(K + 1) * I +
           (size_t)(K + 1) * H;
}

constexpr int MAX_E = 256;   // experts per layer the kernels support
static_assert(MAX_E == SC_MAX_E, "the post holds every logit");

// batched layer: pairs dispatched expert-major, experts from slots or a store
struct GroupedArgs {
    const int32_t *offsets;     // [E+1] from the dispatch
    const int32_t *perm;        // [P] pair index t*K + k, expert-major
    const float *w;             // [n_tok*K] gate weights
    const int32_t *table;       // [E] slot per expert (>= n_slots: not resident) or null
    const uint8_t *slot_pool;   // [n_slots][slot_bytes] in HBM
    uint64_t slot_bytes;
    int n_slots;
    const uint8_t *store;       // [n_store][expert_bytes]: HBM or device view of pinned memory
    uint64_t expert_bytes;
    int n_store;
    int E, K, H, I, down_type;
    int P;                      // pairs dispatched (n_tok * K): picks the pass chunking
    const uint16_t *xa;         // [n_tok][H] Q8_K values of x as fp16
    const float *xdx;           // [n_tok][H/256]
    const uint16_t *xbs;        // [n_tok][H/16] group sums as fp16
    float *y2;                  // [P][2I] up and gate rows of every pair, dispatch order
    const uint16_t *ha;         // [P][I] Q8_K of h as fp16
    const float *hdx;           // [P][I/256]
    const uint16_t *hbs;        // [P][I/16]
    float *ypair;               // [P][H] weighted rows, pair (t*K + k) order
    const uint8_t *host_mask;   // [E] or null: experts the host computes (their rows read as zeros)
};

hipError_t launch_dispatch(const int32_t *ids, int P, int E, int32_t *counts, int32_t *offsets, int32_t *perm,
                           hipStream_t st);
hipError_t launch_quant_rows(const void *src, int bf16, int n_rows, int n, uint16_t *q16, float *dx, uint16_t *bs16,
                             hipStream_t st);
hipError_t launch_gateup_grouped(const GroupedArgs &a, hipStream_t st, hipEvent_t e0, hipEvent_t e1);
hipError_t launch_down_grouped(const GroupedArgs &a, hipStream_t st, hipEvent_t e0, hipEvent_t e1);
hipError_t launch_combine(const float *ypair, int n_tok, int K, int H, float *out, int accumulate, hipStream_t st);
// the same sum with the rows of pairs flagged in hflag [n_tok*K] taken from hrows [n_tok*K][H]
// (the host's, in mapped memory) instead of ypair
hipError_t launch_combine_host(const float *ypair, const float *hrows, const uint8_t *hflag, int n_tok, int K, int H,
                               float *out, int accumulate, hipStream_t st);
hipError_t launch_iota(int n, int32_t *offsets, int32_t *perm, float *ones, hipStream_t st);
// the allocation-free grouped entry point's workspace: this device's address
// of a static device array of STATIC_SCRATCH_BYTES
constexpr size_t STATIC_SCRATCH_BYTES = 16ull << 20;
hipError_t static_scratch(void **ptr);
// h = silu(gate) * up from y2 and its Q8_K (h itself to h_out when not null)
hipError_t launch_swiglu_quant(const float *y2, int P, int I, float *h_out, uint16_t *q16, float *dx, uint16_t *bs16,
                               hipStream_t st);

// ev (optional): [logits start, logits end, select start, select end]
hipError_t launch_route(const RouteLaunch &l, hipStream_t st, hipEvent_t *ev = nullptr);
hipError_t launch_experts(const ExpertArgs &a, hipStream_t st);
hipError_t launch_join(const JoinArgs &a, hipStream_t st);
// the fused layer (see FusedArgs); its down rows are of down_type
hipError_t launch_fused(const FusedArgs &a, hipStream_t st, hipEvent_t e0, hipEvent_t e1);
// src: 0 every routed expert, 1 only those resident in HBM slots, 2 only
// those read from the pinned host store.  A src = 2 down launch accumulates
// into out when the caller sets accumulate.
// e0/e1 (optional): stamped at the kernel's start and end of execution
hipError_t launch_gateup(const ExpertArgs &a, int src, hipStream_t st, hipEvent_t e0, hipEvent_t e1);
hipError_t launch_down(const ExpertArgs &a, int src, hipStream_t st, hipEvent_t e0, hipEvent_t e1);
hipError_t launch_synth_experts(uint64_t seed, int layer, int e0, int n_experts, int H, int I, int down_type,
                                float sigma, uint8_t *out, uint64_t stride, hipStream_t st);
// measurement: a streaming read of `bytes` (8 16-byte loads in flight per thread)
hipError_t launch_stream_read(const void *p, uint64_t bytes, uint32_t *out, hipStream_t st, hipEvent_t e0,
                              hipEvent_t e1);
unsigned stream_read_blocks(uint64_t bytes);
hipError_t launch_synth_vec(uint64_t seed, int kind, int a0, int na, int b0, int nb, int n, float sigma,
                            float *out, hipStream_t st);

}  // namespace mp
