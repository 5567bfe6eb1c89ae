// mp_kernels.hip -- gfx950 kernels of the batch-1 MoE decode step.
//
//   route_logits    router GEMV (W_r f32 [E][H]), one wavefront per expert row
//   route_select    softmax -> + cache prior -> top-k -> renormalised gate
//                   weights -> slot lookup, and the Q8_K quantization of x the
//                   expert kernels consume (one workgroup per token)
//   gateup_kernel   for K routed experts: up/gate Q4_K rows against Q8_K(x)
//                   with v_dot4_i32_i8, h = silu(gate) * up.  Resident experts
//                   are read from their HBM slot, absent ones straight from the
//                   pinned host store.
//   down_kernel     Q8_K of each expert's h into LDS, down rows (Q4_K or Q6_K)
//                   staged through LDS in 16-byte aligned chunks of 8 rows (Q6_K
//                   rows are only 2-byte aligned), and the weighted combine over
//                   k in order.
// No kernel communicates across workgroups: on a multi-XCD part that needs a
// device-scope fence (an L2 write-back and invalidate per workgroup), which
// cost more than the kernels' own work; kernel boundaries order the phases.
//
// Numerics: integer dots are exact; fp32 only at the per-super-block scale and
// across super-blocks.  The router follows the canonical order documented with
// the oracle bit for bit (explicit fmaf, fixed butterflies, -ffp-contract=off).
#include <hip/hip_ext.h>
#include <hip/hip_runtime.h>

#include "mp_device.h"
#include "mp_format.h"
#include "mp_internal.h"
#include "mp_synth.h"

namespace mp {

// the bytes of one Q8_K block from a wave's codes (4 per lane) and scale
__device__ void q8k_store(const int q[4], float d, uint8_t *out, int lane) {
    const int gs = q8k_group_sum(q);
    const uint32_t packed = (uint32_t)(q[0] & 0xff) | ((uint32_t)(q[1] & 0xff) << 8) |
                            ((uint32_t)(q[2] & 0xff) << 16) | ((uint32_t)(q[3] & 0xff) << 24);
    *(uint32_t *)(out + 4 + 4 * lane) = packed;
    if ((lane & 3) == 0) *(int16_t *)(out + 4 + QK + 2 * (lane >> 2)) = (int16_t)gs;
    if (lane == 0) *(float *)out = d;
}

// One wavefront quantizes 256 values (4 per lane, lane-major) to a Q8_K block.
__device__ void q8k_wave(const float *x, uint8_t *out, int lane) {
    const float4 v = *(const float4 *)(x + 4 * lane);
    const float xv[4] = {v.x, v.y, v.z, v.w};
    int q[4];
    float d;
    q8k_wave_vals(xv, lane, q, d);
    q8k_store(q, d, out, lane);
}

// A store coherent at system scope: written through the caches to memory
// (global_store ... sc0 sc1).  The records posted to the host are written with
// it: a plain store to host memory may stay in L2, and only a write-back of
// the whole L2 (what a system-scope release does) would push it out.  After
// the wave waits for its stores (vmcnt 0), every word is visible to the host
// before the sequence number that publishes them.
__device__ inline void store_sys(int32_t *p, int32_t v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
}
__device__ inline void store_sys(uint32_t *p, uint32_t v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
}

// The bytes of one Q8_K block (as q8k_store writes them) as 73 words written
// through to host memory: d, 64 words of codes, the 16 group sums two to a
// word.  The wave waits for them before it goes on.
__device__ void q8k_store_sys(const int q[4], float d, uint32_t *out, int lane) {
    const int gs = q8k_group_sum(q);
    const int gs_odd = __shfl_down(gs, 4, 64);       // group 2m + 1 for the lane holding 2m
    const uint32_t packed = (uint32_t)(q[0] & 0xff) | ((uint32_t)(q[1] & 0xff) << 8) |
                            ((uint32_t)(q[2] & 0xff) << 16) | ((uint32_t)(q[3] & 0xff) << 24);
    store_sys(out + 1 + lane, packed);
    if ((lane & 7) == 0) store_sys(out + 1 + QK / 4 + (lane >> 3), ((uint32_t)gs & 0xffffu) | ((uint32_t)gs_odd << 16));
    if (lane == 0) store_sys(out, __float_as_uint(d));
    __builtin_amdgcn_s_waitcnt(0x0f70);
}

// The same words as q8k_store_sys, each as (seq << 32) | word, without the
// wait: a reader takes a word once its tag is seq.
__device__ void q8k_store_tagged_sys(const int q[4], float d, uint64_t *out, uint32_t seq, int lane) {
    const int gs = q8k_group_sum(q);
    const int gs_odd = __shfl_down(gs, 4, 64);
    const uint32_t packed = (uint32_t)(q[0] & 0xff) | ((uint32_t)(q[1] & 0xff) << 8) |
                            ((uint32_t)(q[2] & 0xff) << 16) | ((uint32_t)(q[3] & 0xff) << 24);
    const uint64_t tag = (uint64_t)seq << 32;
    __hip_atomic_store(out + 1 + lane, tag | packed, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
    if ((lane & 7) == 0)
        __hip_atomic_store(out + 1 + QK / 4 + (lane >> 3), tag | (((uint32_t)gs & 0xffffu) | ((uint32_t)gs_odd << 16)),
                           __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
    if (lane == 0) __hip_atomic_store(out, tag | __float_as_uint(d), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
}

// ---------------------------------------------------------------------------
// router
struct RouteArgs {
    const float *W;        // [E][H]
    const float *x;        // [n_tok][H]
    const float *bias;     // [n_tok][E] or null
    const float *prior;    // [E] or null
    const int32_t *table;  // [E] or null
    int32_t dummy;         // slot value for "absent" when no table
    int prior_on_logits;   // 1: prior added to the logits for the selection
    int E, H, K;
    const float *logits_in; // [n_tok][E] given logits (the GEMV is skipped; bias still added) or null
    float *logits;         // scratch [n_tok][E]
    uint32_t *counter;     // scratch [n_tok], zero between launches
    int32_t *ids;          // [n_tok][K]
    float *w;              // [n_tok][K]
    int32_t *slots;        // [n_tok][K]
    float *probs;          // [n_tok][E] or null
    uint8_t *q8x;          // [n_tok][H/256 * 292]
    SidecarPost *post;     // batch 1 with CPU-assisted serving, or null
    const uint32_t *seq;   // or null: seq_val
    uint32_t seq_val;
    int an, ak;            // router lookahead: target layers (0..2), candidates per target
    const float *aW[2];
    const float *ar[2];
    const int32_t *atbl[2];
    int32_t adummy[2], atarget[2], alayer;
    float *alog;           // [2][E]
    AheadPost *apost;
    uint32_t *fresh;       // table words may flip during the token (see STREAM_BIT)
};

constexpr int RL_WAVES = 4;                      // router GEMV: waves (row quarters) per workgroup

// One quarter of a router row's dot product in the canonical order: wave q
// of the row's workgroup, lane j accumulates with fmaf (from 0) the products
// W[Q q + 256 i + 4 j + c] * x[...] over i, then c, and the 64 lanes are
// summed by a butterfly.  With r, the product x * r (rounded to f32) takes
// x's place (router lookahead).
__device__ inline float router_quarter(const float *w, const float *x, const float *r, int H, int q, int lane) {
    const int Q = H / RL_WAVES;
    float acc = 0.0f;
    for (int i = 0; i < Q / 256; ++i) {
        const int o = Q * q + 256 * i + 4 * lane;
        const float4 wv = *(const float4 *)(w + o);
        float4 xv = *(const float4 *)(x + o);
        if (r) {
            const float4 rv = *(const float4 *)(r + o);
            xv.x = xv.x * rv.x; xv.y = xv.y * rv.y; xv.z = xv.z * rv.z; xv.w = xv.w * rv.w;
        }
        acc = fmaf(wv.x, xv.x, acc);
        acc = fmaf(wv.y, xv.y, acc);
        acc = fmaf(wv.z, xv.z, acc);
        acc = fmaf(wv.w, xv.w, acc);
    }
    return wave_sum_canon(acc);
}

// One workgroup of RL_WAVES waves per router row: wave q sums quarter q, and
// the four quarter sums are added in order (s0 + s1) + s2 + s3, plus the
// steering bias when given.  The first H/256 workgroups also write the Q8_K
// blocks of x.  With router lookahead (batch 1) E more workgroups per target
// layer T score T's router on the products x[i] * r_T[i] in the same order.
__global__ __launch_bounds__(64 * RL_WAVES) void route_logits_kernel(RouteArgs a) {
    const int tok = blockIdx.y;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int t = (int)blockIdx.x / a.E;             // 0: this layer, 1..an: lookahead target t - 1
    const int e = (int)blockIdx.x - t * a.E;
    const float *x = a.x + (size_t)tok * a.H;
    __shared__ float s_q[RL_WAVES];
    const float *w = t > 0 ? a.aW[t - 1] + (size_t)e * a.H : a.W + (size_t)e * a.H;
    const float part = router_quarter(w, x, t > 0 ? a.ar[t - 1] : nullptr, a.H, wave, lane);
    if (lane == 0) s_q[wave] = part;
    __syncthreads();
    if (threadIdx.x == 0) {
        float acc = s_q[0];
#pragma unroll
        for (int q = 1; q < RL_WAVES; ++q) acc = acc + s_q[q];
        if (t > 0) {
            a.alog[(size_t)(t - 1) * a.E + e] = acc;
        } else {
            if (a.bias) acc = acc + a.bias[(size_t)tok * a.E + e];
            a.logits[(size_t)tok * a.E + e] = acc;
        }
    }
    // Q8_K of x: workgroup b (one of the first H/256) quantizes block b; with
    // CPU-assisted serving (batch 1) also into the host's post, written
    // through before this kernel ends, so that the select kernel's post only
    // adds the ids
    if (t == 0 && a.q8x && wave == 0 && (int)blockIdx.x < a.H / QK) {
        const float4 v = *(const float4 *)(x + QK * blockIdx.x + 4 * lane);
        const float xv[4] = {v.x, v.y, v.z, v.w};
        int q[4];
        float d;
        q8k_wave_vals(xv, lane, q, d);
        q8k_store(q, d, a.q8x + ((size_t)tok * (a.H / QK) + blockIdx.x) * Q8K_BYTES, lane);
        if (a.post && tok == 0) q8k_store_sys(q, d, (uint32_t *)(a.post->q8x + (size_t)blockIdx.x * Q8K_BYTES), lane);
    }
}

// ---------------------------------------------------------------------------
// Router lookahead (batch 1).  The router's GEMV kernel scored the target
// layers' routers on x * r_T; the select kernel ranks those scores with the
// threads its own ranking leaves idle (descending, the lower id first on a
// tie, a NaN with -inf) into s_top, and one wave -- beside the wave that posts
// the layer's own routing -- keeps the top ak whose table word is the dummy
// (best first) and posts the record with the GPU clock, every word written
// through to host memory, and the token's sequence number last.  Every layer posts, with no
// target too: the record also tells the host the layer has read its table.
__device__ inline void ahead_rank(const RouteArgs &a, const float (*s_asel)[256], int (*s_top)[AHEAD_K], int i) {
    const int t = i / a.E, e = i - t * a.E;
    const float v = s_asel[t][e];
    int rank = 0;
    for (int j = 0; j < a.E; j += 4) {
        const float4 u = *(const float4 *)&s_asel[t][j];
        rank += (u.x > v) | ((u.x == v) & (j < e));
        rank += (u.y > v) | ((u.y == v) & (j + 1 < e));
        rank += (u.z > v) | ((u.z == v) & (j + 2 < e));
        rank += (u.w > v) | ((u.w == v) & (j + 3 < e));
    }
    if (rank < a.ak) s_top[t][rank] = e;
}

__device__ void ahead_post(const RouteArgs &a, const int (*s_top)[AHEAD_K], uint32_t seq, int lane) {
    AheadPost *r = a.apost;
    const int t = lane >> 3, j = lane & 7;          // lanes 0-7 target 0, 8-15 target 1: one round of loads
    bool keep = false;
    int e = -1;
    if (lane < 16 && t < a.an && j < a.ak) {
        // a plain load: a word the copy stream flipped a moment ago may still
        // read as the dummy here, which only offers the host an expert it
        // already streams (it drops it); the layer's own read is fresh
        e = s_top[t][j];
        keep = a.atbl[t][e] == a.adummy[t];
    }
    // every load before the first store: a wait after a write-through store
    // would also wait for it to land
    const int32_t target = lane == 0 ? a.atarget[0] : a.atarget[1];
    const uint64_t m = __ballot(keep);
    const uint64_t mt = (m >> (8 * t)) & 0xffull;
    __builtin_amdgcn_s_waitcnt(0x0f70);
    if (keep) store_sys(&r->ids[t][__popcll(mt & ((1ull << j) - 1ull))], e);
    if (lane < 2) {
        store_sys(&r->n[lane], lane < a.an ? (int32_t)__popcll((m >> (8 * lane)) & 0xffull) : 0);
        store_sys(&r->target[lane], lane < a.an ? target : -1);
    }
    if (lane == 0) {
        const uint64_t now = wall_clock64();
        store_sys(&r->layer, (uint32_t)a.alayer);
        store_sys(&r->t_lo, (uint32_t)now);
        store_sys(&r->t_hi, (uint32_t)(now >> 32));
    }
    // written through (store_sys): waiting for them orders them before the
    // sequence number, with no write-back of the whole L2
    __builtin_amdgcn_s_waitcnt(0x0f70);
    if (lane == 0) __hip_atomic_store(&r->seq, seq, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
}

// One workgroup per token.  Wave c owns experts 64c .. 64c+63: logits, the
// wave's max and its 64-lane butterfly sum of exp (the canonical per-chunk
// sums, added in chunk order), probabilities and the selection value (+ prior).
// Top-k by rank: thread e counts the experts ahead of e in (selection
// descending, id ascending) order -- no dependent shuffle chain -- and rank < K
// places e.  With given logits, also the Q8_K of x (all four waves) when x and
// q8x are given; otherwise the router GEMV kernel wrote it.
__global__ __launch_bounds__(256) void route_select_kernel(RouteArgs a) {
    const int tok = blockIdx.x;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int nc = a.E / 64;
    __shared__ float s_p[256];
    __shared__ __attribute__((aligned(16))) uint64_t s_key[256];
    __shared__ float s_m[4], s_cs[4];
    __shared__ int s_ids[16];
    __shared__ __attribute__((aligned(16))) float s_asel[2][256];   // lookahead scores
    __shared__ int s_top[2][AHEAD_K];
    __shared__ int32_t s_tbl[256];
    // Every global load first, all in flight together: the table word of
    // expert tid (at system scope when the host's copy stream may write words
    // while the token runs), the lookahead scores, the logits, the sequence
    // number.  The selection then needs no dependent round trip.
    const bool look = a.apost && !a.logits_in;
    int32_t tword = 0;
    if (a.table && tid < a.E)
        tword = a.fresh ? __hip_atomic_load(a.table + tid, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM)
                        : a.table[tid];
    float av[2] = {0.0f, 0.0f};
    if (look)
        for (int j = 0; j < 2; ++j)
            if (tid + 256 * j < a.an * a.E) av[j] = a.alog[tid + 256 * j];
    float l = 0.0f, pr = 0.0f;
    if (wave < nc) {
        const int ee = 64 * wave + lane;
        if (a.logits_in) {
            l = a.logits_in[(size_t)tok * a.E + ee];
            if (a.bias) l = l + a.bias[(size_t)tok * a.E + ee];
        } else {
            l = a.logits[(size_t)tok * a.E + ee];
        }
        if (a.prior) pr = a.prior[ee];
    }
    const uint32_t seqv = a.seq ? *a.seq : a.seq_val;
    if (a.table && tid < a.E) s_tbl[tid] = tword;
    if (look)
        for (int j = 0; j < 2; ++j) {
            const int i = tid + 256 * j;
            if (i < a.an * a.E) {
                const int t = i / a.E, e = i - t * a.E;
                s_asel[t][e] = av[j] != av[j] ? -INFINITY : av[j];
            }
        }
    if (wave < nc) {
        const float m = wave_max(l);
        if (lane == 0) s_m[wave] = m;
    }
    __syncthreads();
    float ex = 0.0f;
    if (wave < nc) {
        float m = s_m[0];
        for (int c = 1; c < nc; ++c) m = fmaxf(m, s_m[c]);
        ex = canon_expf(l - m);
        const float cs = wave_sum_canon(ex);
        if (lane == 0) s_cs[wave] = cs;
    }
    __syncthreads();
    if (wave < nc) {
        float sum = s_cs[0];
        for (int c = 1; c < nc; ++c) sum = sum + s_cs[c];
        const int ee = 64 * wave + lane;
        const float p = ex / sum;
        s_p[ee] = p;
        if (a.probs) a.probs[(size_t)tok * a.E + ee] = p;
        float sel = !a.prior ? p : (a.prior_on_logits ? l + pr : p + pr);
        s_key[ee] = sel_key(sel, ee);                 // a NaN sorts last
    }
    __syncthreads();
    if (tid < a.E) {
        const int rank = key_rank(s_key, a.E, s_key[tid]);
        if (rank < a.K) s_ids[rank] = tid;
    } else if (look) {
        for (int i = tid - a.E; i < a.an * a.E; i += 256 - a.E) ahead_rank(a, s_asel, s_top, i);
    }
    __syncthreads();
    if (look && a.E >= 256) {            // no idle threads above: a phase of its own
        for (int i = tid; i < a.an * a.E; i += 256) ahead_rank(a, s_asel, s_top, i);
        __syncthreads();
    }
    if (wave == 0) {
        // lane k finishes slot k; the weight sum is the same left-to-right sum on every lane
        float ws = 0.0f;
        for (int k = 0; k < a.K; ++k) ws = ws + s_p[s_ids[k]];
        int slot = a.dummy;
        bool streamed = false;
        if (lane < a.K) {
            const int id = s_ids[lane];
            a.ids[(size_t)tok * a.K + lane] = id;
            a.w[(size_t)tok * a.K + lane] = s_p[id] / ws;
            if (a.table && a.fresh) {
                const int32_t v = s_tbl[id];
                streamed = (v & STREAM_BIT) != 0;
                slot = v & SLOT_MASK;
            } else if (a.table) {
                slot = s_tbl[id];
            }
            a.slots[(size_t)tok * a.K + lane] = slot;
        }
        if (a.fresh) {
            const bool any = __ballot(streamed) != 0;
            if (lane == 0) *a.fresh = any ? 1u : 0u;
        }
        // CPU-assisted serving: post each id with the slot read, tagged with
        // the token's sequence number, one 8-byte store written through to
        // host memory per word (no L2 write-back, no wait: the host checks
        // every word's tag).  Only on the router-GEMV path, whose kernel wrote
        // the Q8_K of x into the post and waited for it before this kernel.
        if (a.post && !a.logits_in && lane < a.K)
            __hip_atomic_store(&a.post->tag[lane], sc_tag(seqv, slot, s_ids[lane]), __ATOMIC_RELAXED,
                               __HIP_MEMORY_SCOPE_SYSTEM);
    }
    if (look && wave == 1) ahead_post(a, s_top, seqv, lane);      // beside wave 0's own post
    if (!a.logits_in || !a.x || !a.q8x) return;
    const float *x = a.x + (size_t)tok * a.H;
    uint8_t *q8 = a.q8x + (size_t)tok * (a.H / QK) * Q8K_BYTES;
    for (int b = wave; b < a.H / QK; b += 4) q8k_wave(x + QK * b, q8 + (size_t)b * Q8K_BYTES, lane);
}

// ---------------------------------------------------------------------------
// which experts a launch serves: all of them, only those resident in an HBM
// slot, or only those read from the pinned host store
constexpr int SRC_ALL = 0, SRC_HBM = 1, SRC_HOST = 2;

// routed expert k is absent from the slots and inside the store
__device__ inline bool absent_in_store(const int32_t *slots, const int32_t *ids, const uint8_t *slot_pool,
                                       int n_slots, const uint8_t *host_store, int n_experts, int k) {
    const int slot = slots[k], id = ids[k];
    return !(slot_pool && slot >= 0 && slot < n_slots) && host_store && id >= 0 && id < n_experts;
}

// CPU-assisted serving: the host computes absent expert k when its rank r
// among the absent experts (in k order) has r % den < num
__device__ inline bool cpu_served(const int32_t *slots, const int32_t *ids, const uint8_t *slot_pool, int n_slots,
                                  const uint8_t *host_store, int n_experts, int num, int den, int K, int k) {
    if (den <= 0 || k >= K) return false;
    if (!absent_in_store(slots, ids, slot_pool, n_slots, host_store, n_experts, k)) return false;
    int r = 0;
    for (int j = 0; j < k; ++j) r += absent_in_store(slots, ids, slot_pool, n_slots, host_store, n_experts, j);
    return r % den < num;
}

__device__ inline bool cpu_served(const ExpertArgs &a, int k) {
    return cpu_served(a.slots, a.ids, a.slot_pool, a.n_slots, a.host_store, a.n_experts, a.cpu_num, a.cpu_den, a.K,
                      k);
}

__device__ inline bool serves(const ExpertArgs &a, int k, int src) {
    if (cpu_served(a, k)) return false;
    if (src == SRC_ALL) return true;
    if (k >= a.K) return src == SRC_HBM;     // the shared expert lives in HBM
    const int slot = a.slots[k];
    const bool resident = a.slot_pool && slot >= 0 && slot < a.n_slots;
    return src == SRC_HBM ? resident : !resident;
}

// expert pointers: resident -> HBM slot, absent -> pinned host store
// (null for an id outside the store: that expert contributes zero)
__device__ inline const uint8_t *expert_base(const ExpertArgs &a, int k) {
    if (k >= a.K) return a.shared;
    const int slot = a.slots[k];
    if (a.slot_pool && slot >= 0 && slot < a.n_slots) return a.slot_pool + (size_t)slot * a.slot_bytes;
    const int id = a.ids[k];
    if (!a.host_store || id < 0 || id >= a.n_experts) return nullptr;
    return a.host_store + (size_t)id * a.expert_bytes;
}

// where the bytes of routed expert k go when the launch reads it from the
// pinned store: its staging area (null when not staging or not absent)
__device__ inline uint8_t *stage_base(const ExpertArgs &a, int k) {
    if (!a.stage || k >= a.K || cpu_served(a, k)) return nullptr;
    const int slot = a.slots[k];
    if (a.slot_pool && slot >= 0 && slot < a.n_slots) return nullptr;
    const int id = a.ids[k];
    if (!a.host_store || id < 0 || id >= a.n_experts) return nullptr;
    return a.stage + (size_t)k * a.stage_stride;
}

// Q4_K super-block partial of one lane: 16 qs bytes (chunk u) against the
// matching 32 activation bytes; returns (scale-weighted int dot, min-weighted bsum)
__device__ inline void q4k_lane(uint4 hdr, uint4 qs, int u, const uint32_t *xlo, const uint32_t *xhi,
                                int bslo, int bshi, int32_t &si, int32_t &mi) {
    const int j = u >> 1;  // 64-element group
    int sl, ml, sh, mh;
    q4k_sm(hdr, 2 * j, sl, ml);
    q4k_sm(hdr, 2 * j + 1, sh, mh);
    const uint32_t q[4] = {qs.x, qs.y, qs.z, qs.w};
    int32_t dl = 0, dh = 0;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        dl = sdot4(q[i] & 0x0F0F0F0Fu, xlo[i], dl);
        dh = sdot4((q[i] >> 4) & 0x0F0F0F0Fu, xhi[i], dh);
    }
    si = sl * dl + sh * dh;
    mi = ml * bslo + mh * bshi;
}

constexpr int GU_WAVES = 4;                      // gate/up: waves per workgroup
template <int R, int SRC>
__global__ __launch_bounds__(64 * GU_WAVES) void gateup_kernel(ExpertArgs a) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int k = blockIdx.y;
    if (!serves(a, k, SRC)) return;
    // a slot of this layer was written by the copy stream during the token:
    // drop cached lines of its previous contents before reading weights
    if (a.fresh && *a.fresh) __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
    const int b = lane >> 3, u = lane & 7;
    const int j = u >> 1;
    const uint8_t *base = expert_base(a, k);
    const size_t rb = (size_t)(a.H / QK) * Q4K_BYTES;     // 1152 at H = 2048
    const uint8_t *up = base, *gate = base + (size_t)a.I * rb;
    const bool valid = base != nullptr;

    // this lane's activation bytes, held for every row
    const uint8_t *xq = a.q8x + (size_t)b * Q8K_BYTES;
    const float dx = *(const float *)xq;
    uint32_t xlo[4], xhi[4];
    const uint32_t *plo = (const uint32_t *)(xq + 4 + 64 * j + 16 * (u & 1));
    const uint32_t *phi = (const uint32_t *)(xq + 4 + 64 * j + 32 + 16 * (u & 1));
#pragma unroll
    for (int i = 0; i < 4; ++i) { xlo[i] = plo[i]; xhi[i] = phi[i]; }
    const int16_t *bs = (const int16_t *)(xq + 4 + QK);
    const int bslo = bs[4 * j + (u & 1)], bshi = bs[4 * j + 2 + (u & 1)];

    const int row0 = (blockIdx.x * GU_WAVES + wave) * R;
    uint4 hg[R], qg[R], hu[R], qu[R];
#pragma unroll
    for (int r = 0; r < R; ++r) {
        const size_t off = (size_t)(row0 + r) * rb + (size_t)b * Q4K_BYTES;
        const uint4 z = make_uint4(0, 0, 0, 0);
        hg[r] = valid ? *(const uint4 *)(gate + off) : z;
        qg[r] = valid ? *(const uint4 *)(gate + off + 16 + 16 * u) : z;
        hu[r] = valid ? *(const uint4 *)(up + off) : z;
        qu[r] = valid ? *(const uint4 *)(up + off + 16 + 16 * u) : z;
    }
    if (SRC != SRC_HBM) {
        uint8_t *sb = stage_base(a, k);
        if (sb) {       // the same bytes, same offsets, into the staging area
            uint8_t *su = sb, *sg = sb + (size_t)a.I * rb;
#pragma unroll
            for (int r = 0; r < R; ++r) {
                const size_t off = (size_t)(row0 + r) * rb + (size_t)b * Q4K_BYTES;
                if (u == 0) {
                    *(uint4 *)(sg + off) = hg[r];
                    *(uint4 *)(su + off) = hu[r];
                }
                *(uint4 *)(sg + off + 16 + 16 * u) = qg[r];
                *(uint4 *)(su + off + 16 + 16 * u) = qu[r];
            }
        }
    }
#pragma unroll
    for (int r = 0; r < R; ++r) {
        float res[2];
#pragma unroll
        for (int m = 0; m < 2; ++m) {
            const uint4 hdr = m == 0 ? hg[r] : hu[r];
            const uint4 qs = m == 0 ? qg[r] : qu[r];
            int32_t si, mi;
            q4k_lane(hdr, qs, u, xlo, xhi, bslo, bshi, si, mi);
            si = sum8_dpp(si);
            mi = sum8_dpp(mi);
            const float d = h2f_dev((uint16_t)(hdr.x & 0xffff)) * dx;
            const float dm = h2f_dev((uint16_t)(hdr.x >> 16)) * dx;
            const int ps = __builtin_bit_cast(int, d * (float)si), pm = __builtin_bit_cast(int, dm * (float)mi);
            // the 8 super-blocks in row order, scale term then min term, as
            // the CPU vec_dot accumulates them (lane 8b holds block b)
            float v = 0.0f;
#pragma unroll
            for (int bb = 0; bb < 8; ++bb) {
                v = v + __builtin_bit_cast(float, __builtin_amdgcn_readlane(ps, 8 * bb));
                v = v - __builtin_bit_cast(float, __builtin_amdgcn_readlane(pm, 8 * bb));
            }
            res[m] = v;
        }
        if (lane == 0) {
            const float g = res[0], uu = res[1];
            a.h[(size_t)k * a.I + row0 + r] = g / (1.0f + canon_expf(-g)) * uu;
        }
    }

}

// Order a wave's LDS writes before its own lanes' later reads of them: the
// LDS executes one wave's instructions in order, so waiting for the wave's
// LDS operations and keeping the compiler from moving them across is enough.
__device__ inline void wave_lds_sync() {
    __builtin_amdgcn_s_waitcnt(0xc07f);          // lgkmcnt(0)
    __builtin_amdgcn_wave_barrier();
}

// ---------------------------------------------------------------------------
// down + combine.  Workgroup = 8 waves, 8 output rows; wave w owns expert
// kb + w of each group of 8 experts.
constexpr int DN_ROWS = 8;
constexpr int DN_LDS_ROWS = 8 * 3 * Q6K_PAD;   // 8 padded Q6_K rows at I = 768
constexpr int DN_LDS_Q8 = 3 * Q8K_BYTES;    // I <= 768

// One wave's 8 down rows (LDS: row g of the tile at g * rowb; Q4_K rows
// lane-contiguous as loaded, Q6_K blocks at the padded stride) against the
// Q8_K blocks of h (LDS): lane (g, u) works on row g,
// part u of each super-block; the row's value is complete on lanes with
// u == 0.  Super-blocks in order, scale term then min term (the CPU vec_dot
// order).
template <int DT>
__device__ inline float down_rows_dot(const uint8_t *s_wt, const uint8_t *s_q8h, int nb, int rowb, int lane) {
    const int g = lane >> 3, u = lane & 7;
    float y = 0.0f;
    for (int b = 0; b < nb; ++b) {
        const uint8_t *xq = s_q8h + b * Q8K_BYTES;
        const float dx = *(const float *)xq;
        int32_t si = 0, mi = 0;
        float d, dm = 0.0f;
        if (DT == TYPE_Q4K) {
            const uint8_t *blk = s_wt + g * rowb + b * Q4K_BYTES;
            const uint4 hdr = *(const uint4 *)blk;
            const uint4 qs = *(const uint4 *)(blk + 16 + 16 * u);
            const int j = u >> 1;
            const uint32_t *plo = (const uint32_t *)(xq + 4 + 64 * j + 16 * (u & 1));
            const uint32_t *phi = (const uint32_t *)(xq + 4 + 64 * j + 32 + 16 * (u & 1));
            uint32_t xlo[4], xhi[4];
            for (int i = 0; i < 4; ++i) { xlo[i] = plo[i]; xhi[i] = phi[i]; }
            const int16_t *bs = (const int16_t *)(xq + 4 + QK);
            q4k_lane(hdr, qs, u, xlo, xhi, bs[4 * j + (u & 1)], bs[4 * j + 2 + (u & 1)], si, mi);
            d = h2f_dev((uint16_t)(hdr.x & 0xffff)) * dx;
            dm = h2f_dev((uint16_t)(hdr.x >> 16)) * dx;
        } else {
            // Q6_K blocks at the padded stride (q6k_rows_store): aligned reads
            const uint8_t *blk = s_wt + g * rowb + b * Q6K_PAD;
            const int hh = u >> 2, up4 = u & 3;
            const uint2 va = *(const uint2 *)(blk + 64 * hh + 8 * up4);
            const uint2 vb = *(const uint2 *)(blk + 64 * hh + 8 * up4 + 32);
            const uint2 vh = *(const uint2 *)(blk + 128 + 32 * hh + 8 * up4);
            const uint2 vs = *(const uint2 *)(blk + 192 + 8 * hh);        // the half's 8 scales
            const uint32_t a0 = va.x, a1 = va.y, b0 = vb.x, b1 = vb.y, h0 = vh.x, h1 = vh.y;
            // scale of sub-block (up4 >> 1) + 2 q, q = 0..3: bytes (up4 >> 1) + 2 q of the 8
            const uint32_t sh = (uint32_t)(up4 >> 1) * 8;
            const uint32_t sw = ((vs.x >> sh) & 0x00ff00ffu) | (((vs.y >> sh) & 0x00ff00ffu) << 8);
            const int8_t sc[8] = {(int8_t)sw, 0, (int8_t)(sw >> 16), 0, (int8_t)(sw >> 8), 0, (int8_t)(sw >> 24), 0};
            const uint32_t L = 0x0F0F0F0Fu, Hm = 0x30303030u;
            const uint32_t qv[4][2] = {
                {(a0 & L) | ((h0 << 4) & Hm), (a1 & L) | ((h1 << 4) & Hm)},
                {(b0 & L) | ((h0 << 2) & Hm), (b1 & L) | ((h1 << 2) & Hm)},
                {((a0 >> 4) & L) | (h0 & Hm), ((a1 >> 4) & L) | (h1 & Hm)},
                {((b0 >> 4) & L) | ((h0 >> 2) & Hm), ((b1 >> 4) & L) | ((h1 >> 2) & Hm)}};
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const uint32_t *px = (const uint32_t *)(xq + 4 + 128 * hh + 32 * q + 8 * up4);
                const uint32_t x0 = px[0], x1 = px[1];
                int32_t dq = sdot4(qv[q][0], x0, sdot4(qv[q][1], x1, 0));
                const int32_t sx = sdot4(0x01010101u, x0, sdot4(0x01010101u, x1, 0));
                dq -= 32 * sx;
                si += (int32_t)sc[2 * q] * dq;
            }
            d = h2f_dev(*(const uint16_t *)(blk + 208)) * dx;
        }
        si = sum8_dpp(si);
        // super-block order, scale term then min term (CPU vec_dot order)
        y = y + d * (float)si;
        if (DT == TYPE_Q4K) {
            mi = sum8_dpp(mi);
            y = y - dm * (float)mi;
        }
    }
    return y;
}

template <int DT, int SRC>
__global__ __launch_bounds__(512) void down_kernel(ExpertArgs a) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int r0 = blockIdx.x * DN_ROWS;
    const int nb = a.I / QK;
    const int rowb = nb * (DT == TYPE_Q6K ? Q6K_BYTES : Q4K_BYTES);
    __shared__ __attribute__((aligned(16))) uint8_t s_w[8][DN_LDS_ROWS];
    __shared__ __attribute__((aligned(16))) uint8_t s_q8[8][DN_LDS_Q8 + 4];
    __shared__ float s_y[17][DN_ROWS];   // up to 16 routed experts + the shared one

    const int g = lane >> 3, u = lane & 7;   // g: row within the tile, u: part of a super-block
    const int kt = a.K + a.n_shared;
    if (a.fresh && *a.fresh) __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");   // as in gateup_kernel
    // the combine's inputs other than the rows, loaded now rather than after
    // the last barrier: the gate weights, and the output being added to
    float wk[16], prev = 0.0f;
    if (threadIdx.x < DN_ROWS) {
#pragma unroll
        for (int k = 0; k < 16; ++k)
            if (k < a.K) wk[k] = a.w[k];
        if (a.accumulate) prev = a.out[r0 + threadIdx.x];
    }
    for (int kb = 0; kb < kt; kb += 8) {
        const int k = kb + wave;
        // this expert's h first: vector loads return in the order they were
        // issued, so h is in registers before the weights issued after it
        // land, and its Q8_K is computed while they are in flight
        float xv[3][4];
        if (nb == 3 && k < kt) {
#pragma unroll
            for (int b = 0; b < 3; ++b) {
                const float4 v = *(const float4 *)(a.h + (size_t)k * a.I + QK * b + 4 * lane);
                xv[b][0] = v.x; xv[b][1] = v.y; xv[b][2] = v.z; xv[b][3] = v.w;
            }
        }
        const bool mine = k < kt && serves(a, k, SRC);
        bool direct = false;
        if (k < kt && !mine && lane < DN_ROWS)      // the other launch's expert
            s_y[k][lane] = a.join ? a.ypart[(size_t)k * a.H + r0 + lane] : 0.0f;
        if (mine) {
            const uint8_t *eb = expert_base(a, k);
            const int nvec = DN_ROWS * rowb / 16;           // <= 315
            const uint4 *src = eb ? (const uint4 *)(eb + 2ull * a.I * (a.H / QK) * Q4K_BYTES + (size_t)r0 * rowb)
                                  : nullptr;
            // Q8_K of h into LDS (every workgroup quantizes the same h the
            // same way: identical bytes)
            auto quantize_h = [&]() {
                if (nb == 3) {
                    int q[3][4];
                    float d[3];
                    q8k_wave_vals_n<3>(xv, lane, q, d);
#pragma unroll
                    for (int b = 0; b < 3; ++b) q8k_store(q[b], d[b], s_q8[wave] + b * Q8K_BYTES, lane);
                } else {
                    for (int b = 0; b < nb; ++b)
                        q8k_wave(a.h + (size_t)k * a.I + QK * b, s_q8[wave] + b * Q8K_BYTES, lane);
                }
            };
            // Rows that need no staging copy go straight from memory into LDS
            // (16 bytes a lane, lane-contiguous: the layout the dots read).
            // The others pass through registers on their way to the staging
            // area too.  Each branch quantizes h after issuing its loads.
            uint8_t *sb = SRC != SRC_HBM ? stage_base(a, k) : nullptr;
            direct = DT == TYPE_Q4K && src && !sb;
            if (DT == TYPE_Q6K) {
                Q6Rows rows;
                q6k_rows_load(rows, (const uint8_t *)src, DN_ROWS * nb, lane);
                quantize_h();
                q6k_rows_store(rows, s_w[wave],
                               sb ? sb + 2ull * a.I * (a.H / QK) * Q4K_BYTES + (size_t)r0 * rowb : nullptr,
                               DN_ROWS * nb, lane);
            } else if (direct) {
#pragma unroll
                for (int j = 0; j < 5; ++j) {
                    const int i = lane + 64 * j;
                    if (i < nvec)
                        __builtin_amdgcn_global_load_lds((const void *)(src + i),
                                                         (__attribute__((address_space(3))) void *)(s_w[wave] + 1024 * j),
                                                         16, 0, 0);
                }
                quantize_h();
            } else {
                uint4 buf[5];
#pragma unroll
                for (int j = 0; j < 5; ++j) {
                    const int i = lane + 64 * j;
                    buf[j] = (src && i < nvec) ? src[i] : make_uint4(0, 0, 0, 0);
                }
                quantize_h();
                uint4 *dst = (uint4 *)s_w[wave];
#pragma unroll
                for (int j = 0; j < 5; ++j) {
                    const int i = lane + 64 * j;
                    if (i < nvec) dst[i] = buf[j];
                }
                if (sb) {
                    uint4 *sd = (uint4 *)(sb + 2ull * a.I * (a.H / QK) * Q4K_BYTES + (size_t)r0 * rowb);
#pragma unroll
                    for (int j = 0; j < 5; ++j) {
                        const int i = lane + 64 * j;
                        if (i < nvec) sd[i] = buf[j];
                    }
                }
            }
        }
        // s_w[wave] and s_q8[wave] are written and read by this wave only:
        // the waves go on without waiting for each other's weights (the
        // loads into LDS count as vector memory operations: wait for those too)
        if (direct) __builtin_amdgcn_s_waitcnt(0x0f70);       // vmcnt(0)
        wave_lds_sync();
        if (mine) {
            const float y = down_rows_dot<DT>(s_w[wave], s_q8[wave], nb, nb * (DT == TYPE_Q6K ? Q6K_PAD : Q4K_BYTES), lane);
            if (u == 0) {
                s_y[k][g] = y;
                if (a.ypart && !a.join) a.ypart[(size_t)k * a.H + r0 + g] = y;
            }
        }
        wave_lds_sync();        // the next group's writes come after this wave's reads
    }
    __syncthreads();            // every wave's s_y before the combine
    if (threadIdx.x < DN_ROWS) {
        const int t = threadIdx.x;
        float acc = wk[0] * s_y[0][t];
#pragma unroll
        for (int k = 1; k < 16; ++k)
            if (k < a.K) acc = acc + wk[k] * s_y[k][t];
        if (a.n_shared) acc = acc + s_y[a.K][t];        // weight 1, after the routed experts
        a.out[r0 + t] = a.accumulate ? prev + acc : acc;
    }
}

// ---------------------------------------------------------------------------
// A batch-1 decode layer in one launch (see FusedArgs).  The phases hand over
// tagged words written and read at agent scope (coherent across the XCDs'
// L2s without a cache write-back or invalidation); every wait is for
// workgroups of a lower index, which the dispatcher starts first, and is
// bounded by the wall clock.  The gate/up workgroups route the token
// themselves; the down rows' weights are requested once the selection's
// record is seen, while the gate/up rows are still being read.

__device__ inline void store_tagged(uint64_t *p, uint64_t v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ inline uint64_t load_tagged(const uint64_t *p) {
    return __hip_atomic_load((uint64_t *)p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ inline uint64_t tagged(uint32_t seq, float v) { return ((uint64_t)seq << 32) | __float_as_uint(v); }
__device__ inline void fused_late(const FusedArgs &a, uint32_t seq) {
    __hip_atomic_store(a.err, seq, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// LDS of one fused workgroup, shared by the roles (each uses its own part)
constexpr int FUSED_LDS_W = 4 * DN_LDS_ROWS;                  // down: each wave's 8 weight rows
constexpr int FUSED_LDS_Q8 = 3 * Q8K_BYTES + 4;               // down: the Q8_K of h (I <= 768)
constexpr int FUSED_LDS_RS = FUSED_LDS_W + FUSED_LDS_Q8 + 8 * FUSED_REC + 16;   // the routing
constexpr int FUSED_LDS = FUSED_LDS_RS + 256;

// The routing record (copy `copy`): wave 0 polls until the words the
// workgroup needs carry seq -- with need_ids the K routing words, with need_w
// the K gate weights -- and leaves them in s_rec for the workgroup (the words
// not polled are 0).  false: the wait ran out (reported through a.err).
__device__ bool fused_record(const FusedArgs &a, int copy, uint32_t seq, bool need_ids, bool need_w, uint64_t *s_rec,
                             int *s_flag) {
    const int K = a.x.K;
    if (threadIdx.x < 64) {
        const int lane = threadIdx.x;
        const uint64_t *src = a.rec + (size_t)copy * FUSED_REC;
        const bool want = (need_ids && lane < K) || (need_w && lane >= 16 && lane < 16 + K);
        bool ok = !want;
        uint64_t v = 0;
        int late = 0;
        const uint64_t t0 = wall_clock64();
        for (;;) {
            if (!ok) {
                v = load_tagged(src + lane);
                ok = (uint32_t)(v >> 32) == seq;
            }
            if (__all(ok)) break;
            if (wall_clock64() - t0 > a.wait_ticks) {
                late = 1;
                break;
            }
            __builtin_amdgcn_s_sleep(2);
        }
        if (lane < FUSED_REC) s_rec[lane] = v;
        if (lane == 0) *s_flag = late;
    }
    __syncthreads();
    const bool late = *s_flag != 0;
    if (late && threadIdx.x == 0) fused_late(a, seq);
    return !late;
}

// where routed expert k's bytes are, from the routing words: an HBM slot, the pinned
// store (absent), or nothing (an id outside the store contributes zero); cpu:
// the host computes it (absent, rank r among the absent experts in k order
// with r % den < num)
struct ExpertSrc {
    const uint8_t *base;
    bool absent, cpu;
};
// one routed expert in rank order (id, its table word as 16 bits): the
// source if it is rank k, else its count among the absent ranks before k
__device__ inline void expert_src_step(const ExpertArgs &x, int id, int slot16, bool is_k, int &absent_before,
                                       ExpertSrc &r) {
    const bool res = x.slot_pool && slot16 < x.n_slots;
    const bool absent = !res && x.host_store && id < x.n_experts;
    if (!is_k) {
        absent_before += absent;
        return;
    }
    r.absent = absent;
    r.cpu = x.cpu_den > 0 && absent && absent_before % x.cpu_den < x.cpu_num;
    r.base = res ? x.slot_pool + (size_t)slot16 * x.slot_bytes
                 : absent ? x.host_store + (size_t)id * x.expert_bytes : nullptr;
}
template <class Word>          // Word(kk): the routing word of rank kk (sc_tag layout)
__device__ inline ExpertSrc expert_src(const ExpertArgs &x, int k, Word word) {
    if (k >= x.K) return {x.shared, false, false};
    int absent_before = 0;
    ExpertSrc r{nullptr, false, false};
    for (int kk = 0; kk <= k; ++kk) {
        const uint64_t w = word(kk);
        expert_src_step(x, (int)(w & 0xffffu), (int)((w >> 16) & 0xffffu), kk == k, absent_before, r);
    }
    return r;
}

// router row e: the canonical four-quarter dot, + the steering bias, posted
// as a tagged word in every copy of the logits
__device__ void fused_router(const FusedArgs &a, int e, uint32_t seq, uint8_t *smem) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    float *s_q = (float *)smem;
    const float part = router_quarter(a.r.W + (size_t)e * a.r.H, a.r.x, nullptr, a.r.H, wave, lane);
    if (lane == 0) s_q[wave] = part;
    __syncthreads();
    if (threadIdx.x <= FUSED_LOG_COPIES) {
        float acc = s_q[0];
#pragma unroll
        for (int q = 1; q < RL_WAVES; ++q) acc = acc + s_q[q];
        if (a.r.bias) acc = acc + a.r.bias[e];
        if (threadIdx.x < FUSED_LOG_COPIES)
            store_tagged(a.xlog + (size_t)threadIdx.x * MAX_E + e, tagged(seq, acc));
        else if (a.r.post)          // the host routes the token from these (CPU-assisted serving)
            __hip_atomic_store(&a.r.post->logit[e], tagged(seq, acc), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
    }
}

// CPU-assisted serving: Q8_K block b of x for the host, as tagged words (no
// wait for the stores: every word validates itself).  These workgroups come
// first in the launch, so x's codes reach the host before the logits.
__device__ void fused_post_q8x(const FusedArgs &a, int b, uint32_t seq) {
    if (threadIdx.x >= 64) return;
    const int lane = threadIdx.x;
    const float4 v = *(const float4 *)(a.r.x + QK * b + 4 * lane);
    const float xv[4] = {v.x, v.y, v.z, v.w};
    int q[4];
    float d;
    q8k_wave_vals(xv, lane, q, d);
    q8k_store_tagged_sys(q, d, a.r.post->q8x_words + (size_t)b * (Q8K_BYTES / 4), seq, lane);
}

// LDS of the in-workgroup routing
struct RouteScratch {
    int ids[16];              // the ids in rank order
    int slots[16];            // their table words
    float psel[16];           // their probabilities
    int late;
};
static_assert(FUSED_LDS_RS + sizeof(RouteScratch) <= FUSED_LDS, "routing LDS");
static_assert((2048 / QK) * Q8K_BYTES <= FUSED_LDS_W, "gate/up: the Q8_K of x (H = 2048)");

// The token's routing as every wave that needs it computes it: poll the
// posted logits (copy `copy`), then the softmax over 64-expert chunks (each
// chunk's sum in the canonical order, the chunks added in order), the prior,
// the score of each expert -- the same code on the same bits as
// route_select_kernel -- and the n_top best experts, best first, by n_top
// rounds of a wave-wide maximum of the scores (on a tie the lowest id, as
// the 64-bit keys order them), each round removing its expert.  Each round's
// expert is a uniform value: with want_k >= 0 its table word follows by a
// lane read and the source of rank want_k accumulates in scalars (src).
// With s, lane k keeps the id of rank k, and the ids, table words and
// probabilities go to s in one lane exchange after the last round.  false:
// the wait for the logits ran out.
template <int NC>
__device__ bool route_wave(const FusedArgs &a, uint32_t seq, int copy, int n_top, int want_k, RouteScratch *s,
                           ExpertSrc &src) {
    const RouteLaunch &r = a.r;
    const int lane = threadIdx.x & 63;
    float pr[NC];
    int32_t tbl[NC];
#pragma unroll
    for (int c = 0; c < NC; ++c) {
        pr[c] = r.prior ? r.prior[64 * c + lane] : 0.0f;
        tbl[c] = r.table[64 * c + lane];
    }
    const uint64_t *lsrc = a.xlog + (size_t)copy * MAX_E;
    uint64_t v[NC];
    bool ok[NC];
#pragma unroll
    for (int c = 0; c < NC; ++c) ok[c] = false;
    const uint64_t t0 = wall_clock64();
    for (;;) {
        bool all = true;
#pragma unroll
        for (int c = 0; c < NC; ++c)
            if (!ok[c]) v[c] = load_tagged(lsrc + 64 * c + lane);
#pragma unroll
        for (int c = 0; c < NC; ++c) {
            if (!ok[c]) ok[c] = (uint32_t)(v[c] >> 32) == seq;
            all = all && ok[c];
        }
        if (__all(all)) break;
        if (wall_clock64() - t0 > a.wait_ticks) return false;
        __builtin_amdgcn_s_sleep(1);
    }
    // a chain of dependent cross-lane steps on which the workgroup waits:
    // ahead of the other workgroups' dot products on this SIMD
    __builtin_amdgcn_s_setprio(3);
    float l[NC], ex[NC], p[NC];
    float m = 0.0f;
#pragma unroll
    for (int c = 0; c < NC; ++c) {
        l[c] = __uint_as_float((uint32_t)v[c]);
        const float mc = wave_max(l[c]);
        m = c == 0 ? mc : fmaxf(m, mc);
    }
    float sum = 0.0f;
#pragma unroll
    for (int c = 0; c < NC; ++c) {
        ex[c] = canon_expf(l[c] - m);
        const float cs = wave_sum_canon(ex[c]);
        sum = c == 0 ? cs : sum + cs;
    }
    uint32_t u[NC];
#pragma unroll
    for (int c = 0; c < NC; ++c) {
        p[c] = ex[c] / sum;
        u[c] = sel_bits(!r.prior ? p[c] : (r.prior_on_logits ? l[c] + pr[c] : p[c] + pr[c]));
    }
    int my_id = 0;                          // lane k < n_top: the id of rank k
    int absent_before = 0;
    for (int k = 0; k < n_top; ++k) {
        uint32_t mx = u[0];
#pragma unroll
        for (int c = 1; c < NC; ++c) mx = max(mx, u[c]);
        mx = wave_max_u32_bcast(mx);
        int id = -1;
#pragma unroll
        for (int c = 0; c < NC; ++c) {
            const uint64_t b = __ballot(u[c] == mx);
            if (id < 0 && b) id = 64 * c + (int)__builtin_ctzll(b);
        }
#pragma unroll
        for (int c = 0; c < NC; ++c)
            if (64 * c + lane == id) u[c] = 0;                // below every score
        if (s) my_id = lane == k ? id : my_id;
        if (want_k >= 0) {
            int32_t slot = 0;
#pragma unroll
            for (int c = 0; c < NC; ++c)
                if ((id >> 6) == c) slot = __builtin_amdgcn_readlane(tbl[c], id & 63);
            expert_src_step(a.x, id, (int)(uint16_t)slot, k == want_k, absent_before, src);
        }
    }
    if (s) {
        int32_t slot = 0;
        float pk = 0.0f;
#pragma unroll
        for (int c = 0; c < NC; ++c) {
            const int32_t t = __shfl(tbl[c], my_id & 63);
            const float q = __shfl(p[c], my_id & 63);
            if ((my_id >> 6) == c) {
                slot = t;
                pk = q;
            }
        }
        if (lane < n_top) {
            s->ids[lane] = my_id;
            s->slots[lane] = slot;
            s->psel[lane] = pk;
        }
    }
    __builtin_amdgcn_s_setprio(0);
    return true;
}
template <int NC>
__device__ bool route_wave(const FusedArgs &a, uint32_t seq, int copy, int n_top, int want_k, RouteScratch *s) {
    ExpertSrc unused{nullptr, false, false};
    return route_wave<NC>(a, seq, copy, n_top, want_k, s, unused);
}
// every wave routes the token itself (same code, same bits): no hand-over
// of the routing between waves
__device__ bool route_in_wave(const FusedArgs &a, uint32_t seq, int copy, int n_top, int want_k, ExpertSrc &src) {
    switch (a.r.E >> 6) {
    case 1: return route_wave<1>(a, seq, copy, n_top, want_k, nullptr, src);
    case 2: return route_wave<2>(a, seq, copy, n_top, want_k, nullptr, src);
    case 3: return route_wave<3>(a, seq, copy, n_top, want_k, nullptr, src);
    default: return route_wave<4>(a, seq, copy, n_top, want_k, nullptr, src);
    }
}
// wave 0 routes into s, one barrier hands it to the workgroup; false: the
// wait for the logits ran out (the caller reports it)
__device__ bool fused_route(const FusedArgs &a, uint32_t seq, int copy, RouteScratch *s, int n_top) {
    if ((threadIdx.x >> 6) == 0) {
        bool ok;
        switch (a.r.E >> 6) {
        case 1: ok = route_wave<1>(a, seq, copy, n_top, -1, s); break;
        case 2: ok = route_wave<2>(a, seq, copy, n_top, -1, s); break;
        case 3: ok = route_wave<3>(a, seq, copy, n_top, -1, s); break;
        default: ok = route_wave<4>(a, seq, copy, n_top, -1, s); break;
        }
        if ((threadIdx.x & 63) == 0) s->late = !ok;
    }
    __syncthreads();
    return !s->late;
}

// the selection's outputs: ids, gate weights, slots, the host's post and the
// routing record the down and combine workgroups read
__device__ void fused_select(const FusedArgs &a, uint32_t seq, uint8_t *smem) {
    const RouteLaunch &r = a.r;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    RouteScratch *s = (RouteScratch *)(smem + FUSED_LDS_RS);
    int *s_slot = (int *)smem;
    float *s_w = (float *)(s_slot + 16);
    if (!fused_route(a, seq, 0, s, r.K)) {
        if (tid == 0) fused_late(a, seq);
        return;
    }
    if (wave == 0) {
        float ws = 0.0f;                // the routed probabilities' sum, in rank order
        for (int k = 0; k < r.K; ++k) ws = ws + s->psel[k];
        if (lane < r.K) {
            const int id = s->ids[lane];
            const int slot = s->slots[lane];
            const float w = s->psel[lane] / ws;
            r.ids[lane] = id;
            r.w[lane] = w;
            r.slots[lane] = slot;
            s_slot[lane] = slot;
            s_w[lane] = w;
            if (r.post)
                __hip_atomic_store(&r.post->tag[lane], sc_tag(seq, slot, id), __ATOMIC_RELAXED,
                                   __HIP_MEMORY_SCOPE_SYSTEM);
        }
    }
    __syncthreads();
    const int *ids = s->ids;
    for (int i = tid; i < FUSED_COPIES * FUSED_REC; i += 256) {
        const int k = i % FUSED_REC;
        if (k < r.K) store_tagged(a.rec + i, sc_tag(seq, s_slot[k], ids[k]));
        else if (k >= 16 && k - 16 < r.K) store_tagged(a.rec + i, tagged(seq, s_w[k - 16]));
    }
}

// Gate/up rows of routed expert k (or of the shared expert, which needs no
// routing), 16 rows a workgroup, 4 a wave: lane (m, i, b) -- m gate or up,
// row i, super-block b -- holds one whole Q4_K super-block (144 bytes, 256
// weights) and its integer dots against the Q8_K of x (in LDS, quantized by
// the workgroup before the routing is known).  The row's eight terms are
// added in super-block order by a lane-to-lane scan, scale term then min
// term, as the CPU vec_dot accumulates them; h = silu(gate) * up is posted as
// a tagged word.
__device__ void fused_gateup(const FusedArgs &a, int g, uint32_t seq, uint8_t *smem) {
    const ExpertArgs &x = a.x;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int per = x.I / FUSED_GU_TILE;
    const int k = g / per, tile = g - k * per;
    uint8_t *s_q8x = smem;                                          // [H / 256][292]
    for (int b = wave; b < x.H / QK; b += 4) {         // the bytes route_logits_kernel writes
        const float4 v = *(const float4 *)(a.r.x + QK * b + 4 * lane);
        const float xv[4] = {v.x, v.y, v.z, v.w};
        int q[4];
        float d;
        q8k_wave_vals(xv, lane, q, d);
        q8k_store(q, d, s_q8x + b * Q8K_BYTES, lane);
    }
    __syncthreads();                                   // the Q8_K of x, for every wave
    ExpertSrc src{x.shared, false, false};
    if (k < x.K) {
        if (!route_in_wave(a, seq, g % FUSED_LOG_COPIES, k + 1, k, src)) {
            if (lane == 0) fused_late(a, seq);
            return;
        }
        if (src.cpu) return;
    }
    const int b = lane & 7, i = (lane >> 3) & 3;
    const bool is_gate = lane < 32;
    const size_t rb = (size_t)(x.H / QK) * Q4K_BYTES;     // 1152 at H = 2048
    const int row = tile * FUSED_GU_TILE + wave * 4 + i;
    const size_t off = (size_t)(is_gate ? x.I : 0) * rb + (size_t)row * rb + (size_t)b * Q4K_BYTES;
    uint4 blk[9];
    if (src.base) {
        const uint4 *p = (const uint4 *)(src.base + off);
#pragma unroll
        for (int j = 0; j < 9; ++j) blk[j] = p[j];
        if (src.absent && x.stage) {          // the same bytes, same offsets, into the staging area
            uint4 *sp = (uint4 *)(x.stage + (size_t)k * x.stage_stride + off);
#pragma unroll
            for (int j = 0; j < 9; ++j) sp[j] = blk[j];
        }
    } else {
#pragma unroll
        for (int j = 0; j < 9; ++j) blk[j] = make_uint4(0, 0, 0, 0);
    }
    const uint8_t *xb = s_q8x + b * Q8K_BYTES;
    const float dx = *(const float *)xb;
    const int16_t *bs = (const int16_t *)(xb + 4 + QK);
    int32_t si = 0, mi = 0;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        int sl, ml, sh, mh;
        q4k_sm(blk[0], 2 * j, sl, ml);
        q4k_sm(blk[0], 2 * j + 1, sh, mh);
        const uint4 *xw = (const uint4 *)(xb + 4 + 64 * j);
        const uint4 xl0 = xw[0], xl1 = xw[1], xh0 = xw[2], xh1 = xw[3];
        const uint32_t xl[8] = {xl0.x, xl0.y, xl0.z, xl0.w, xl1.x, xl1.y, xl1.z, xl1.w};
        const uint32_t xh[8] = {xh0.x, xh0.y, xh0.z, xh0.w, xh1.x, xh1.y, xh1.z, xh1.w};
        const uint4 q0 = blk[1 + 2 * j], q1 = blk[2 + 2 * j];
        const uint32_t w[8] = {q0.x, q0.y, q0.z, q0.w, q1.x, q1.y, q1.z, q1.w};
        int32_t dl = 0, dh = 0;
#pragma unroll
        for (int t = 0; t < 8; ++t) {
            dl = sdot4(w[t] & 0x0F0F0F0Fu, xl[t], dl);
            dh = sdot4((w[t] >> 4) & 0x0F0F0F0Fu, xh[t], dh);
        }
        si += sl * dl + sh * dh;
        mi += ml * ((int)bs[4 * j] + (int)bs[4 * j + 1]) + mh * ((int)bs[4 * j + 2] + (int)bs[4 * j + 3]);
    }
    const float d = h2f_dev((uint16_t)(blk[0].x & 0xffff)) * dx;
    const float dm = h2f_dev((uint16_t)(blk[0].x >> 16)) * dx;
    const float t = d * (float)si, m = dm * (float)mi;
    // v = 0; v += t_0; v -= m_0; v += t_1; ...: lane b continues lane b - 1's sum
    float acc = (0.0f + t) - m;
#pragma unroll
    for (int sb = 1; sb < 8; ++sb) {
        const float prev = __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(acc), 0x111, 0xF, 0xF, false));
        if (b == sb) acc = (prev + t) - m;                         // row_shr:1 -- the lane below
    }
    const float upv = __shfl(acc, lane + 32, 64);                  // row i's up sum, for the gate lanes
    if (is_gate && b == 7)
        store_tagged(a.hx + (size_t)k * x.I + row, tagged(seq, acc / (1.0f + canon_expf(-acc)) * upv));
}

// FUSED_DN_TILE down rows of expert k, 8 per wave: the weights into LDS as
// soon as the routing is known; then h (posted by the gate/up workgroups) in
// Q8_K, the dots as down_kernel computes them, and the rows posted as tagged
// words (or, for the join kernel, stored to x.ypart)
template <int DT>
__device__ void fused_down(const FusedArgs &a, int g, uint32_t seq, uint8_t *smem) {
    const ExpertArgs &x = a.x;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int per = x.H / FUSED_DN_TILE;
    const int k = g / per, tile = g - k * per;
    uint8_t *s_wt = smem + wave * DN_LDS_ROWS;
    uint8_t *s_q8h = smem + FUSED_LDS_W;
    uint64_t *s_rec = (uint64_t *)(smem + FUSED_LDS_W + FUSED_LDS_Q8);
    int *s_flag = (int *)(s_rec + FUSED_REC);
    ExpertSrc src{x.shared, false, false};
    if (k < x.K) {
        // the selection's record (the down rows' weights are not needed
        // before h, and requested later they leave the memory system to the
        // gate/up rows first)
        if (!fused_record(a, g % FUSED_COPIES, seq, true, false, s_rec, s_flag)) return;
        src = expert_src(x, k, [s_rec](int kk) { return s_rec[kk]; });
        if (src.cpu) return;
    }
    const int nb = x.I / QK;
    const int rowb = nb * (DT == TYPE_Q6K ? Q6K_BYTES : Q4K_BYTES);
    const int r0 = tile * FUSED_DN_TILE + wave * 8;
    const int nvec = 8 * rowb / 16;                 // <= 315
    const size_t dn_off = 2ull * x.I * (x.H / QK) * Q4K_BYTES + (size_t)r0 * rowb;
    const uint4 *wsrc = src.base ? (const uint4 *)(src.base + dn_off) : nullptr;
    uint8_t *sb = src.absent && x.stage ? x.stage + (size_t)k * x.stage_stride + dn_off : nullptr;
    // The weights first.  Q4_K rows go straight into LDS (16 bytes a lane,
    // lane-contiguous), all by the last wave: a wave's loads return in the
    // order they were issued, so the waves that poll for h must not have
    // weights queued ahead of their polls.  Rows that are also staged pass
    // through registers, each wave its own 8; so do Q6_K rows, which LDS
    // holds at the padded block stride (q6k_rows_load).
    uint4 buf[5];
    Q6Rows q6;
    if (DT == TYPE_Q6K) {
        // each wave its own 8 rows, through registers into the padded layout
        q6k_rows_load(q6, (const uint8_t *)wsrc, 8 * nb, lane);
    } else if (wsrc && !sb) {
        if (wave == 3) {
            const uint4 *w0 = (const uint4 *)(src.base + 2ull * x.I * (x.H / QK) * Q4K_BYTES +
                                              (size_t)tile * FUSED_DN_TILE * rowb);
#pragma unroll
            for (int ww = 0; ww < 4; ++ww)
#pragma unroll
                for (int j = 0; j < 5; ++j) {
                    const int i = lane + 64 * j;
                    if (i < nvec)
                        __builtin_amdgcn_global_load_lds(
                            (const void *)(w0 + (size_t)ww * nvec + i),
                            (__attribute__((address_space(3))) void *)(smem + ww * DN_LDS_ROWS + 1024 * j), 16, 0, 0);
                }
        }
    } else if (wsrc) {
#pragma unroll
        for (int j = 0; j < 5; ++j) {
            const int i = lane + 64 * j;
            buf[j] = i < nvec ? wsrc[i] : make_uint4(0, 0, 0, 0);
        }
    }
    // h of expert k, block `wave`: its four words a lane, once each carries
    // seq.  Until then the wave polls only the last row of each of the
    // block's 16 gate/up tiles (16 words, not 256: thousands of waves poll
    // at once, and their reads share the memory system with the weights)
    if (wave < nb) {
        const uint64_t *hb = a.hx + (size_t)k * x.I + QK * wave;
        const uint64_t *hp = hb + 4 * lane;
        uint64_t hv[4] = {0, 0, 0, 0};
        uint32_t pending = 0xfu;
        int late = 0;
        const uint64_t t0 = wall_clock64();
        bool seen = lane >= QK / FUSED_GU_TILE;
        for (;;) {
            if (!seen) seen = (uint32_t)(load_tagged(hb + FUSED_GU_TILE * lane + FUSED_GU_TILE - 1) >> 32) == seq;
            if (__all(seen)) break;
            if (wall_clock64() - t0 > a.wait_ticks) break;
            __builtin_amdgcn_s_sleep(1);
        }
        for (;;) {
#pragma unroll
            for (int j = 0; j < 4; ++j)
                if (pending >> j & 1u) hv[j] = load_tagged(hp + j);
#pragma unroll
            for (int j = 0; j < 4; ++j)
                if ((pending >> j & 1u) && (uint32_t)(hv[j] >> 32) == seq) pending &= ~(1u << j);
            if (__all(pending == 0)) break;
            if (wall_clock64() - t0 > a.wait_ticks) {
                late = 1;
                break;
            }
            __builtin_amdgcn_s_sleep(1);
        }
        if (late && lane == 0) fused_late(a, seq);
        const float xv[4] = {__uint_as_float((uint32_t)hv[0]), __uint_as_float((uint32_t)hv[1]),
                             __uint_as_float((uint32_t)hv[2]), __uint_as_float((uint32_t)hv[3])};
        int q[4];
        float d;
        q8k_wave_vals(xv, lane, q, d);
        q8k_store(q, d, s_q8h + wave * Q8K_BYTES, lane);
    }
    if (DT == TYPE_Q6K) {
        if (wsrc) q6k_rows_store(q6, s_wt, sb, 8 * nb, lane);
    } else if (wsrc && !sb) {
        if (wave == 3) __builtin_amdgcn_s_waitcnt(0x0f70);      // vmcnt(0): the weights have landed in LDS
    } else if (wsrc) {
        uint4 *dst = (uint4 *)s_wt;
#pragma unroll
        for (int j = 0; j < 5; ++j) {
            const int i = lane + 64 * j;
            if (i < nvec) dst[i] = buf[j];
        }
        uint4 *sd = (uint4 *)sb;
#pragma unroll
        for (int j = 0; j < 5; ++j) {
            const int i = lane + 64 * j;
            if (i < nvec) sd[i] = buf[j];
        }
    }
    __syncthreads();                // the Q8_K blocks of h and every wave's weights
    const float y = wsrc ? down_rows_dot<DT>(s_wt, s_q8h, nb, nb * (DT == TYPE_Q6K ? Q6K_PAD : Q4K_BYTES), lane) : 0.0f;
    if ((lane & 7) == 0) {
        const int row = r0 + (lane >> 3);
        if (x.ypart) x.ypart[(size_t)k * x.H + row] = y;
        else store_tagged(a.yx + (size_t)k * x.H + row, tagged(seq, y));
    }
}

// one output row: out = sum_k w_k y_k in k order, then the shared expert
// (weight 1), as down_kernel's combine adds them
__device__ void fused_combine_row(const FusedArgs &a, int row, uint32_t seq, const uint64_t *s_rec) {
    const ExpertArgs &x = a.x;
    const int kt = x.K + x.n_shared;
    // every row word requested in each round (one round trip, not one per
    // expert); a round re-reads only the words not yet valid
    constexpr int MK = 17;
    uint64_t v[MK];
    uint32_t pending = (1u << kt) - 1u;
    int late = 0;
    const uint64_t t0 = wall_clock64();
    for (;;) {
#pragma unroll
        for (int k = 0; k < MK; ++k)
            if (pending >> k & 1u) v[k] = load_tagged(a.yx + (size_t)k * x.H + row);
#pragma unroll
        for (int k = 0; k < MK; ++k)
            if ((pending >> k & 1u) && (uint32_t)(v[k] >> 32) == seq) pending &= ~(1u << k);
        if (!pending) break;
        if (wall_clock64() - t0 > a.wait_ticks) {
            late = 1;
            break;
        }
        __builtin_amdgcn_s_sleep(1);
    }
    if (late) fused_late(a, seq);
    float y[MK];
#pragma unroll
    for (int k = 0; k < MK; ++k) y[k] = __uint_as_float((uint32_t)v[k]);
    float acc = __uint_as_float((uint32_t)s_rec[16]) * y[0];
    for (int k = 1; k < x.K; ++k) acc = acc + __uint_as_float((uint32_t)s_rec[16 + k]) * y[k];
    if (x.n_shared) acc = acc + y[x.K];
    // publishing: written through to memory (performed before the workgroup
    // counts itself done), so a reader on another stream or engine sees the
    // row once the host has the done word, before the launch has retired
    if (a.pub) __hip_atomic_store(x.out + row, acc, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
    else x.out[row] = acc;
}

// The layer's last combine workgroup publishes the routed experts (the routing
// record's words, (seq << 32) | slot << 16 | id) as tagged words in mapped host
// memory, and in the token's last layer the late word, tagged too: each word
// carries the token's number, so the host needs no ordering between them and
// no fence is spent here.  The slots keep the record's 16 bits (a table word
// below 2^16: a slot, or the slot count for an absent expert).
__device__ void fused_publish(const FusedArgs &a, uint32_t seq, const uint64_t *s_rec) {
    __syncthreads();                        // this workgroup's output rows are written
    if (threadIdx.x != 0) return;
    const int n_comb = (a.x.H + 255) / 256;
    uint64_t old = __hip_atomic_load(a.pub_ctr, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT), nv;
    do {
        nv = (uint32_t)(old >> 32) == seq ? old + 1 : ((uint64_t)seq << 32) | 1u;
    } while (!__hip_atomic_compare_exchange_strong(a.pub_ctr, &old, nv, __ATOMIC_ACQ_REL, __ATOMIC_RELAXED,
                                                   __HIP_MEMORY_SCOPE_AGENT));
    if ((uint32_t)nv != (uint32_t)n_comb) return;
    const int K = a.x.K;
    for (int k = 0; k < K; ++k)
        __hip_atomic_store(a.pub + (size_t)a.pub_layer * K + k, s_rec[k], __ATOMIC_RELAXED,
                           __HIP_MEMORY_SCOPE_SYSTEM);
    if (a.pub_done) {
        const uint32_t late = __hip_atomic_load(a.err, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __hip_atomic_store(a.pub + (size_t)a.pub_L * K, ((uint64_t)seq << 32) | late, __ATOMIC_RELAXED,
                           __HIP_MEMORY_SCOPE_SYSTEM);
    }
}

// 256 output rows of the combine, then (publishing) the count of finished
// combine workgroups
__device__ void fused_combine(const FusedArgs &a, int c, uint32_t seq, uint8_t *smem) {
    uint64_t *s_rec = (uint64_t *)(smem + FUSED_LDS_W + FUSED_LDS_Q8);
    int *s_flag = (int *)(s_rec + FUSED_REC);
    if (!fused_record(a, c % FUSED_COPIES, seq, a.pub != nullptr, true, s_rec, s_flag)) return;
    const int row = c * 256 + (int)threadIdx.x;
    if (row < a.x.H) fused_combine_row(a, row, seq, s_rec);
    if (a.pub) fused_publish(a, seq, s_rec);
}

template <int DT>
__global__ __launch_bounds__(256) void fused_kernel(FusedArgs a) {
    __shared__ __attribute__((aligned(16))) uint8_t smem[FUSED_LDS];
    const uint32_t seq = a.r.seq ? *a.r.seq : a.r.seq_val;
    const int E = a.r.E;
    const int kt = a.x.K + a.x.n_shared;
    const int nG = kt * (a.x.I / FUSED_GU_TILE), nD = kt * (a.x.H / FUSED_DN_TILE);
    int g = (int)blockIdx.x;
    if (a.r.post) {
        if (g < a.r.H / QK) {
            fused_post_q8x(a, g, seq);
            return;
        }
        g -= a.r.H / QK;
    }
    if (g < E) {
        fused_router(a, g, seq, smem);
    } else if (g == E) {
        fused_select(a, seq, smem);
    } else if ((g -= E + 1) < nG) {
        fused_gateup(a, g, seq, smem);
    } else if ((g -= nG) < nD) {
        fused_down<DT>(a, g, seq, smem);
    } else {
        fused_combine(a, g - nD, seq, smem);
    }
}

// ---------------------------------------------------------------------------
// synthetic data on the device
__global__ void synth_experts_kernel(uint64_t seed, int layer, int e0, int n_experts, int H, int I,
                                     int down_type, float sigma, uint8_t *out, uint64_t stride) {
    const synth::ExpertShape sh{H, I, down_type};
    const uint64_t nblk = (uint64_t)sh.n_blocks();
    const uint64_t t = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (t >= nblk * (uint64_t)n_experts) return;
    const int e = (int)(t / nblk), blk = (int)(t % nblk);
    synth::expert_block(seed, layer, e0 + e, sh, blk, sigma, out + (uint64_t)e * stride + sh.block_offset(blk));
}

__global__ void synth_vec_kernel(uint64_t seed, int kind, int a0, int na, int b0, int nb, int n,
                                 float sigma, float *out) {
    const uint64_t t = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
    const uint64_t total = (uint64_t)na * nb * n;
    if (t >= total) return;
    const int i = (int)(t % n);
    const int bb = (int)((t / n) % nb);
    const int aa = (int)(t / ((uint64_t)n * nb));
    out[t] = synth::vec_value(seed, kind, a0 + aa, b0 + bb, i, sigma);
}

// ---------------------------------------------------------------------------
// launchers (shapes were checked by the caller).  With events, the launch
// goes through hipExtLaunchKernelGGL: the dispatch itself stamps ev0/ev1 at
// the start and end of the kernel's execution (the window a profiler reports),
// with no host or queue latency inside it.
template <typename F, typename... A>
static hipError_t launch(F k, dim3 grid, dim3 block, hipStream_t st, hipEvent_t ev0, hipEvent_t ev1, A... args) {
    if (ev0) hipExtLaunchKernelGGL(k, grid, block, 0, st, ev0, ev1, 0, args...);
    else hipLaunchKernelGGL(k, grid, block, 0, st, args...);
    return hipGetLastError();
}

hipError_t launch_route(const RouteLaunch &l, hipStream_t st, hipEvent_t *ev) {
    RouteArgs a;
    a.W = l.W; a.x = l.x; a.bias = l.bias; a.prior = l.prior; a.table = l.table; a.dummy = l.dummy;
    a.prior_on_logits = l.prior_on_logits;
    a.E = l.E; a.H = l.H; a.K = l.K;
    a.logits = l.logits; a.counter = l.counter; a.ids = l.ids; a.w = l.w; a.slots = l.slots;
    a.probs = l.probs; a.q8x = l.q8x; a.logits_in = l.logits_in;
    a.post = l.post; a.seq = l.seq; a.seq_val = l.seq_val ? l.seq_val : 1u;
    a.an = l.an; a.ak = l.ak;
    for (int t = 0; t < 2; ++t) {
        a.aW[t] = l.aW[t]; a.ar[t] = l.ar[t]; a.atbl[t] = l.atbl[t];
        a.adummy[t] = l.adummy[t]; a.atarget[t] = l.atarget[t];
    }
    a.alayer = l.alayer; a.alog = l.alog; a.apost = l.apost; a.fresh = l.fresh;
    if (l.logits_in)
        return launch(route_select_kernel, dim3((unsigned)l.n_tok), dim3(256), st, ev ? ev[2] : nullptr,
                      ev ? ev[3] : nullptr, a);
    const hipError_t e = launch(route_logits_kernel, dim3((unsigned)l.E * (unsigned)(1 + (l.apost ? l.an : 0)),
                                                         (unsigned)l.n_tok),
                                dim3(64 * RL_WAVES), st, ev ? ev[0] : nullptr, ev ? ev[1] : nullptr, a);
    if (e != hipSuccess) return e;
    return launch(route_select_kernel, dim3((unsigned)l.n_tok), dim3(256), st, ev ? ev[2] : nullptr,
                  ev ? ev[3] : nullptr, a);
}

template <int SRC>
static hipError_t gateup_src(const ExpertArgs &a, hipStream_t st, hipEvent_t e0, hipEvent_t e1) {
    constexpr int R = 1;
    return launch(gateup_kernel<R, SRC>, dim3((unsigned)(a.I / (GU_WAVES * R)), (unsigned)(a.K + a.n_shared)),
                  dim3(64 * GU_WAVES), st,
                  e0, e1, a);
}

template <int SRC>
static hipError_t down_src(const ExpertArgs &a, hipStream_t st, hipEvent_t e0, hipEvent_t e1) {
    if (a.down_type == TYPE_Q6K)
        return launch(down_kernel<TYPE_Q6K, SRC>, dim3((unsigned)(a.H / DN_ROWS)), dim3(512), st, e0, e1, a);
    return launch(down_kernel<TYPE_Q4K, SRC>, dim3((unsigned)(a.H / DN_ROWS)), dim3(512), st, e0, e1, a);
}

hipError_t launch_gateup(const ExpertArgs &a, int src, hipStream_t st, hipEvent_t e0, hipEvent_t e1) {
    return src == SRC_HBM ? gateup_src<SRC_HBM>(a, st, e0, e1) : src == SRC_HOST ? gateup_src<SRC_HOST>(a, st, e0, e1)
                                                                                   : gateup_src<SRC_ALL>(a, st, e0, e1);
}

hipError_t launch_down(const ExpertArgs &a, int src, hipStream_t st, hipEvent_t e0, hipEvent_t e1) {
    return src == SRC_HBM ? down_src<SRC_HBM>(a, st, e0, e1) : src == SRC_HOST ? down_src<SRC_HOST>(a, st, e0, e1)
                                                                                 : down_src<SRC_ALL>(a, st, e0, e1);
}

// ---------------------------------------------------------------------------
// join after CPU-assisted serving.  One thread per workgroup waits for the
// host's answer: bounded by the 100 MHz wall clock, and ended early by
// SC_ABORT; a timeout is reported through resp->err and the rows are zero.
__global__ __launch_bounds__(256) void join_kernel(JoinArgs a) {
    __shared__ int s_ok;
    __shared__ int s_cpu[16];
    if (threadIdx.x < 16)
        s_cpu[threadIdx.x] = cpu_served(a.slots, a.ids, a.slot_pool, a.n_slots, a.host_store, a.n_experts, a.cpu_num,
                                        a.cpu_den, a.K, (int)threadIdx.x);
    __syncthreads();
    const int r = blockIdx.x * 256 + threadIdx.x;
    // the gate weights and the GPU's rows (an earlier kernel's: in memory)
    // are requested before the wait for the host, so that after it only the
    // host's rows cross PCIe
    constexpr int MK = 16;
    float y[MK], wk[MK];
    float ys = 0.0f;
    if (r < a.H) {
#pragma unroll
        for (int k = 0; k < MK; ++k)
            if (k < a.K) {
                wk[k] = a.w[k];
                y[k] = s_cpu[k] ? 0.0f : a.ypart[(size_t)k * a.H + r];
            }
        if (a.n_shared) ys = a.ypart[(size_t)a.K * a.H + r];
    }
    if (threadIdx.x == 0) {
        const uint32_t want = a.seq ? *a.seq : a.seq_val;
        const uint64_t t0 = wall_clock64();
        int ok = 0;
        // relaxed polls (system-scope loads bypass the caches), one acquire
        // once the answer is there: no cache invalidation per poll
        for (;;) {
            const uint32_t v = __hip_atomic_load(&a.resp->seq, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
            if (v == want) {
                __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "");    // system scope
                ok = 1;
                break;
            }
            if (v == SC_ABORT) {        // the host gave up: the token fails, never passes silently
                if (blockIdx.x == 0) __hip_atomic_store(&a.resp->err, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
                break;
            }
            if (wall_clock64() - t0 > a.timeout_ticks) {
                if (blockIdx.x == 0) __hip_atomic_store(&a.resp->err, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
                break;
            }
            __builtin_amdgcn_s_sleep(4);
        }
        s_ok = ok;
    }
    __syncthreads();
    if (r >= a.H) return;
    if (!s_ok) {
        a.out[r] = 0.0f;
        return;
    }
    // every host row's load issued before the first is used: one round trip
    // over PCIe (system scope: the host's rows bypass the caches)
#pragma unroll
    for (int k = 0; k < MK; ++k)
        if (k < a.K && s_cpu[k]) y[k] = __hip_atomic_load(a.hrows + (size_t)k * a.H + r, __ATOMIC_RELAXED,
                                                          __HIP_MEMORY_SCOPE_SYSTEM);
    float acc = wk[0] * y[0];
#pragma unroll
    for (int k = 1; k < MK; ++k)
        if (k < a.K) acc = acc + wk[k] * y[k];
    if (a.n_shared) acc = acc + ys;     // weight 1, after the routed experts
    a.out[r] = acc;
}

// the serving channel's self-test: one workgroup, rounds in order
__global__ __launch_bounds__(256) void sc_selftest_kernel(ScSelfTestArgs a) {
    __shared__ int s_ok;
    for (int r = 0; r < a.n_rounds; ++r) {
        const uint32_t seq = a.seq0 + (uint32_t)r;
        const uint64_t tag = (uint64_t)seq << 32;
        for (int i = threadIdx.x; i < a.E; i += blockDim.x)
            __hip_atomic_store(&a.post->logit[i], tag | sc_test_word(seq, i, 0), __ATOMIC_RELAXED,
                               __HIP_MEMORY_SCOPE_SYSTEM);
        for (int i = threadIdx.x; i < a.n_q8_words; i += blockDim.x)
            __hip_atomic_store(&a.post->q8x_words[i], tag | sc_test_word(seq, i, 1), __ATOMIC_RELAXED,
                               __HIP_MEMORY_SCOPE_SYSTEM);
        if (threadIdx.x == 0) {
            const uint64_t t0 = wall_clock64();
            int ok = 1;
            while (__hip_atomic_load(&a.resp->seq, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM) != seq) {
                if (wall_clock64() - t0 > a.timeout_ticks) {
                    ok = 0;
                    break;
                }
                __builtin_amdgcn_s_sleep(2);
            }
            if (ok) __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "");     // system scope
            s_ok = ok;
        }
        __syncthreads();
        if (!s_ok) {
            if (threadIdx.x == 0)
                __hip_atomic_fetch_add(a.bad, (uint32_t)(a.n_rounds - r), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            return;
        }
        int wrong = 0;
        for (int i = threadIdx.x; i < a.H; i += blockDim.x) {
            const float v = __hip_atomic_load(a.rows + i, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
            wrong |= __float_as_uint(v) != (sc_test_word(seq, i, 2) & 0x3fffffffu);
        }
        wrong = __syncthreads_or(wrong);
        if (wrong && threadIdx.x == 0) __hip_atomic_fetch_add(a.bad, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
}

hipError_t launch_sc_selftest(const ScSelfTestArgs &a, hipStream_t st) {
    hipLaunchKernelGGL(sc_selftest_kernel, dim3(1), dim3(256), 0, st, a);
    return hipGetLastError();
}

hipError_t launch_join(const JoinArgs &a, hipStream_t st) {
    hipLaunchKernelGGL(join_kernel, dim3((unsigned)((a.H + 255) / 256)), dim3(256), 0, st, a);
    return hipGetLastError();
}

hipError_t launch_fused(const FusedArgs &a, hipStream_t st, hipEvent_t e0, hipEvent_t e1) {
    const int kt = a.x.K + a.x.n_shared;
    const unsigned n = (unsigned)((a.r.post ? a.r.H / QK : 0) + a.r.E + 1 + kt * (a.x.I / FUSED_GU_TILE) +
                                  kt * (a.x.H / FUSED_DN_TILE) + (a.x.ypart ? 0 : a.x.H / 256));
    if (a.x.down_type == TYPE_Q6K) return launch(fused_kernel<TYPE_Q6K>, dim3(n), dim3(256), st, e0, e1, a);
    return launch(fused_kernel<TYPE_Q4K>, dim3(n), dim3(256), st, e0, e1, a);
}

hipError_t launch_experts(const ExpertArgs &a, hipStream_t st) {
    const hipError_t e = launch_gateup(a, SRC_ALL, st, nullptr, nullptr);
    return e != hipSuccess ? e : launch_down(a, SRC_ALL, st, nullptr, nullptr);
}

// ---------------------------------------------------------------------------
// streaming read, for the size-matched read ceiling the decode kernels are
// compared with: each thread issues 8 independent 16-byte loads, xors them,
// one word per workgroup
constexpr int SR_U = 8;
__global__ __launch_bounds__(256) void stream_read_kernel(const uint4 *__restrict__ p, uint64_t n16, uint32_t *out) {
    const uint64_t base = (uint64_t)blockIdx.x * 256 * SR_U + threadIdx.x;
    uint4 v[SR_U];
#pragma unroll
    for (int i = 0; i < SR_U; ++i) {
        const uint64_t j = base + (uint64_t)i * 256;
        v[i] = j < n16 ? p[j] : make_uint4(0, 0, 0, 0);
    }
    uint32_t a = 0;
#pragma unroll
    for (int i = 0; i < SR_U; ++i) a ^= v[i].x ^ v[i].y ^ v[i].z ^ v[i].w;
    __shared__ uint32_t s[256];
    s[threadIdx.x] = a;
    __syncthreads();
    if (threadIdx.x == 0) {
        uint32_t t = 0;
        for (int i = 0; i < 256; ++i) t ^= s[i];
        out[blockIdx.x] = t;
    }
}

unsigned stream_read_blocks(uint64_t bytes) { return (unsigned)((bytes / 16 + 256 * SR_U - 1) / (256 * SR_U)); }

hipError_t launch_stream_read(const void *p, uint64_t bytes, uint32_t *out, hipStream_t st, hipEvent_t e0,
                              hipEvent_t e1) {
    return launch(stream_read_kernel, dim3(stream_read_blocks(bytes)), dim3(256), st, e0, e1, (const uint4 *)p,
                  (uint64_t)(bytes / 16), out);
}

hipError_t launch_synth_experts(uint64_t seed, int layer, int e0, int n_experts, int H, int I, int down_type,
                                float sigma, uint8_t *out, uint64_t stride, hipStream_t st) {
    const synth::ExpertShape sh{H, I, down_type};
    const uint64_t total = (uint64_t)sh.n_blocks() * (uint64_t)n_experts;
    const unsigned blocks = (unsigned)((total + 127) / 128);
    hipLaunchKernelGGL(synth_experts_kernel, dim3(blocks), dim3(128), 0, st, seed, layer, e0, n_experts, H, I,
                       down_type, sigma, out, stride);
    return hipGetLastError();
}

hipError_t launch_synth_vec(uint64_t seed, int kind, int a0, int na, int b0, int nb, int n, float sigma,
                            float *out, hipStream_t st) {
    const uint64_t total = (uint64_t)na * nb * n;
    const unsigned blocks = (unsigned)((total + 255) / 256);
    hipLaunchKernelGGL(synth_vec_kernel, dim3(blocks), dim3(256), 0, st, seed, kind, a0, na, b0, nb, n, sigma, out);
    return hipGetLastError();
}

}  // namespace mp
