// mp_batched.hip -- gfx950 kernels of the batched MoE layer (prefill chunks and
// decode at batch > 1).
//
//   dispatch_kernel      per-expert histogram, exclusive scan and the stable
//                        permutation of (token, k) pairs (one workgroup)
//   quant_rows_kernel    Q8_K of rows (x per token) into the form the matrix
//                        cores consume: the int8 values as fp16 codes, the
//                        block scale, and the 16-value group sums as fp16 --
//                        all exact
//   grouped_q4_kernel    per (64-row tile, expert): the expert's Q4_K rows
//                        against the activations of every pair dispatched to
//                        it, on MFMA 16x16x32 f16; up and gate as one 2I-row
//                        matrix (the expert's [up | gate] layout), and Q4_K
//                        down with the pair's gate weight, scattered to the
//                        pair's row
//   grouped_q6_kernel    the same for a Q6_K down matrix
//   swiglu_quant_kernel  h = silu(gate) * up, and its Q8_K
//   combine_kernel       out[t] = sum over k of the weighted rows, k in order
//
// Exact integer products on fp16 matrix cores.  A Q4_K weight is
// d*sc*q - dmin*m with q a nibble and sc, m six-bit.  The B operand holds sc*q
// (<= 945, an integer fp16 represents exactly: 11-bit significand; bf16's 8 bits
// cannot), the A operand the Q8_K integers of the activation (|q8| <= 127,
// exact).  Each 128-value half of a 256-value super-block accumulates in fp32
// exactly (below 2^24), and the halves add once: the block's integer sum
// sum_j sc_j * sum_i q_i q8_i of ggml's vec_dot_q4_K_q8_K rounded once, as its
// (float)sumi.  The min
// term sum_j m_j * bsum_j is a second, 16-deep MFMA of the six-bit mins
// against the Q8_K group sums (|bsum16| <= 2032, exact).  fp32 appears only
// where ggml has it, in ggml's order: y += (d*dx)*sumi; y -= (dmin*dx)*summ per
// super-block, so a row's value is the CPU chain's bit for bit.  Q6_K weights
// are (q - 32) * sc with an int8 sc, split into two exact products (below).
//
// Every MFMA pairs the k-th element of lane group g of A with the k-th element
// of lane group g of B, so the order of the K elements inside one instruction
// is free: each lane feeds the 8 weights its own 16-byte load decodes, and the
// activation rows are read at the same positions.
#include <hip/hip_ext.h>
#include <hip/hip_runtime.h>

#include <mutex>

#include "mp_device.h"
#include "mp_format.h"
#include "mp_internal.h"

namespace mp {

typedef _Float16 half4_t __attribute__((ext_vector_type(4)));
typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef float float4_t __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) void lptr_t;

// ---------------------------------------------------------------------------
// dispatch: ids [P] (P = n_tok * K, pair i = t*K + k) -> counts[E], offsets[E+1],
// perm[offsets[e] + r] = i of the r-th pair routed to e in pair order.
// Pass 1 counts with LDS atomics (order-free) and one wave turns the counts
// into offsets with a prefix sum (lane l holds experts 4l .. 4l+3); pass 2
// places 64-pair chunks: lanes holding the same id find each other with 8
// ballots (one per id bit), their rank inside the chunk is a popcount, and a
// per-expert scan over the chunks of the pass (continuing a running count)
// gives each chunk's base.
constexpr int DSP_CHUNKS = 64;
static_assert(MAX_E <= 256, "4 experts a lane in the offsets' prefix sum");

// inclusive prefix sum over the 64 lanes of a wave
__device__ inline int wave_incl_sum(int v, int lane) {
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) {
        const int t = __shfl_up(v, d, 64);
        if (lane >= d) v += t;
    }
    return v;
}

__global__ __launch_bounds__(1024) void dispatch_kernel(const int32_t *ids, int P, int E, int32_t *counts,
                                                        int32_t *offsets, int32_t *perm) {
    __shared__ int s_off[MAX_E + 1];
    __shared__ int s_run[MAX_E];
    __shared__ uint16_t s_c[DSP_CHUNKS][MAX_E];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    for (int e = tid; e < E; e += blockDim.x) { s_off[e] = 0; s_run[e] = 0; }
    __syncthreads();
    for (int i = tid; i < P; i += blockDim.x) {
        const int e = ids[i];
        if (e >= 0 && e < E) atomicAdd(&s_off[e], 1);
    }
    __syncthreads();
    if (wave == 0) {
        int c[4], sum = 0;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int e = 4 * lane + j;
            c[j] = e < E ? s_off[e] : 0;
            sum += c[j];
        }
        const int incl = wave_incl_sum(sum, lane);
        int acc = incl - sum;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int e = 4 * lane + j;
            if (e < E) {
                counts[e] = c[j];
                offsets[e] = acc;
                s_off[e] = acc;
            }
            acc += c[j];
        }
        if (lane == 63) offsets[E] = incl;
    }
    __syncthreads();
    const int nwaves = blockDim.x >> 6;
    for (int base = 0; base < P; base += DSP_CHUNKS * 64) {
        const int nc = min(DSP_CHUNKS, (P - base + 63) / 64);      // chunks holding pairs
        for (int i = tid; i < nc * E; i += blockDim.x) s_c[i / E][i % E] = 0;
        __syncthreads();
        int my_e[DSP_CHUNKS / 16], my_r[DSP_CHUNKS / 16];
        for (int j = 0, c = wave; c < DSP_CHUNKS; ++j, c += nwaves) {
            if (c >= nc) break;
            const int i = base + 64 * c + lane;
            const int e = i < P ? ids[i] : -1;
            const bool valid = e >= 0 && e < E;
            uint64_t m = __ballot(valid);
#pragma unroll
            for (int b = 0; b < 8; ++b) {
                const bool bit = (e >> b) & 1;
                const uint64_t bb = __ballot(valid && bit);
                m &= bit ? bb : ~bb;
            }
            const int r = __popcll(m & ((1ull << lane) - 1ull));
            if (valid && r == 0) s_c[c][e] = (uint16_t)__popcll(m);
            my_e[j] = valid ? e : -1;
            my_r[j] = r;
        }
        __syncthreads();
        for (int e = tid; e < E; e += blockDim.x) {
            int run = s_run[e];
#pragma unroll 16
            for (int c = 0; c < nc; ++c) {
                const int v = s_c[c][e];
                s_c[c][e] = (uint16_t)run;
                run += v;
            }
            s_run[e] = run;
        }
        __syncthreads();
        for (int j = 0, c = wave; c < DSP_CHUNKS; ++j, c += nwaves) {
            if (c >= nc) break;
            const int e = my_e[j];
            if (e >= 0) perm[s_off[e] + s_c[c][e] + my_r[j]] = base + 64 * c + lane;
        }
        __syncthreads();
    }
}

// ---------------------------------------------------------------------------
// Q8_K rows for the matrix cores: one wavefront per (row, 256-value block)
__device__ inline uint32_t h16(int v) { return (uint32_t)__builtin_bit_cast(uint16_t, (_Float16)(float)v); }

// the wave's 4 values per lane -> fp16 codes, block scale and group sums
__device__ inline void q8_rows_out(const float xv[4], int lane, size_t off, size_t row, int b, int n,
                                   uint16_t *q16, float *dx, uint16_t *bs16) {
    int q[4];
    float d;
    q8k_wave_vals(xv, lane, q, d);
    const int gs = q8k_group_sum(q);
    uint2 o;
    o.x = h16(q[0]) | (h16(q[1]) << 16);
    o.y = h16(q[2]) | (h16(q[3]) << 16);
    *(uint2 *)(q16 + off) = o;
    if ((lane & 3) == 0) bs16[row * (n / 16) + b * 16 + (lane >> 2)] = (uint16_t)h16(gs);
    if (lane == 0) dx[row * (n / QK) + b] = d;
}

__global__ __launch_bounds__(256) void quant_rows_kernel(const void *src, int bf16, int n_rows, int n,
                                                         uint16_t *q16, float *dx, uint16_t *bs16) {
    const int lane = threadIdx.x & 63;
    const int nb = n / QK;
    const int64_t blk = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (blk >= (int64_t)n_rows * nb) return;
    const int64_t row = blk / nb;
    const int b = (int)(blk % nb);
    const size_t off = (size_t)row * n + (size_t)b * QK + 4 * lane;
    float xv[4];
    if (bf16) {
        const uint2 v = *(const uint2 *)((const uint16_t *)src + off);
        xv[0] = bits_f32(v.x << 16);
        xv[1] = bits_f32(v.x & 0xffff0000u);
        xv[2] = bits_f32(v.y << 16);
        xv[3] = bits_f32(v.y & 0xffff0000u);
    } else {
        const float4 v = *(const float4 *)((const float *)src + off);
        xv[0] = v.x; xv[1] = v.y; xv[2] = v.z; xv[3] = v.w;
    }
    q8_rows_out(xv, lane, off, (size_t)row, b, n, q16, dx, bs16);
}

// SiLU with the canonical exp (the oracle evaluates the same function)
__device__ inline float silu_mul(float g, float u) { return g / (1.0f + canon_expf(-g)) * u; }

// h = silu(gate) * up from the up/gate rows y2 [P][2I] (up first), then its
// Q8_K: one wavefront per (pair, 256-value block); h itself to h_out if given
__global__ __launch_bounds__(256) void swiglu_quant_kernel(const float *y2, int P, int I, float *h_out, uint16_t *q16,
                                                           float *dx, uint16_t *bs16) {
    const int lane = threadIdx.x & 63;
    const int nb = I / QK;
    const int64_t blk = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (blk >= (int64_t)P * nb) return;
    const int64_t p = blk / nb;
    const int b = (int)(blk % nb);
    const float *yr = y2 + (size_t)p * 2 * I + (size_t)b * QK + 4 * lane;
    const float4 u = *(const float4 *)yr;
    const float4 g = *(const float4 *)(yr + I);
    const float hv[4] = {silu_mul(g.x, u.x), silu_mul(g.y, u.y), silu_mul(g.z, u.z), silu_mul(g.w, u.w)};
    const size_t off = (size_t)p * I + (size_t)b * QK + 4 * lane;
    if (h_out) *(float4 *)(h_out + off) = make_float4(hv[0], hv[1], hv[2], hv[3]);
    q8_rows_out(hv, lane, off, (size_t)p, b, I, q16, dx, bs16);
}

// ---------------------------------------------------------------------------
// grouped expert products

__device__ inline const uint8_t *grouped_expert(const GroupedArgs &a, int e) {
    if (a.host_mask && a.host_mask[e]) return nullptr;          // computed by the host
    if (a.table) {
        const int s = a.table[e];
        if (a.slot_pool && s >= 0 && s < a.n_slots) return a.slot_pool + (size_t)s * a.slot_bytes;
    }
    if (!a.store || e >= a.n_store) return nullptr;
    return a.store + (size_t)e * a.expert_bytes;
}

// 8 small unsigned bytes (two words) -> 8 fp16 holding 1024 + v: byte v under
// the exponent byte 0x64 (1024 has a unit last place up to 2048)
__device__ inline half8_t pack_1024(uint32_t w0, uint32_t w1) {
    const uint32_t K = 0x64646464u;
    uint4 r;
    r.x = __builtin_amdgcn_perm(K, w0, 0x04010400u);
    r.y = __builtin_amdgcn_perm(K, w0, 0x04030402u);
    r.z = __builtin_amdgcn_perm(K, w1, 0x04010400u);
    r.w = __builtin_amdgcn_perm(K, w1, 0x04030402u);
    return __builtin_bit_cast(half8_t, r);
}

__device__ inline half8_t splat8(_Float16 v) { return half8_t{v, v, v, v, v, v, v, v}; }

// (1024 + q) * sc - 1024 * sc = q * sc, one rounding of an exact value
__device__ inline half8_t q4_scaled(uint32_t w0, uint32_t w1, int sc) {
    const _Float16 s = (_Float16)(float)sc;
    const _Float16 nb = (_Float16)(float)(-1024 * sc);
    return __builtin_elementwise_fma(pack_1024(w0, w1), splat8(s), splat8(nb));
}

__device__ inline float4_t mfma32(half8_t a, half8_t b, float4_t c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}

// Q4_K lane layout.  Lane (n = lane & 15: row, h = lane >> 4) of a wave loads
// the 16-byte header and qs bytes 16h .. 16h+15 (group g_0 = h >> 1) and
// 64+16h .. 64+16h+15 (group g_1 = 2 + (h >> 1)) of each super-block: elements
// 16*(h & 1) .. +15 of sub-blocks 2g_L (low nibbles) and 2g_L + 1 (high).  MFMA
// i = 4L + 2*nibble + half multiplies 8 of them; the activation values at the
// same positions sit at this offset of the 256-value block:
__device__ inline int q4_a_offset(int h, int i) {
    const int L = i >> 2, nib = (i >> 1) & 1, half = i & 1;
    const int g = (h >> 1) + 2 * L;
    return 32 * (2 * g + nib) + 16 * (h & 1) + 8 * half;
}

// Q4_K B operand of MFMA i from the lane's raw 16-byte qs load of group g_L
__device__ inline half8_t q4_b(const uint4 &q, int i, int sc) {
    const uint32_t M = 0x0F0F0F0Fu;
    uint32_t w0 = (i & 1) ? q.z : q.x, w1 = (i & 1) ? q.w : q.y;
    if ((i >> 1) & 1) { w0 >>= 4; w1 >>= 4; }
    return q4_scaled(w0 & M, w1 & M, sc);
}

struct Q4Scales {
    int sc[2][2];      // [L][nibble]
    half4_t bm;        // min operand: mins of sub-blocks 2g, 2g+1, g = g_{h & 1}, each twice
    float d, dmin;
};

__device__ inline void q4_scales(const uint4 &hdr, int h, Q4Scales &o) {
    o.d = h2f_dev((uint16_t)(hdr.x & 0xffff));
    o.dmin = h2f_dev((uint16_t)(hdr.x >> 16));
#pragma unroll
    for (int L = 0; L < 2; ++L) {
        const int g = (h >> 1) + 2 * L;
        int m0, m1;
        q4k_sm(hdr, 2 * g, o.sc[L][0], m0);
        q4k_sm(hdr, 2 * g + 1, o.sc[L][1], m1);
        if (L == (h & 1)) {
            const _Float16 x0 = (_Float16)(float)m0, x1 = (_Float16)(float)m1;
            o.bm = half4_t{x0, x0, x1, x1};
        }
    }
}

// ---- activation staging ------------------------------------------------------
// One 256-value block of the activation rows of a pass's pairs, in LDS.  The
// 16-byte chunk c of row r sits at position c ^ (r & 15), so the 16 rows one
// fragment read touches fall in distinct banks.

// R activation rows (32 for two M tiles of 16 pairs, 16 for one) and the group
// sums of up to 32
template <int R>
struct __attribute__((aligned(16))) AStageR {
    _Float16 a[R][QK];
    _Float16 bs[32][16];
};

template <int R>
__device__ inline half8_t stage_frag(const AStageR<R> &st, int r, int off) {
    const int c = (off >> 3) ^ (r & 15);
    return *(const half8_t *)&st.a[r][8 * c];
}

// Staging by direct buffer -> LDS loads: lane l of an instruction writes
// base + 16*l.  rows[r]: activation row of pair r of the pass (r < np); rows
// are K values long.  Wave w stages rows (R/4)w .. (R/4)w + R/4 - 1 (two per
// instruction), wave 0 also the group sums; rows past np are not loaded.  The
// activation codes and the group sums are raw buffers, the lane's byte offsets
// are computed once per pass of a chunk and block s's offset s*QK*2 is a
// scalar: a step's staging costs no per-lane address arithmetic (up/gate at
// 512 tokens 104.0 -> 97.8 us a launch against 64-bit pointers per load).
constexpr int BUF_WORD3 = 0x00020000;    // raw buffer, 32-bit elements (gfx9)
typedef int i32x4_t __attribute__((ext_vector_type(4)));
__device__ void buffer_load_lds(i32x4_t rsrc, lptr_t *lds, int size, int voffset, int soffset, int offset,
                                int aux) __asm("llvm.amdgcn.raw.buffer.load.lds");
__device__ i32x4_t buffer_load_v4(i32x4_t rsrc, int voffset, int soffset, int aux) __asm("llvm.amdgcn.raw.buffer.load.v4i32");
typedef int i32x2_t __attribute__((ext_vector_type(2)));
__device__ i32x2_t buffer_load_v2(i32x4_t rsrc, int voffset, int soffset, int aux) __asm("llvm.amdgcn.raw.buffer.load.v2i32");
__device__ short buffer_load_i16(i32x4_t rsrc, int voffset, int soffset, int aux) __asm("llvm.amdgcn.raw.buffer.load.i16");
// a buffer resource over [p, p + bytes): base address, no stride, the size, raw
// (the words are the same in every lane: scalar registers)
__device__ inline i32x4_t raw_buffer(const void *p, uint32_t bytes) {
    const uint64_t a = (uint64_t)p;
    i32x4_t r;
    r.x = __builtin_amdgcn_readfirstlane((int)(uint32_t)a);
    r.y = __builtin_amdgcn_readfirstlane((int)((uint32_t)(a >> 32) & 0xffffu));
    r.z = __builtin_amdgcn_readfirstlane((int)bytes);
    r.w = BUF_WORD3;
    return r;
}
template <int R>
struct StageOff {
    int a[R / 8];       // instruction j: the lane's row and swizzled chunk, bytes
    int bs;             // the lane's group-sum chunk (wave 0), bytes
};
template <int R>
__device__ inline void stage_offsets(StageOff<R> &o, const int *rows, int np, int K, int wave, int lane) {
#pragma unroll
    for (int j = 0; j < R / 8; ++j) {
        const int r0 = (R / 4) * wave + 2 * j;
        const int r = min(r0 + (lane >> 5), np - 1);
        const int c = (lane & 31) ^ ((r0 + (lane >> 5)) & 15);
        o.a[j] = 2 * (rows[max(r, 0)] * K + 8 * c);
    }
    const int r = min(lane >> 1, np - 1);
    o.bs = 2 * (rows[max(r, 0)] * (K / 16) + 8 * (lane & 1));
}
template <int R, bool SUMS = true>
__device__ inline void stage_a_buf(AStageR<R> &st, const StageOff<R> &o, int np, i32x4_t ra, i32x4_t rbs, int s,
                                   int wave) {
#pragma unroll
    for (int j = 0; j < R / 8; ++j) {
        const int r0 = (R / 4) * wave + 2 * j;
        if (r0 >= np) break;
        buffer_load_lds(ra, (lptr_t *)&st.a[r0][0], 16, o.a[j], s * QK * 2, 0, 0);
    }
    if (SUMS && wave == 0) buffer_load_lds(rbs, (lptr_t *)&st.bs[0][0], 16, o.bs, s * 32, 0, 0);
}
__device__ inline uint4 buf_load16(i32x4_t r, int voff, int soff) {
    const i32x4_t v = buffer_load_v4(r, voff, soff, 0);
    return make_uint4((uint32_t)v.x, (uint32_t)v.y, (uint32_t)v.z, (uint32_t)v.w);
}

// Workgroup -> (row tile, expert).  Workgroups go to the 8 XCDs round-robin
// (workgroup L on XCD L % 8); with E a multiple of 8, every row tile of
// expert e lands on XCD e % 8, so the tiles of an expert share one L2 copy of
// its activation rows instead of fetching them into all eight.
__device__ inline void tile_expert(int L, int T, int E, int &tile, int &e) {
    if (E % 8 == 0) {
        const int j = L >> 3;
        e = (L & 7) + 8 * (j / T);
        tile = j % T;
    } else {
        e = L / T;
        tile = L % T;
    }
}

// ---------------------------------------------------------------------------
// Q6_K lane layout of the streamed kernel.  Lane (n = row, h) takes, of the
// 128-value half hh = h >> 1, the 16 positions l = 16*(h & 1) .. +15 of each
// of its four 32-value groups g: ql bytes 64hh + l (g = 0 low nibbles, g = 2
// high) and 64hh + 32 + l (g = 1, 3), qh bytes 32hh + l (two bits a group),
// so each group's 16 values share one scale, 8hh + 2g + (h & 1).  MFMA
// i = 2g + half multiplies positions l = 16*(h & 1) + 8*half .. +7 of group g;
// the activation values at those positions sit at this offset of the block:
__device__ inline int q6_a_offset(int h, int i) {
    return 128 * (h >> 1) + 32 * (i >> 1) + 16 * (h & 1) + 8 * (i & 1);
}

struct Q6Lane {
    uint4 qa, qb, qh;      // ql bytes 64hh + l, 64hh + 32 + l, qh bytes 32hh + l
    uint2 sc;              // scales 8hh .. 8hh + 7
    uint32_t d;            // the block's fp16 scale in the low half
};

// The lane's offsets into its row's blocks, and one block's pieces by buffer
// loads at the block's offset (a scalar).  A Q6_K block starts 2-byte aligned
// (210-byte blocks); the loads are unaligned.
struct Q6Off {
    int qa, qb, qh, sc, d;
};
__device__ inline Q6Off q6_lane_offsets(int row_off, int h) {
    const int hh = h >> 1, l0 = 16 * (h & 1);
    return Q6Off{row_off + 64 * hh + l0, row_off + 64 * hh + 32 + l0, row_off + 128 + 32 * hh + l0,
                 row_off + 192 + 8 * hh, row_off + 208};
}
__device__ inline void q6_lane_load(Q6Lane &w, i32x4_t rw, const Q6Off &o, int blk_off) {
    const i32x4_t a = buffer_load_v4(rw, o.qa, blk_off, 0), b = buffer_load_v4(rw, o.qb, blk_off, 0);
    const i32x4_t q = buffer_load_v4(rw, o.qh, blk_off, 0);
    const i32x2_t sc = buffer_load_v2(rw, o.sc, blk_off, 0);
    w.qa = make_uint4((uint32_t)a.x, (uint32_t)a.y, (uint32_t)a.z, (uint32_t)a.w);
    w.qb = make_uint4((uint32_t)b.x, (uint32_t)b.y, (uint32_t)b.z, (uint32_t)b.w);
    w.qh = make_uint4((uint32_t)q.x, (uint32_t)q.y, (uint32_t)q.z, (uint32_t)q.w);
    w.sc = make_uint2((uint32_t)sc.x, (uint32_t)sc.y);
    w.d = (uint16_t)buffer_load_i16(rw, o.d, blk_off, 0);
}

// The B operands of MFMA i: (q - 32) * sc in two exact halves, sc = 16*sh + sl
// (|(q - 32) * sh| <= 256, |(q - 32) * sl| <= 480); (1024 + q)*s - 1056*s is
// one rounding of an exact integer.
__device__ inline void q6_lane_b(const Q6Lane &w, int i, int h, half8_t &bh, half8_t &bl) {
    const uint32_t M = 0x0F0F0F0Fu, HM = 0x30303030u;
    const int g = i >> 1, half = i & 1;
    const uint4 &ql = (g & 1) ? w.qb : w.qa;
    uint32_t l0 = half ? ql.z : ql.x, l1 = half ? ql.w : ql.y;
    uint32_t q0 = half ? w.qh.z : w.qh.x, q1 = half ? w.qh.w : w.qh.y;
    if (g >= 2) {
        l0 >>= 4;
        l1 >>= 4;
    }
    // group g's two high bits (qh bits 2g, 2g+1) to bits 4, 5 of each byte
    if (g == 0) { q0 <<= 4; q1 <<= 4; }
    if (g == 1) { q0 <<= 2; q1 <<= 2; }
    if (g == 3) { q0 >>= 2; q1 >>= 2; }
    const half8_t q = pack_1024((l0 & M) | (q0 & HM), (l1 & M) | (q1 & HM));
    const int j = 2 * g + (h & 1);
    const int sc = (int)(int8_t)(uint8_t)((j < 4 ? w.sc.x : w.sc.y) >> (8 * (j & 3)));
    const _Float16 sh = (_Float16)(float)(sc >> 4), sl = (_Float16)(float)(sc & 15);   // arithmetic shift
    bh = __builtin_elementwise_fma(q, splat8(sh), splat8((_Float16)(float)(-1056 * (sc >> 4))));
    bl = __builtin_elementwise_fma(q, splat8(sl), splat8((_Float16)(float)(-1056 * (sc & 15))));
}

// The grouped down product for a Q6_K matrix, the lane's weights streamed from
// HBM into registers as in grouped_q4_kernel (block s+1 in flight while block
// s is multiplied, no LDS tile), in chunks of up to CH passes of MT M tiles of
// 16 pairs: each block's weights are loaded once for the chunk and decoded per
// pass.  CH = 1, (256, 4): four workgroups a CU; CH = 2 for large batches,
// (256, 3).  A block's two integer sums stay below 2^24 (256 * 32 * 8 * 127
// and 256 * 32 * 15 * 127), so each is exact and 16*acc_h + acc_l rounds once,
// as ggml's (float)sumi.  y = the pair's gate weight times the row value, to
// the pair's (t*K + k) row.
template <int NB, int CH, int MT>
__global__ __launch_bounds__(256, CH == 1 ? 4 : 3) void grouped_q6_kernel(GroupedArgs a) {
    constexpr int GK = 16 * MT;
    int e, tile;
    tile_expert(blockIdx.x, a.H / 64, a.E, tile, e);
    const int n0 = a.offsets[e], ne = a.offsets[e + 1] - n0;
    if (ne <= 0) return;
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int n = lane & 15, h = lane >> 4;
    const int r0 = tile * 64;
    const int row = r0 + wave * 16 + n;
    constexpr int K = NB * QK;
    const uint8_t *base = grouped_expert(a, e);
    if (!base) {
        for (int i = tid; i < ne * 64; i += 256) {
            const int pos = n0 + i / 64, c = r0 + (i % 64);
            a.ypair[(size_t)a.perm[pos] * a.H + c] = 0.0f;
        }
        return;
    }
    // the expert's down matrix and the Q8_K codes of h as raw buffers
    const i32x4_t rw = raw_buffer(base + 2ull * a.I * (a.H / QK) * Q4K_BYTES, (uint32_t)(a.H * NB * Q6K_BYTES));
    const i32x4_t ra = raw_buffer(a.ha, 0xffffffffu);
    const Q6Off wo = q6_lane_offsets(row * (NB * Q6K_BYTES), h);

    __shared__ AStageR<GK> st[2];
    __shared__ int s_rows[CH * GK];
    __shared__ __attribute__((aligned(16))) float s_dx[NB][CH * GK];

    for (int cb = 0; cb < ne; cb += CH * GK) {
        const int npc = min(CH * GK, ne - cb);
        const int nps = (npc + GK - 1) / GK;
        if (tid < CH * GK) s_rows[tid] = n0 + cb + min(tid, npc - 1);   // h rows are in dispatch order
        __syncthreads();
        for (int i = tid; i < CH * GK * NB; i += 256)
            s_dx[i % NB][i / NB] = a.hdx[(size_t)s_rows[i / NB] * NB + (i % NB)];
        StageOff<GK> so[CH];
#pragma unroll
        for (int p = 0; p < CH; ++p)
            if (p < nps) stage_offsets(so[p], s_rows + p * GK, min(GK, npc - p * GK), K, wave, lane);
        stage_a_buf<GK, false>(st[0], so[0], min(GK, npc), ra, ra, 0, wave);
        Q6Lane cw, nw;
        q6_lane_load(cw, rw, wo, 0);
        __builtin_amdgcn_s_waitcnt(0);
        __syncthreads();
        float y[CH][MT][4];
#pragma unroll
        for (int p = 0; p < CH; ++p)
#pragma unroll
            for (int t = 0; t < MT; ++t)
#pragma unroll
                for (int i = 0; i < 4; ++i) y[p][t][i] = 0.0f;
        int j = 0;                       // step j = s * nps + p
#pragma unroll 1
        for (int s = 0; s < NB; ++s) {
            if (s + 1 < NB) q6_lane_load(nw, rw, wo, (s + 1) * Q6K_BYTES);
            const float d = h2f_dev((uint16_t)cw.d);
#pragma unroll
            for (int p = 0; p < CH; ++p) {
                if (p < nps) {
                    // both M tiles always (skipping an empty second tile, as the Q4_K kernel does,
                    // made this kernel ~1.7 us a launch slower at 512 tokens)
                    constexpr bool full = true;
                    const AStageR<GK> &S = st[j & 1];
                    const int jn = j + 1;
                    if (jn < NB * nps) {
                        const int s2 = jn / nps, p2 = jn - s2 * nps;
                        StageOff<GK> sp = so[0];
                        if constexpr (CH > 1) {
#pragma unroll
                            for (int q = 0; q < GK / 8; ++q) sp.a[q] = p2 ? so[1].a[q] : so[0].a[q];
                        }
                        stage_a_buf<GK, false>(st[jn & 1], sp, min(GK, npc - p2 * GK), ra, ra, s2, wave);
                    }
                    float4_t acc[MT], accl[MT];
#pragma unroll
                    for (int t = 0; t < MT; ++t) acc[t] = accl[t] = float4_t{0, 0, 0, 0};
                    half8_t fa[2][MT];
#pragma unroll
                    for (int t = 0; t < MT; ++t) if (t == 0 || full) fa[0][t] = stage_frag(S, 16 * t + n, q6_a_offset(h, 0));
#pragma unroll
                    for (int i = 0; i < 8; ++i) {
                        if (i + 1 < 8) {
#pragma unroll
                            for (int t = 0; t < MT; ++t) if (t == 0 || full)
                                fa[(i + 1) & 1][t] = stage_frag(S, 16 * t + n, q6_a_offset(h, i + 1 < 8 ? i + 1 : 0));
                        }
                        half8_t bh, bl;
                        q6_lane_b(cw, i, h, bh, bl);
#pragma unroll
                        for (int t = 0; t < MT; ++t) if (t == 0 || full) {
                            acc[t] = mfma32(fa[i & 1][t], bh, acc[t]);
                            accl[t] = mfma32(fa[i & 1][t], bl, accl[t]);
                        }
                    }
#pragma unroll
                    for (int t = 0; t < MT; ++t) if (t == 0 || full) {
                        const float4 dxv = *(const float4 *)&s_dx[s][p * GK + 16 * t + 4 * h];
#pragma unroll
                        for (int i = 0; i < 4; ++i) {
                            const float dx = i == 0 ? dxv.x : i == 1 ? dxv.y : i == 2 ? dxv.z : dxv.w;
                            const float sumi = 16.0f * acc[t][i] + accl[t][i];
                            y[p][t][i] = y[p][t][i] + (d * dx) * sumi;   // ggml's order: acc += (d*dx)*sumi
                        }
                    }
                    __builtin_amdgcn_s_waitcnt(0);
                    __syncthreads();
                    ++j;
                }
            }
            cw = nw;
        }
#pragma unroll
        for (int p = 0; p < CH; ++p) {
#pragma unroll
            for (int t = 0; t < MT; ++t) {
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const int r = p * GK + 16 * t + 4 * h + i;
                    if (r < npc) {
                        const int q = a.perm[n0 + cb + r];
                        a.ypair[(size_t)q * a.H + row] = a.w[q] * y[p][t][i];
                    }
                }
            }
        }
        __syncthreads();
    }
}

// the trivial dispatch of one expert over n pairs: offsets {0, n}, perm = 0..n-1,
// weights 1 (the always-on shared expert)
__global__ void iota_kernel(int n, int32_t *offsets, int32_t *perm, float *ones) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) {
        perm[i] = i;
        ones[i] = 1.0f;
    }
    if (i == 0) {
        offsets[0] = 0;
        offsets[1] = n;
    }
}

// out[t] (+)= sum_k ypair[t*K + k], k ascending; one float4 per thread
__global__ __launch_bounds__(256) void combine_kernel(const float *ypair, int n_tok, int K, int H, float *out,
                                                      int accumulate) {
    const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
    const size_t h4 = (size_t)H / 4;
    if (i >= (size_t)n_tok * h4) return;
    const size_t t = i / h4, c = i % h4;
    const float4 *y = (const float4 *)ypair + (size_t)t * K * h4 + c;
    float4 s = y[0];
    for (int k = 1; k < K; ++k) {
        const float4 v = y[(size_t)k * h4];
        s.x = s.x + v.x; s.y = s.y + v.y; s.z = s.z + v.z; s.w = s.w + v.w;
    }
    float4 *o = (float4 *)out + i;
    if (accumulate) {
        const float4 p = *o;
        s.x = p.x + s.x; s.y = p.y + s.y; s.z = p.z + s.z; s.w = p.w + s.w;
    }
    *o = s;
}

// the same with the host's rows: pair i's row from hrows when hflag[i] (mapped
// host memory, read over PCIe), else from ypair; k ascending either way
__global__ __launch_bounds__(256) void combine_host_kernel(const float *ypair, const float *hrows, const uint8_t *hflag,
                                                           int n_tok, int K, int H, float *out, int accumulate) {
    const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
    const size_t h4 = (size_t)H / 4;
    if (i >= (size_t)n_tok * h4) return;
    const size_t t = i / h4, c = i % h4;
    auto row = [&](int k) {
        const size_t pr = (size_t)t * K + k;
        return hflag[pr] ? ((const float4 *)hrows)[pr * h4 + c] : ((const float4 *)ypair)[pr * h4 + c];
    };
    float4 s = row(0);
    for (int k = 1; k < K; ++k) {
        const float4 v = row(k);
        s.x = s.x + v.x; s.y = s.y + v.y; s.z = s.z + v.z; s.w = s.w + v.w;
    }
    float4 *o = (float4 *)out + i;
    if (accumulate) {
        const float4 p = *o;
        s.x = p.x + s.x; s.y = p.y + s.y; s.z = p.z + s.z; s.w = p.w + s.w;
    }
    *o = s;
}

// ---------------------------------------------------------------------------
// launchers (shapes checked by the caller)
template <typename F, typename... A>
static hipError_t launch_b(F k, dim3 grid, dim3 block, hipStream_t st, hipEvent_t ev0, hipEvent_t ev1, A... args) {
    if (ev0) hipExtLaunchKernelGGL(k, grid, block, 0, st, ev0, ev1, 0, args...);
    else hipLaunchKernelGGL(k, grid, block, 0, st, args...);
    return hipGetLastError();
}

hipError_t launch_dispatch(const int32_t *ids, int P, int E, int32_t *counts, int32_t *offsets, int32_t *perm,
                           hipStream_t st) {
    return launch_b(dispatch_kernel, dim3(1), dim3(1024), st, nullptr, nullptr, ids, P, E, counts, offsets, perm);
}

hipError_t launch_quant_rows(const void *src, int bf16, int n_rows, int n, uint16_t *q16, float *dx, uint16_t *bs16,
                             hipStream_t st) {
    const int64_t blocks = ((int64_t)n_rows * (n / QK) + 3) / 4;
    if (blocks == 0) return hipSuccess;
    return launch_b(quant_rows_kernel, dim3((unsigned)blocks), dim3(256), st, nullptr, nullptr, src, bf16, n_rows, n,
                    q16, dx, bs16);
}

hipError_t launch_swiglu_quant(const float *y2, int P, int I, float *h_out, uint16_t *q16, float *dx, uint16_t *bs16,
                               hipStream_t st) {
    const int64_t blocks = ((int64_t)P * (I / QK) + 3) / 4;
    if (blocks == 0) return hipSuccess;
    return launch_b(swiglu_quant_kernel, dim3((unsigned)blocks), dim3(256), st, nullptr, nullptr, y2, P, I, h_out, q16,
                    dx, bs16);
}

// ---------------------------------------------------------------------------
// The Q4_K grouped product with the weights read and decoded once per chunk
// of up to CH passes (CH * 16 * MT pairs): for each super-block s, the lane's
// weights are loaded once (block s+1 in flight meanwhile) and turned into the
// eight MFMA B operands once, then every pass of the chunk multiplies its
// staged activation rows by them.  Each pair still accumulates its
// super-blocks in order 0, 1, ..., so the arithmetic is the one-pass kernel's.
// CH = 2 for large batches, (256, 3): up to 168 registers, which the eight
// operands of two passes need; CH = 1 when experts rarely get more than 32
// pairs, (256, 4): four waves per SIMD.  MT = 1 (one 16-row M tile a pass)
// when experts average at most 8 pairs: half the staged rows and products,
// which would be empty anyway (batch 64 at 128 experts: up/gate 67.0 -> 63.4
// us a launch, batch 16: 53.1 -> 51.1).  The (256, 5) bound, which the MT = 1
// kernels fit without spills (73-94 registers), was no faster (batch 64:
// 10,629 -> 10,633 tok/s).
template <int NB, bool DOWN, int CH, int MT>
__global__ __launch_bounds__(256, CH == 1 ? 4 : 3) void grouped_q4_kernel(GroupedArgs a) {
    constexpr int GK = 16 * MT;           // pairs per pass: MT M tiles of 16
    int e, tile;
    tile_expert(blockIdx.x, (DOWN ? a.H : 2 * a.I) / 64, a.E, tile, e);
    const int n0 = a.offsets[e], ne = a.offsets[e + 1] - n0;
    if (ne <= 0) return;
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int n = lane & 15, h = lane >> 4;
    const int r0 = tile * 64;
    const int row = r0 + wave * 16 + n;
    constexpr int K = NB * QK;
    constexpr int ROWB = NB * Q4K_BYTES;
    const int out_n = DOWN ? a.H : 2 * a.I;
    const uint8_t *base = grouped_expert(a, e);
    if (!base) {
        for (int i = tid; i < ne * 64; i += 256) {
            const int pos = n0 + i / 64, c = r0 + (i % 64);
            if (DOWN) a.ypair[(size_t)a.perm[pos] * a.H + c] = 0.0f;
            else a.y2[(size_t)pos * out_n + c] = 0.0f;
        }
        return;
    }
    const uint8_t *mat = DOWN ? base + 2ull * a.I * (a.H / QK) * Q4K_BYTES : base;
    const uint16_t *act = DOWN ? a.ha : a.xa;
    const uint16_t *abs16 = DOWN ? a.hbs : a.xbs;
    const float *adx = DOWN ? a.hdx : a.xdx;

    __shared__ AStageR<GK> st[2];
    __shared__ int s_rows[CH * GK];
    __shared__ __attribute__((aligned(16))) float s_dx[NB][CH * GK];   // [block][pair]: a lane's 4 rows in one read
    const int gm = (h >> 1) + 2 * (h & 1);
    // the expert's matrix, the activation codes and their group sums as raw
    // buffers; the lane's weight offsets (header, the two qs loads) fixed
    const i32x4_t rw = raw_buffer(mat, (uint32_t)((DOWN ? a.H : 2 * a.I) * ROWB));
    const i32x4_t ra = raw_buffer(act, 0xffffffffu), rbs = raw_buffer(abs16, 0xffffffffu);
    const int wo0 = row * ROWB, wo1 = wo0 + 16 + 16 * h, wo2 = wo0 + 80 + 16 * h;

    for (int cb = 0; cb < ne; cb += CH * GK) {
        const int npc = min(CH * GK, ne - cb);
        const int nps = (npc + GK - 1) / GK;
        if (tid < CH * GK) {
            const int pos = n0 + cb + min(tid, npc - 1);
            s_rows[tid] = DOWN ? pos : a.perm[pos] / a.K;
        }
        __syncthreads();
        for (int i = tid; i < CH * GK * NB; i += 256) s_dx[i % NB][i / NB] = adx[(size_t)s_rows[i / NB] * NB + (i % NB)];
        StageOff<GK> so[CH];
#pragma unroll
        for (int p = 0; p < CH; ++p)
            if (p < nps) stage_offsets(so[p], s_rows + p * GK, min(GK, npc - p * GK), K, wave, lane);
        stage_a_buf(st[0], so[0], min(GK, npc), ra, rbs, 0, wave);
        uint4 cw[3], nw[3];
        cw[0] = buf_load16(rw, wo0, 0);
        cw[1] = buf_load16(rw, wo1, 0);
        cw[2] = buf_load16(rw, wo2, 0);
        __builtin_amdgcn_s_waitcnt(0);
        __syncthreads();
        float y[CH][MT][4];
#pragma unroll
        for (int p = 0; p < CH; ++p)
#pragma unroll
            for (int t = 0; t < MT; ++t)
#pragma unroll
                for (int i = 0; i < 4; ++i) y[p][t][i] = 0.0f;
        int j = 0;                       // step j = s * nps + p
#pragma unroll 1
        for (int s = 0; s < NB; ++s) {
            if (s + 1 < NB) {
                nw[0] = buf_load16(rw, wo0, (s + 1) * Q4K_BYTES);
                nw[1] = buf_load16(rw, wo1, (s + 1) * Q4K_BYTES);
                nw[2] = buf_load16(rw, wo2, (s + 1) * Q4K_BYTES);
            }
            Q4Scales sc;
            q4_scales(cw[0], h, sc);
            half8_t b[CH > 1 ? 8 : 1];          // kept across the passes (one pass: built where used)
            if constexpr (CH > 1) {
#pragma unroll
                for (int i = 0; i < 8; ++i) {
                    const int L = i >> 2, nib = (i >> 1) & 1;
                    b[i] = q4_b(L ? cw[2] : cw[1], i, sc.sc[L][nib]);
                }
            }
#pragma unroll
            for (int p = 0; p < CH; ++p) {
                if (p < nps) {
                    // two-pass chunks: a pass whose second M tile holds no pair skips its reads,
                    // products and sums (512 tokens: up/gate 4.71 -> 4.62 ms per 48 layers;
                    // in one-pass chunks the branch cost more than it saved)
                    const bool full = MT == 1 || CH == 1 || npc - p * GK > 16;
                    const AStageR<GK> &S = st[j & 1];
                    const int jn = j + 1;
                    if (jn < NB * nps) {
                        const int s2 = jn / nps, p2 = jn - s2 * nps;
                        // the pass's offsets by selects (a runtime index would put so in scratch)
                        StageOff<GK> sp = so[0];
                        if constexpr (CH > 1) {
#pragma unroll
                            for (int q = 0; q < GK / 8; ++q) sp.a[q] = p2 ? so[1].a[q] : so[0].a[q];
                            sp.bs = p2 ? so[1].bs : so[0].bs;
                        }
                        stage_a_buf(st[jn & 1], sp, min(GK, npc - p2 * GK), ra, rbs, s2, wave);
                    }
                    // each 128-value half of the super-block in its own accumulator:
                    // a half's products sum to at most 128 * 63 * 15 * 127 < 2^24, so
                    // it is exact in fp32, and one add gives ggml's (float)sumi (a
                    // whole block's sum can pass 2^24, where a running fp32 sum rounds)
                    float4_t acc[MT], acc0[MT];
#pragma unroll
                    for (int t = 0; t < MT; ++t) acc[t] = float4_t{0, 0, 0, 0};
                    // the fragments of K chunk i+1 are read before chunk i's products
                    half8_t fa[2][MT];
#pragma unroll
                    for (int t = 0; t < MT; ++t) if (t == 0 || full) fa[0][t] = stage_frag(S, 16 * t + n, q4_a_offset(h, 0));
#pragma unroll
                    for (int i = 0; i < 8; ++i) {
                        if (i + 1 < 8) {
#pragma unroll
                            for (int t = 0; t < MT; ++t) if (t == 0 || full)
                                fa[(i + 1) & 1][t] = stage_frag(S, 16 * t + n, q4_a_offset(h, i + 1 < 8 ? i + 1 : 0));
                        }
                        half8_t bi;
                        if constexpr (CH > 1) {
                            bi = b[i];
                        } else {
                            const int L = i >> 2, nib = (i >> 1) & 1;
                            bi = q4_b(L ? cw[2] : cw[1], i, sc.sc[L][nib]);
                        }
                        if (i == 4) {
#pragma unroll
                            for (int t = 0; t < MT; ++t) {
                                acc0[t] = acc[t];
                                acc[t] = float4_t{0, 0, 0, 0};
                            }
                        }
#pragma unroll
                        for (int t = 0; t < MT; ++t) if (t == 0 || full) acc[t] = mfma32(fa[i & 1][t], bi, acc[t]);
                    }
#pragma unroll
                    for (int t = 0; t < MT; ++t) acc[t] = acc0[t] + acc[t];
                    float4 dxv[MT];
#pragma unroll
                    for (int t = 0; t < MT; ++t) dxv[t] = *(const float4 *)&s_dx[s][p * GK + 16 * t + 4 * h];
#pragma unroll
                    for (int t = 0; t < MT; ++t) if (t == 0 || full) {
                        const half4_t am = *(const half4_t *)&S.bs[16 * t + n][4 * gm];
                        float4_t z = {0, 0, 0, 0};
                        z = __builtin_amdgcn_mfma_f32_16x16x16f16(am, sc.bm, z, 0, 0, 0);
#pragma unroll
                        for (int i = 0; i < 4; ++i) {
                            // ggml's order: acc += (d*dx)*sumi; acc -= (dmin*dx)*summ
                            const float dx = i == 0 ? dxv[t].x : i == 1 ? dxv[t].y : i == 2 ? dxv[t].z : dxv[t].w;
                            y[p][t][i] = y[p][t][i] + (sc.d * dx) * acc[t][i];
                            y[p][t][i] = y[p][t][i] - (sc.dmin * dx) * z[i];
                        }
                    }
                    __builtin_amdgcn_s_waitcnt(0);
                    __syncthreads();
                    ++j;
                }
            }
            cw[0] = nw[0];
            cw[1] = nw[1];
            cw[2] = nw[2];
        }
#pragma unroll
        for (int p = 0; p < CH; ++p) {
#pragma unroll
            for (int t = 0; t < MT; ++t) {
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const int r = p * GK + 16 * t + 4 * h + i;
                    if (r < npc) {
                        const int pos = n0 + cb + r;
                        if (DOWN) {
                            const int pp = a.perm[pos];
                            a.ypair[(size_t)pp * a.H + row] = a.w[pp] * y[p][t][i];
                        } else {
                            a.y2[(size_t)pos * out_n + row] = y[p][t][i];
                        }
                    }
                }
            }
        }
        __syncthreads();
    }
}

template <bool DOWN>
static hipError_t launch_gg(const GroupedArgs &a, hipStream_t st, hipEvent_t e0, hipEvent_t e1) {
    const int rows = DOWN ? a.H : 2 * a.I;
    const int nb = (DOWN ? a.I : a.H) / QK;
    const dim3 grid((unsigned)(rows / 64 * a.E)), blk(256);     // (row tile, expert) from the linear id
    const bool two = a.P > 16 * a.E;                            // many experts above 32 pairs
    const bool one = a.P <= 8 * a.E;                            // few pairs: one 16-row M tile a pass
    if (DOWN) {
        if (a.down_type == TYPE_Q6K) {
            if (two) {
                if (nb == 3) return launch_b(grouped_q6_kernel<3, 2, 2>, grid, blk, st, e0, e1, a);
                if (nb == 2) return launch_b(grouped_q6_kernel<2, 2, 2>, grid, blk, st, e0, e1, a);
                return launch_b(grouped_q6_kernel<1, 2, 2>, grid, blk, st, e0, e1, a);
            }
            if (one) {
                if (nb == 3) return launch_b(grouped_q6_kernel<3, 1, 1>, grid, blk, st, e0, e1, a);
                if (nb == 2) return launch_b(grouped_q6_kernel<2, 1, 1>, grid, blk, st, e0, e1, a);
                return launch_b(grouped_q6_kernel<1, 1, 1>, grid, blk, st, e0, e1, a);
            }
            if (nb == 3) return launch_b(grouped_q6_kernel<3, 1, 2>, grid, blk, st, e0, e1, a);
            if (nb == 2) return launch_b(grouped_q6_kernel<2, 1, 2>, grid, blk, st, e0, e1, a);
            return launch_b(grouped_q6_kernel<1, 1, 2>, grid, blk, st, e0, e1, a);
        }
        if (two) {
            if (nb == 3) return launch_b(grouped_q4_kernel<3, true, 2, 2>, grid, blk, st, e0, e1, a);
            if (nb == 2) return launch_b(grouped_q4_kernel<2, true, 2, 2>, grid, blk, st, e0, e1, a);
            return launch_b(grouped_q4_kernel<1, true, 2, 2>, grid, blk, st, e0, e1, a);
        }
        if (one) {
            if (nb == 3) return launch_b(grouped_q4_kernel<3, true, 1, 1>, grid, blk, st, e0, e1, a);
            if (nb == 2) return launch_b(grouped_q4_kernel<2, true, 1, 1>, grid, blk, st, e0, e1, a);
            return launch_b(grouped_q4_kernel<1, true, 1, 1>, grid, blk, st, e0, e1, a);
        }
        if (nb == 3) return launch_b(grouped_q4_kernel<3, true, 1, 2>, grid, blk, st, e0, e1, a);
        if (nb == 2) return launch_b(grouped_q4_kernel<2, true, 1, 2>, grid, blk, st, e0, e1, a);
        return launch_b(grouped_q4_kernel<1, true, 1, 2>, grid, blk, st, e0, e1, a);
    }
    if (two) return launch_b(grouped_q4_kernel<8, false, 2, 2>, grid, blk, st, e0, e1, a);
    if (one) return launch_b(grouped_q4_kernel<8, false, 1, 1>, grid, blk, st, e0, e1, a);
    return launch_b(grouped_q4_kernel<8, false, 1, 2>, grid, blk, st, e0, e1, a);
}

hipError_t launch_gateup_grouped(const GroupedArgs &a, hipStream_t st, hipEvent_t e0, hipEvent_t e1) {
    return launch_gg<false>(a, st, e0, e1);
}

hipError_t launch_down_grouped(const GroupedArgs &a, hipStream_t st, hipEvent_t e0, hipEvent_t e1) {
    return launch_gg<true>(a, st, e0, e1);
}

hipError_t launch_iota(int n, int32_t *offsets, int32_t *perm, float *ones, hipStream_t st) {
    return launch_b(iota_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), st, nullptr, nullptr, n, offsets, perm,
                    ones);
}

hipError_t launch_combine(const float *ypair, int n_tok, int K, int H, float *out, int accumulate, hipStream_t st) {
    const size_t n4 = (size_t)n_tok * H / 4;
    if (n4 == 0) return hipSuccess;
    return launch_b(combine_kernel, dim3((unsigned)((n4 + 255) / 256)), dim3(256), st, nullptr, nullptr, ypair, n_tok,
                    K, H, out, accumulate);
}

hipError_t launch_combine_host(const float *ypair, const float *hrows, const uint8_t *hflag, int n_tok, int K, int H,
                               float *out, int accumulate, hipStream_t st) {
    const size_t n4 = (size_t)n_tok * (H / 4);
    return launch_b(combine_host_kernel, dim3((unsigned)((n4 + 255) / 256)), dim3(256), st, nullptr, nullptr, ypair,
                    hrows, hflag, n_tok, K, H, out, accumulate);
}

// ---------------------------------------------------------------------------
// Scratch of the allocation-free grouped entry point: the workspace of one
// call (Q8_K codes of x and h, the up/gate rows, the weighted pair rows) in
// a file-scope array.  Every device the library runs on holds its own copy
// at its own address from the code object's load until the process ends.
// In host code `scratch` names a host-side stand-in, not device memory:
// kernels are given the address static_scratch() looks up.
static __device__ __align__(256) uint8_t scratch[STATIC_SCRATCH_BYTES];

hipError_t static_scratch(void **ptr) {
    constexpr int MAX_DEV = 64;
    static std::mutex m;
    static void *addr[MAX_DEV] = {};
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return e;
    if (dev < 0 || dev >= MAX_DEV) return hipErrorInvalidDevice;
    std::lock_guard<std::mutex> lk(m);
    if (!addr[dev]) {           // once per device, with that device current
        void *p = nullptr;
        e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess) return e;
        addr[dev] = p;
    }
    *ptr = addr[dev];
    return hipSuccess;
}

}  // namespace mp
