// mp_batched.hip -- gfx950 kernels of the batched MoE layer (prefill chunks and
// decode at batch > 1).
//
//   dispatch_kernel    per-expert histogram, exclusive scan and the stable
//                      permutation of (token, k) pairs (one workgroup)
//   quant_rows_kernel  Q8_K of rows (x per token, h per dispatched pair) into
//                      the form the matrix cores consume: the int8 values as
//                      fp16 codes, the block scale, and the 16-value group
//                      sums as fp16 -- all exact
//   gateup_grouped     per expert: [tokens x H] . [H x I] for up and gate on
//                      MFMA 16x16x32 f16, SwiGLU fused, h in dispatch order
//   down_grouped       per expert: [pairs x I] . [I x H], times the gate
//                      weight, scattered to the pair's (token, k) row
//   combine_kernel     out[t] = sum over k of the weighted rows, k in order
//
// Exact integer products on fp16 matrix cores.  A Q4_K weight is
// d*sc*q - dmin*m with q a nibble and sc, m six-bit.  The B operand holds sc*q
// (<= 945, an integer fp16 represents exactly: 11-bit significand; bf16's 8 bits
// cannot), the A operand the Q8_K integers of the activation (|q8| <= 127,
// exact), so the fp32 accumulation over a 256-value super-block is the exact
// integer sum_j sc_j * sum_i q_i q8_i of ggml's vec_dot_q4_K_q8_K.  The min
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

#include "mp_device.h"
#include "mp_format.h"
#include "mp_internal.h"

namespace mp {

typedef _Float16 half4_t __attribute__((ext_vector_type(4)));
typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef float float4_t __attribute__((ext_vector_type(4)));

// ---------------------------------------------------------------------------
// dispatch: ids [P] (P = n_tok * K, pair i = t*K + k) -> counts[E], offsets[E+1],
// perm[offsets[e] + r] = i of the r-th pair routed to e in pair order.
// Pass 1 counts with LDS atomics (order-free); pass 2 places 64-pair chunks:
// lanes holding the same id find each other with 8 ballots (one per id bit),
// their rank inside the chunk is a popcount, and a per-expert scan over the
// chunks of the pass (continuing a running count) gives each chunk's base.
constexpr int DSP_CHUNKS = 64;

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
    if (tid == 0) {
        int acc = 0;
        for (int e = 0; e < E; ++e) {
            const int c = s_off[e];
            counts[e] = c;
            offsets[e] = acc;
            s_off[e] = acc;
            acc += c;
        }
        offsets[E] = acc;
    }
    __syncthreads();
    const int nwaves = blockDim.x >> 6;
    for (int base = 0; base < P; base += DSP_CHUNKS * 64) {
        for (int i = tid; i < DSP_CHUNKS * E; i += blockDim.x) s_c[i / E][i % E] = 0;
        __syncthreads();
        int my_e[DSP_CHUNKS / 16], my_r[DSP_CHUNKS / 16];
        for (int j = 0, c = wave; c < DSP_CHUNKS; ++j, c += nwaves) {
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
            for (int c = 0; c < DSP_CHUNKS; ++c) {
                const int v = s_c[c][e];
                s_c[c][e] = (uint16_t)run;
                run += v;
            }
            s_run[e] = run;
        }
        __syncthreads();
        for (int j = 0, c = wave; c < DSP_CHUNKS; ++j, c += nwaves) {
            const int e = my_e[j];
            if (e >= 0) perm[s_off[e] + s_c[c][e] + my_r[j]] = base + 64 * c + lane;
        }
        __syncthreads();
    }
}

// ---------------------------------------------------------------------------
// Q8_K rows for the matrix cores: one wavefront per (row, 256-value block)
__device__ inline uint32_t h16(int v) { return (uint32_t)__builtin_bit_cast(uint16_t, (_Float16)(float)v); }

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
    int q[4];
    float d;
    q8k_wave_vals(xv, lane, q, d);
    const int gs = q8k_group_sum(q);
    uint2 o;
    o.x = h16(q[0]) | (h16(q[1]) << 16);
    o.y = h16(q[2]) | (h16(q[3]) << 16);
    *(uint2 *)(q16 + off) = o;
    if ((lane & 3) == 0) bs16[(size_t)row * (n / 16) + b * 16 + (lane >> 2)] = (uint16_t)h16(gs);
    if (lane == 0) dx[(size_t)row * nb + b] = d;
}

// ---------------------------------------------------------------------------
// grouped expert products

__device__ inline const uint8_t *grouped_expert(const GroupedArgs &a, int e) {
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

// SiLU with the canonical exp (the oracle evaluates the same function)
__device__ inline float silu_mul(float g, float u) { return g / (1.0f + canon_expf(-g)) * u; }

// B operands of one Q4_K super-block for the lane's row: two 16-byte qs loads
// (group g_L = (h >> 1) + 2L, elements 16*(h & 1) .. +15 of sub-blocks 2g_L and
// 2g_L + 1), MFMA index 4L + 2*nibble + half.  Also the min operand for the
// sub-blocks of group g_{h & 1} and the row's d, dmin.
struct Q4Frag {
    half8_t b[8];
    half4_t bm;
    float d, dmin;
};

__device__ inline void q4_frag(const uint8_t *blk, int h, Q4Frag &f) {
    const uint4 hdr = *(const uint4 *)blk;
    const uint4 q0 = *(const uint4 *)(blk + 16 + 16 * h);
    const uint4 q1 = *(const uint4 *)(blk + 16 + 64 + 16 * h);
    f.d = h2f((uint16_t)(hdr.x & 0xffff));
    f.dmin = h2f((uint16_t)(hdr.x >> 16));
#pragma unroll
    for (int L = 0; L < 2; ++L) {
        const uint4 q = L ? q1 : q0;
        const int g = (h >> 1) + 2 * L;
        int sl, ml, sh, mh;
        q4k_sm(hdr, 2 * g, sl, ml);
        q4k_sm(hdr, 2 * g + 1, sh, mh);
        const uint32_t M = 0x0F0F0F0Fu;
        f.b[4 * L + 0] = q4_scaled(q.x & M, q.y & M, sl);
        f.b[4 * L + 1] = q4_scaled(q.z & M, q.w & M, sl);
        f.b[4 * L + 2] = q4_scaled((q.x >> 4) & M, (q.y >> 4) & M, sh);
        f.b[4 * L + 3] = q4_scaled((q.z >> 4) & M, (q.w >> 4) & M, sh);
        if (L == (h & 1)) {
            const _Float16 a = (_Float16)(float)ml, b = (_Float16)(float)mh;
            f.bm = half4_t{a, a, b, b};
        }
    }
}

// A operand: the 8 activation values MFMA `i` pairs with the lane's weights
__device__ inline int q4_a_offset(int h, int i) {
    const int L = i >> 2, nib = (i >> 1) & 1, half = i & 1;
    const int g = (h >> 1) + 2 * L;
    return 32 * (2 * g + nib) + 16 * (h & 1) + 8 * half;
}

// The pass covers up to NT tiles of 16 dispatched pairs of one expert.
template <int NT>
struct Tiles {
    int n;                 // tiles in this pass
    int arow[NT];          // A-side activation row (lane & 15) of each tile, clamped to a valid one
    int drow[NT][4];       // D-side pair positions 4*(lane>>4) + i, -1 past the expert's pairs
    int dact[NT][4];       // their activation rows (for the block scales), clamped
};

// rows: for the gate/up pass the activation row is the pair's token, for the
// down pass the pair's own position
template <int NT, bool TOKEN_ROWS>
__device__ inline void tile_rows(const GroupedArgs &a, int n0, int ne, int pb, int lane, Tiles<NT> &T) {
    const int left = ne - pb;
    T.n = min(NT, (left + 15) / 16);
#pragma unroll
    for (int t = 0; t < NT; ++t) {
        const int ma = 16 * t + (lane & 15);
        const int pa = n0 + pb + (ma < left ? ma : 0);
        T.arow[t] = TOKEN_ROWS ? a.perm[pa] / a.K : pa;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int md = 16 * t + 4 * (lane >> 4) + i;
            const int pd = n0 + pb + (md < left ? md : 0);
            T.drow[t][i] = md < left ? pd : -1;
            T.dact[t][i] = TOKEN_ROWS ? a.perm[pd] / a.K : pd;
        }
    }
}

// Workgroup = 8 waves: waves 0-3 take 64 rows of up, waves 4-7 the same 64
// rows of gate (16 rows per wave); one workgroup per (row tile, expert).  Up
// results meet their gate rows in LDS for the SwiGLU.  Every pass streams the
// rows once for up to NT*16 of the expert's pairs.
template <int NT>
__global__ __launch_bounds__(512) void gateup_grouped_kernel(GroupedArgs a) {
    const int e = blockIdx.y;
    const int n0 = a.offsets[e], ne = a.offsets[e + 1] - n0;
    if (ne <= 0) return;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int n = lane & 15, h = lane >> 4;
    const bool is_gate = wave >= 4;
    const int lrow = (wave & 3) * 16 + n;          // row within the tile
    const int row = blockIdx.x * 64 + lrow;
    const int nb = a.H / QK;
    const size_t rb = (size_t)nb * Q4K_BYTES;
    const uint8_t *base = grouped_expert(a, e);
    const uint8_t *mat = base ? base + (is_gate ? (size_t)a.I * rb : 0) + (size_t)row * rb : nullptr;
    __shared__ float s_up[64][16 * NT + 1];

    for (int pb = 0; pb < ne; pb += 16 * NT) {
        Tiles<NT> T;
        tile_rows<NT, true>(a, n0, ne, pb, lane, T);
        float y[NT][4];
#pragma unroll
        for (int t = 0; t < NT; ++t)
#pragma unroll
            for (int i = 0; i < 4; ++i) y[t][i] = 0.0f;
        if (base) {
            for (int s = 0; s < nb; ++s) {
                Q4Frag f;
                q4_frag(mat + (size_t)s * Q4K_BYTES, h, f);
#pragma unroll
                for (int t = 0; t < NT; ++t) {
                    if (t >= T.n) break;
                    const _Float16 *xr = (const _Float16 *)a.xa + (size_t)T.arow[t] * a.H + (size_t)s * QK;
                    float4_t acc = {0, 0, 0, 0};
#pragma unroll
                    for (int i = 0; i < 8; ++i) acc = mfma32(*(const half8_t *)(xr + q4_a_offset(h, i)), f.b[i], acc);
                    const int gm = (h >> 1) + 2 * (h & 1);
                    const half4_t am = *(const half4_t *)((const _Float16 *)a.xbs +
                                                          (size_t)T.arow[t] * (a.H / 16) + s * 16 + 4 * gm);
                    const float4_t z = __builtin_amdgcn_mfma_f32_16x16x16f16(am, f.bm, float4_t{0, 0, 0, 0}, 0, 0, 0);
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        // ggml's order: acc += (d*dx)*sumi; acc -= (dmin*dx)*summ
                        const float dx = a.xdx[(size_t)T.dact[t][i] * nb + s];
                        y[t][i] = y[t][i] + (f.d * dx) * acc[i];
                        y[t][i] = y[t][i] - (f.dmin * dx) * z[i];
                    }
                    __builtin_amdgcn_sched_barrier(0);
                }
            }
        }
        if (!is_gate) {
#pragma unroll
            for (int t = 0; t < NT; ++t)
#pragma unroll
                for (int i = 0; i < 4; ++i) s_up[lrow][16 * t + 4 * h + i] = y[t][i];
        }
        __syncthreads();
        if (is_gate) {
#pragma unroll
            for (int t = 0; t < NT; ++t) {
                if (t >= T.n) break;
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const int dr = T.drow[t][i];
                    if (dr >= 0)
                        a.h[(size_t)dr * a.I + row] = base ? silu_mul(y[t][i], s_up[lrow][16 * t + 4 * h + i]) : 0.0f;
                }
            }
        }
        __syncthreads();
    }
}

// Q6_K B operands of one super-block for the lane's row (bytes in LDS, rows
// only 2-byte aligned): MFMA 4*hh + g covers elements 128*hh + 32*g + 8*h .. +7
// with sc = scales[8*hh + (h >> 1) + 2*g].  (q - 32) * sc reaches 4096, past
// fp16's exact integers, so sc = 16*sh + sl splits it into two exact operands
// (|(q-32)*sh| <= 256, (q-32)*sl <= 480): sumi = 16*acc_h + acc_l.
__device__ inline void q6_frag(const uint8_t *blk, int h, half8_t bh[8], half8_t bl[8], float &d) {
    d = h2f(*(const uint16_t *)(blk + 208));
    const uint32_t M = 0x0F0F0F0Fu, HM = 0x30303030u;
    const half8_t c1056 = splat8((_Float16)1056.0f);
#pragma unroll
    for (int hh = 0; hh < 2; ++hh) {
        const uint8_t *pa = blk + 64 * hh + 8 * h;
        const uint32_t a0 = lds_u32_at2(pa), a1 = lds_u32_at2(pa + 4);
        const uint32_t b0 = lds_u32_at2(pa + 32), b1 = lds_u32_at2(pa + 36);
        const uint32_t q0 = lds_u32_at2(blk + 128 + 32 * hh + 8 * h), q1 = lds_u32_at2(blk + 132 + 32 * hh + 8 * h);
        const uint32_t w[4][2] = {{(a0 & M) | ((q0 << 4) & HM), (a1 & M) | ((q1 << 4) & HM)},
                                  {(b0 & M) | ((q0 << 2) & HM), (b1 & M) | ((q1 << 2) & HM)},
                                  {((a0 >> 4) & M) | (q0 & HM), ((a1 >> 4) & M) | (q1 & HM)},
                                  {((b0 >> 4) & M) | ((q0 >> 2) & HM), ((b1 >> 4) & M) | ((q1 >> 2) & HM)}};
#pragma unroll
        for (int g = 0; g < 4; ++g) {
            const int sc = (int)(int8_t)blk[192 + 8 * hh + (h >> 1) + 2 * g];
            const half8_t q = pack_1024(w[g][0], w[g][1]) - c1056;          // q - 32, exact
            bh[4 * hh + g] = q * splat8((_Float16)(float)(sc >> 4));        // arithmetic shift: -8 .. 7
            bl[4 * hh + g] = q * splat8((_Float16)(float)(sc & 15));
        }
    }
}

constexpr int DG_LDS = 64 * 3 * Q6K_BYTES;   // 64 Q6_K rows at I <= 768

// Workgroup = 4 waves = 64 output rows (16 per wave); one workgroup per (row
// tile, expert).  y times the pair's gate weight goes to the pair's row.
template <int DT, int NT>
__global__ __launch_bounds__(256) void down_grouped_kernel(GroupedArgs a) {
    const int e = blockIdx.y;
    const int n0 = a.offsets[e], ne = a.offsets[e + 1] - n0;
    if (ne <= 0) return;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int n = lane & 15, h = lane >> 4;
    const int r0 = blockIdx.x * 64;
    const int row = r0 + wave * 16 + n;
    const int nb = a.I / QK;
    const int rowb = nb * (DT == TYPE_Q6K ? Q6K_BYTES : Q4K_BYTES);
    const uint8_t *base = grouped_expert(a, e);
    const uint8_t *down = base ? base + 2ull * a.I * (a.H / QK) * Q4K_BYTES : nullptr;
    __shared__ __attribute__((aligned(16))) uint8_t s_w[DT == TYPE_Q6K ? DG_LDS : 16];
    if (DT == TYPE_Q6K && down) {
        // 64 rows * rowb bytes from a 16-byte aligned start (64 * 210 = 840 * 16)
        const uint4 *src = (const uint4 *)(down + (size_t)r0 * rowb);
        uint4 *dst = (uint4 *)s_w;
        const int nvec = 64 * rowb / 16;
        for (int i = threadIdx.x; i < nvec; i += 256) dst[i] = src[i];
        __syncthreads();
    }

    for (int pb = 0; pb < ne; pb += 16 * NT) {
        Tiles<NT> T;
        tile_rows<NT, false>(a, n0, ne, pb, lane, T);
        float y[NT][4];
#pragma unroll
        for (int t = 0; t < NT; ++t)
#pragma unroll
            for (int i = 0; i < 4; ++i) y[t][i] = 0.0f;
        if (base) {
            for (int s = 0; s < nb; ++s) {
                half8_t b[8], bl[8];
                half4_t bm;
                float d, dmin = 0.0f;
                if (DT == TYPE_Q6K) {
                    q6_frag(s_w + (size_t)(wave * 16 + n) * rowb + (size_t)s * Q6K_BYTES, h, b, bl, d);
                } else {
                    Q4Frag f;
                    q4_frag(down + (size_t)row * rowb + (size_t)s * Q4K_BYTES, h, f);
#pragma unroll
                    for (int i = 0; i < 8; ++i) b[i] = f.b[i];
                    bm = f.bm;
                    d = f.d;
                    dmin = f.dmin;
                }
#pragma unroll
                for (int t = 0; t < NT; ++t) {
                    if (t >= T.n) break;
                    const _Float16 *hr = (const _Float16 *)a.ha + (size_t)T.arow[t] * a.I + (size_t)s * QK;
                    float4_t acc = {0, 0, 0, 0}, accl = {0, 0, 0, 0};
#pragma unroll
                    for (int i = 0; i < 8; ++i) {
                        const int off = DT == TYPE_Q6K ? 128 * (i >> 2) + 32 * (i & 3) + 8 * h : q4_a_offset(h, i);
                        const half8_t av = *(const half8_t *)(hr + off);
                        acc = mfma32(av, b[i], acc);
                        if (DT == TYPE_Q6K) accl = mfma32(av, bl[i], accl);
                    }
                    if (DT == TYPE_Q6K) {
#pragma unroll
                        for (int i = 0; i < 4; ++i) acc[i] = 16.0f * acc[i] + accl[i];   // exact integers
                    }
                    float4_t z = {0, 0, 0, 0};
                    if (DT == TYPE_Q4K) {
                        const int gm = (h >> 1) + 2 * (h & 1);
                        const half4_t am = *(const half4_t *)((const _Float16 *)a.hbs +
                                                              (size_t)T.arow[t] * (a.I / 16) + s * 16 + 4 * gm);
                        z = __builtin_amdgcn_mfma_f32_16x16x16f16(am, bm, z, 0, 0, 0);
                    }
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        const float dx = a.hdx[(size_t)T.dact[t][i] * nb + s];
                        y[t][i] = y[t][i] + (d * dx) * acc[i];
                        if (DT == TYPE_Q4K) y[t][i] = y[t][i] - (dmin * dx) * z[i];
                    }
                    __builtin_amdgcn_sched_barrier(0);
                }
            }
        }
#pragma unroll
        for (int t = 0; t < NT; ++t) {
            if (t >= T.n) break;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int dr = T.drow[t][i];
                if (dr < 0) continue;
                const int p = a.perm[dr];
                a.ypair[(size_t)p * a.H + row] = base ? a.w[p] * y[t][i] : 0.0f;
            }
        }
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

constexpr int GG_NT = 4;

hipError_t launch_gateup_grouped(const GroupedArgs &a, hipStream_t st, hipEvent_t e0, hipEvent_t e1) {
    return launch_b(gateup_grouped_kernel<GG_NT>, dim3((unsigned)(a.I / 64), (unsigned)a.E), dim3(512), st, e0, e1, a);
}

hipError_t launch_down_grouped(const GroupedArgs &a, hipStream_t st, hipEvent_t e0, hipEvent_t e1) {
    const dim3 grid((unsigned)(a.H / 64), (unsigned)a.E);
    if (a.down_type == TYPE_Q6K) return launch_b(down_grouped_kernel<TYPE_Q6K, GG_NT>, grid, dim3(256), st, e0, e1, a);
    return launch_b(down_grouped_kernel<TYPE_Q4K, GG_NT>, grid, dim3(256), st, e0, e1, a);
}

hipError_t launch_combine(const float *ypair, int n_tok, int K, int H, float *out, int accumulate, hipStream_t st) {
    const size_t n4 = (size_t)n_tok * H / 4;
    if (n4 == 0) return hipSuccess;
    return launch_b(combine_kernel, dim3((unsigned)((n4 + 255) / 256)), dim3(256), st, nullptr, nullptr, ypair, n_tok,
                    K, H, out, accumulate);
}

}  // namespace mp
