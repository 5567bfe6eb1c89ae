// mp_device.h -- device helpers shared by the batch-1 kernels (mp_kernels.hip)
// and the batched kernels (mp_batched.hip).
#pragma once

#include <hip/hip_runtime.h>

#include "mp_format.h"

namespace mp {

// canonical exp (same polynomial and constants as the oracle's or_expf)
__device__ inline float canon_expf(float x) {
    if (x < -87.0f) return 0.0f;
    if (x > 88.0f) x = 88.0f;
    const float n = rintf(x * 1.44269504088896341f);
    float r = fmaf(n, -0.693145751953125f, x);
    r = fmaf(n, -1.428606765330187045e-06f, r);
    float p = 1.9841269841269841e-04f;
    p = fmaf(p, r, 1.3888888888888889e-03f);
    p = fmaf(p, r, 8.3333333333333333e-03f);
    p = fmaf(p, r, 4.1666666666666667e-02f);
    p = fmaf(p, r, 1.6666666666666667e-01f);
    p = fmaf(p, r, 0.5f);
    p = fmaf(p, r, 1.0f);
    p = fmaf(p, r, 1.0f);
    const uint32_t e = (uint32_t)((int32_t)n + 127);
    return p * bits_f32(e << 23);
}

// binary16 -> binary32 in one hardware conversion (exact for every code,
// subnormals included: each is a normal fp32 value)
__device__ inline float h2f_dev(uint16_t h) { return (float)__builtin_bit_cast(_Float16, h); }

// DPP lane moves within a row of 16 lanes (a VALU operand, no LDS crossbar)
constexpr int DPP_XOR1 = 0xB1;       // quad_perm [1,0,3,2]
constexpr int DPP_XOR2 = 0x4E;       // quad_perm [2,3,0,1]
constexpr int DPP_HALF_MIRROR = 0x141;
constexpr int DPP_MIRROR = 0x140;
template <int CTRL>
__device__ inline int dpp_i(int v) { return __builtin_amdgcn_update_dpp(0, v, CTRL, 0xF, 0xF, false); }
template <int CTRL>
__device__ inline float dpp_f(float v) { return __int_as_float(dpp_i<CTRL>(__float_as_int(v))); }
__device__ inline float lane_f(float v, int l) { return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), l)); }

// Sum of a wave's 64 values in the canonical butterfly order: p_j += p_{j^o}
// for o = 1, 2, 4, 8, 16, 32 (every lane ends with the same bits).  After
// the first two steps each quad holds one value, so the mirror lanes that
// row_half_mirror and row_mirror reach add exactly what lanes j^4 and j^8
// hold; the last two steps add the four rows' values as (r0 + r1) + (r2 + r3).
__device__ inline float wave_sum_canon(float v) {
    v = v + dpp_f<DPP_XOR1>(v);
    v = v + dpp_f<DPP_XOR2>(v);
    v = v + dpp_f<DPP_HALF_MIRROR>(v);
    v = v + dpp_f<DPP_MIRROR>(v);
    return (lane_f(v, 0) + lane_f(v, 16)) + (lane_f(v, 32) + lane_f(v, 48));
}

// maximum over the wave (any order gives the same value)
__device__ inline float wave_max(float v) {
    v = fmaxf(v, dpp_f<DPP_XOR1>(v));
    v = fmaxf(v, dpp_f<DPP_XOR2>(v));
    v = fmaxf(v, dpp_f<DPP_HALF_MIRROR>(v));
    v = fmaxf(v, dpp_f<DPP_MIRROR>(v));
    return fmaxf(fmaxf(lane_f(v, 0), lane_f(v, 16)), fmaxf(lane_f(v, 32), lane_f(v, 48)));
}

__device__ inline int32_t sdot4(uint32_t a, uint32_t b, int32_t c) {
    return __builtin_amdgcn_sdot4((int)a, (int)b, c, false);
}

// Q8_K of 256 values held 4 per lane (lane-major) by one wavefront: the
// largest magnitude (first index on a tie) maps to -127, q = min(127,
// rint(x * iscale)); d = 1 / iscale, 0 for an all-zero block.
// the larger of two (magnitude, value, index) candidates: the larger
// magnitude, the lower index on a tie -- associative and commutative, so any
// reduction order selects the same element
__device__ inline void amax_pick(float &amax, float &mx, int &idx, float oa, float om, int oi) {
    if (oa > amax || (oa == amax && oi < idx)) { amax = oa; mx = om; idx = oi; }
}
template <int CTRL>
__device__ inline void amax_step(float &amax, float &mx, int &idx) {
    amax_pick(amax, mx, idx, dpp_f<CTRL>(amax), dpp_f<CTRL>(mx), dpp_i<CTRL>(idx));
}
// the wave's largest magnitude (first index on a tie), on every lane
__device__ inline void amax_wave(float &amax, float &mx, int &idx) {
    amax_step<DPP_XOR1>(amax, mx, idx);
    amax_step<DPP_XOR2>(amax, mx, idx);
    amax_step<DPP_HALF_MIRROR>(amax, mx, idx);
    amax_step<DPP_MIRROR>(amax, mx, idx);
    float a = lane_f(amax, 0), m = lane_f(mx, 0);
    int i = __builtin_amdgcn_readlane(idx, 0);
#pragma unroll
    for (int r = 16; r < 64; r += 16)
        amax_pick(a, m, i, lane_f(amax, r), lane_f(mx, r), __builtin_amdgcn_readlane(idx, r));
    amax = a;
    mx = m;
    idx = i;
}

// Q8_K of 256 values held 4 per lane (lane-major) by one wavefront: the
// largest magnitude (first index on a tie) maps to -127, q = min(127,
// rint(x * iscale)); d = 1 / iscale, 0 for an all-zero block.
__device__ inline void q8k_wave_vals(const float xv[4], int lane, int q[4], float &d) {
    float amax = 0.0f, mx = 0.0f;
    int idx = 1 << 30;
    for (int i = 0; i < 4; ++i) {
        const float ax = fabsf(xv[i]);
        if (ax > amax) { amax = ax; mx = xv[i]; idx = 4 * lane + i; }
    }
    amax_wave(amax, mx, idx);
    q[0] = q[1] = q[2] = q[3] = 0;
    d = 0.0f;
    if (amax != 0.0f) {
        const float iscale = -127.0f / mx;
        for (int i = 0; i < 4; ++i) {
            const int t = (int)rintf(iscale * xv[i]);
            q[i] = t < 127 ? t : 127;
        }
        d = 1.0f / iscale;
    }
}

// NB blocks at once, each exactly as q8k_wave_vals
template <int NB>
__device__ inline void q8k_wave_vals_n(const float (*xv)[4], int lane, int (*q)[4], float *d) {
    float amax[NB], mx[NB];
    int idx[NB];
#pragma unroll
    for (int b = 0; b < NB; ++b) {
        amax[b] = 0.0f;
        mx[b] = 0.0f;
        idx[b] = 1 << 30;
        for (int i = 0; i < 4; ++i) {
            const float ax = fabsf(xv[b][i]);
            if (ax > amax[b]) { amax[b] = ax; mx[b] = xv[b][i]; idx[b] = 4 * lane + i; }
        }
    }
#pragma unroll
    for (int b = 0; b < NB; ++b) amax_wave(amax[b], mx[b], idx[b]);
#pragma unroll
    for (int b = 0; b < NB; ++b) {
        q[b][0] = q[b][1] = q[b][2] = q[b][3] = 0;
        d[b] = 0.0f;
        if (amax[b] != 0.0f) {
            const float iscale = -127.0f / mx[b];
            for (int i = 0; i < 4; ++i) {
                const int t = (int)rintf(iscale * xv[b][i]);
                q[b][i] = t < 127 ? t : 127;
            }
            d[b] = 1.0f / iscale;
        }
    }
}

// Selection value -> 64-bit key whose unsigned order is the selection order:
// the value's bits mapped onto an unsigned order (a NaN taken as -inf, -0 as
// +0, so that equal values give equal bits), then the lower id first.  The
// rank of an expert is the number of keys above its own -- one unsigned
// comparison per expert, no chain of float compares.
__device__ inline uint64_t sel_key(float v, int id) {
    v = v != v ? -INFINITY : v + 0.0f;
    const uint32_t b = __float_as_uint(v);
    const uint32_t o = (b & 0x80000000u) ? ~b : (b | 0x80000000u);
    return ((uint64_t)o << 32) | (uint64_t)(0xffffffffu - (uint32_t)id);
}

// the score half of sel_key: an order-preserving image of v, every real
// value above 0 (a NaN equal to -inf, -0 equal to +0)
__device__ inline uint32_t sel_bits(float v) { return (uint32_t)(sel_key(v, 0) >> 32); }

// unsigned maximum over the wave, on every lane (a uniform value)
__device__ inline uint32_t wave_max_u32(uint32_t v) {
    v = max(v, (uint32_t)dpp_i<DPP_XOR1>((int)v));
    v = max(v, (uint32_t)dpp_i<DPP_XOR2>((int)v));
    v = max(v, (uint32_t)dpp_i<DPP_HALF_MIRROR>((int)v));
    v = max(v, (uint32_t)dpp_i<DPP_MIRROR>((int)v));
    const uint32_t a = __builtin_amdgcn_readlane(v, 0), b = __builtin_amdgcn_readlane(v, 16);
    const uint32_t c = __builtin_amdgcn_readlane(v, 32), d = __builtin_amdgcn_readlane(v, 48);
    return max(max(a, b), max(c, d));
}

// unsigned maximum over the wave as a uniform value: the row maxima by lane
// moves inside each row of 16 lanes, then row_bcast:15 and row_bcast:31
// carry them across the rows (0 is the identity of the maximum, so the lanes
// those moves leave out keep their value), and lane 63 holds the maximum of
// all -- one read of a lane, not four
__device__ inline uint32_t wave_max_u32_bcast(uint32_t v) {
    v = max(v, (uint32_t)dpp_i<DPP_XOR1>((int)v));
    v = max(v, (uint32_t)dpp_i<DPP_XOR2>((int)v));
    v = max(v, (uint32_t)dpp_i<DPP_HALF_MIRROR>((int)v));
    v = max(v, (uint32_t)dpp_i<DPP_MIRROR>((int)v));
    v = max(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x142, 0xA, 0xF, false));     // row_bcast:15
    v = max(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x143, 0xC, 0xF, false));     // row_bcast:31
    return __builtin_amdgcn_readlane(v, 63);
}

// rank of `key` among n keys in LDS (the count of keys above it)
__device__ inline int key_rank(const uint64_t *s_key, int n, uint64_t key) {
    int rank = 0;
#pragma unroll 8
    for (int j = 0; j < n; j += 2) {
        const uint4 u = *(const uint4 *)&s_key[j];
        rank += (((uint64_t)u.y << 32) | u.x) > key;
        rank += (((uint64_t)u.w << 32) | u.z) > key;
    }
    return rank;
}

// Integer sum over each aligned group of 8 lanes, on every lane of the group,
// by DPP lane moves (no LDS crossbar): swap neighbours, swap pairs, then add
// the mirror lane of the other quad.  Integer sums are exact in any order.
__device__ inline int sum8_dpp(int v) {
    v += __builtin_amdgcn_update_dpp(0, v, 0xB1, 0xF, 0xF, false);     // quad_perm [1,0,3,2]
    v += __builtin_amdgcn_update_dpp(0, v, 0x4E, 0xF, 0xF, false);     // quad_perm [2,3,0,1]
    v += __builtin_amdgcn_update_dpp(0, v, 0x141, 0xF, 0xF, false);    // row_half_mirror
    return v;
}

// the 16-value group sum of the Q8_K block, valid on lanes with (lane & 3) == 0
__device__ inline int q8k_group_sum(const int q[4]) {
    int gs = q[0] + q[1] + q[2] + q[3];
    gs += dpp_i<DPP_XOR1>(gs);
    gs += dpp_i<DPP_XOR2>(gs);
    return gs;
}

// byte i (0..11) of the Q4_K scale field held in three words
__device__ inline int sc_byte(const uint4 &hdr, int i) {
    const uint32_t w = i < 4 ? hdr.y : (i < 8 ? hdr.z : hdr.w);
    return (int)((w >> (8 * (i & 3))) & 0xffu);
}

// six-bit (scale, min) of sub-block j from a Q4_K header (d, dmin, 12 scale bytes)
__device__ inline void q4k_sm(const uint4 &hdr, int j, int &sc, int &m) {
    if (j < 4) {
        sc = sc_byte(hdr, j) & 63;
        m = sc_byte(hdr, j + 4) & 63;
    } else {
        sc = (sc_byte(hdr, j + 4) & 0xF) | ((sc_byte(hdr, j - 4) >> 6) << 4);
        m = (sc_byte(hdr, j + 4) >> 4) | ((sc_byte(hdr, j) >> 6) << 4);
    }
}

constexpr int Q6K_PAD = 224;                // a Q6_K block's stride in LDS (16-byte aligned)


// Q6_K rows into LDS with every 210-byte block at a 224-byte stride, so that
// the dot's 8-byte LDS reads are aligned (at the blocks' own 2-byte
// alignment they run about four times slower under load).  One wave moves
// n_blocks blocks (<= 24: 8 rows at I = 768) from `src` (the rows
// contiguous, so block n at n * 210): chunk c of the padded layout, 16
// bytes, is block c / 14 from byte 16 (c % 14) -- except the 14th chunk of a
// block, which only carries the block's last two bytes (its fp16 scale) and
// is read as the block's last 16 bytes, so no read passes the block's end.
// q6k_rows_load issues the loads; q6k_rows_store writes LDS and, with
// `stage`, the same bytes to the staging copy at their own offsets.
struct Q6Rows {
    uint4 v[6];
};
__device__ inline void q6k_rows_load(Q6Rows &r, const uint8_t *src, int n_blocks, int lane) {
#pragma unroll
    for (int i = 0; i < 6; ++i) {
        const int c = lane + 64 * i;
        r.v[i] = make_uint4(0, 0, 0, 0);
        if (src && c < 14 * n_blocks) {
            const int n = c / 14, j = c - 14 * n;
            const uint8_t *p = src + (size_t)n * Q6K_BYTES + (j < 13 ? 16 * j : Q6K_BYTES - 16);
            __builtin_memcpy(&r.v[i], __builtin_assume_aligned(p, 2), 16);
        }
    }
}
__device__ inline void q6k_rows_store(const Q6Rows &r, uint8_t *s_dst, uint8_t *stage, int n_blocks, int lane) {
#pragma unroll
    for (int i = 0; i < 6; ++i) {
        const int c = lane + 64 * i;
        if (c < 14 * n_blocks) {
            const int n = c / 14, j = c - 14 * n;
            if (j < 13) {
                *(uint4 *)(s_dst + 16 * c) = r.v[i];
                if (stage) __builtin_memcpy(__builtin_assume_aligned(stage + (size_t)n * Q6K_BYTES + 16 * j, 2), &r.v[i], 16);
            } else {
                const uint16_t d = (uint16_t)(r.v[i].w >> 16);
                *(uint16_t *)(s_dst + 16 * c) = d;
                if (stage) *(uint16_t *)(stage + (size_t)n * Q6K_BYTES + Q6K_BYTES - 2) = d;
            }
        }
    }
}

}  // namespace mp
