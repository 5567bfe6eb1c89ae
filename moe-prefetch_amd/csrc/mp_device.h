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

__device__ inline float bfly_add(float v) {
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) v = v + __shfl_xor(v, o, 64);
    return v;
}

__device__ inline int32_t sdot4(uint32_t a, uint32_t b, int32_t c) {
    return __builtin_amdgcn_sdot4((int)a, (int)b, c, false);
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
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) {
        const float oa = __shfl_xor(amax, o, 64);
        const float om = __shfl_xor(mx, o, 64);
        const int oi = __shfl_xor(idx, o, 64);
        if (oa > amax || (oa == amax && oi < idx)) { amax = oa; mx = om; idx = oi; }
    }
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

// NB blocks at once (each exactly as q8k_wave_vals), their cross-lane rounds
// interleaved so that one block's shuffles fill another's latency
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
    for (int o = 32; o >= 1; o >>= 1) {
        float oa[NB], om[NB];
        int oi[NB];
#pragma unroll
        for (int b = 0; b < NB; ++b) {
            oa[b] = __shfl_xor(amax[b], o, 64);
            om[b] = __shfl_xor(mx[b], o, 64);
            oi[b] = __shfl_xor(idx[b], o, 64);
        }
#pragma unroll
        for (int b = 0; b < NB; ++b)
            if (oa[b] > amax[b] || (oa[b] == amax[b] && oi[b] < idx[b])) { amax[b] = oa[b]; mx[b] = om[b]; idx[b] = oi[b]; }
    }
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

// the 16-value group sum of the Q8_K block, valid on lanes with (lane & 3) == 0
__device__ inline int q8k_group_sum(const int q[4]) {
    int gs = q[0] + q[1] + q[2] + q[3];
    gs += __shfl_xor(gs, 1, 64);
    gs += __shfl_xor(gs, 2, 64);
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

__device__ inline uint32_t lds_u32_at2(const uint8_t *p) {   // 2-byte aligned
    const uint16_t *q = (const uint16_t *)p;
    return (uint32_t)q[0] | ((uint32_t)q[1] << 16);
}

}  // namespace mp
