// mp_format.h -- ggml K-quant block layouts as the kernels read them, plus
// fp16 conversion usable on the host and on gfx950.
//
// Layouts (ggml at llama.cpp bccbacd, the format of the reference's
// Qwen3-30B-A3B Q4_K_M weights; sizes in artifacts/expert_bytes_qwen3-30b-a3b-q4km.json):
//   Q4_K  144 B / 256 weights: fp16 d | fp16 dmin | 12 B six-bit (scale, min) x 8 | 128 B nibbles
//   Q6_K  210 B / 256 weights: 128 B low nibbles | 64 B high bit pairs | 16 x int8 scale | fp16 d
//   Q8_K  292 B / 256 values : f32 d | 256 x int8 | 16 x int16 group sums
//
// Expert layout in the pinned host store and in every HBM slot:
//   [ up : I rows x H/256 Q4_K ][ gate : same ][ down : H rows x I/256 Q4_K or Q6_K ]
// so one upload is one contiguous copy of expert_bytes.
#pragma once

#include <stdint.h>

#ifdef __HIPCC__
#include <hip/hip_runtime.h>
#define MP_HD __host__ __device__ inline
#else
#define MP_HD inline
#endif

namespace mp {

constexpr int QK = 256;
constexpr int Q4K_BYTES = 144;
constexpr int Q6K_BYTES = 210;
constexpr int Q8K_BYTES = 292;
constexpr int TYPE_Q4K = 12;   // ggml type ids
constexpr int TYPE_Q6K = 14;

MP_HD int block_bytes(int type) { return type == TYPE_Q6K ? Q6K_BYTES : Q4K_BYTES; }

MP_HD uint64_t expert_bytes(int H, int I, int down_type) {
    return 2ull * (uint64_t)I * (H / QK) * Q4K_BYTES + (uint64_t)H * (I / QK) * block_bytes(down_type);
}

MP_HD float bits_f32(uint32_t b) {
    union { uint32_t u; float f; } v;
    v.u = b;
    return v.f;
}

MP_HD uint32_t f32_bits(float f) {
    union { uint32_t u; float f; } v;
    v.f = f;
    return v.u;
}

// binary16 -> binary32, exact (all codes)
MP_HD float h2f(uint16_t h) {
    const uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    uint32_t exp = (h >> 10) & 0x1fu;
    uint32_t man = h & 0x3ffu;
    if (exp == 0) {
        if (man == 0) return bits_f32(sign);
        int e = -1;
        do { man <<= 1; e++; } while (!(man & 0x400u));
        man &= 0x3ffu;
        return bits_f32(sign | ((uint32_t)(127 - 15 - e) << 23) | (man << 13));
    }
    if (exp == 31) return bits_f32(sign | 0x7f800000u | (man << 13));
    return bits_f32(sign | ((exp + 112u) << 23) | (man << 13));
}

// binary32 -> binary16, round to nearest even
MP_HD uint16_t f2h(float f) {
    const uint32_t x = f32_bits(f);
    const uint32_t sign = (x >> 16) & 0x8000u;
    const uint32_t ax = x & 0x7fffffffu;
    if (ax >= 0x7f800000u) return (uint16_t)(sign | 0x7c00u | (ax > 0x7f800000u ? 0x200u : 0u));
    if (ax >= 0x477ff000u) return (uint16_t)(sign | 0x7c00u);
    if (ax < 0x38800000u) {
        if (ax < 0x33000000u) return (uint16_t)sign;
        const uint32_t e = ax >> 23;
        const uint32_t m = (ax & 0x7fffffu) | 0x800000u;
        const uint32_t shift = 126 - e;
        uint32_t r = m >> shift;
        const uint32_t rem = m & ((1u << shift) - 1);
        const uint32_t half = 1u << (shift - 1);
        if (rem > half || (rem == half && (r & 1))) r++;
        return (uint16_t)(sign | r);
    }
    uint32_t r = (ax >> 13) - (112u << 10);
    const uint32_t rem = ax & 0x1fffu;
    if (rem > 0x1000u || (rem == 0x1000u && (r & 1))) r++;
    return (uint16_t)(sign | r);
}

// Q4_K six-bit (scale, min) of sub-block j from the 12 packed bytes
MP_HD void q4k_scale_min(int j, const uint8_t *q, int &sc, int &m) {
    if (j < 4) {
        sc = q[j] & 63;
        m = q[j + 4] & 63;
    } else {
        sc = (q[j + 4] & 0xF) | ((q[j - 4] >> 6) << 4);
        m = (q[j + 4] >> 4) | ((q[j] >> 6) << 4);
    }
}

}  // namespace mp
