// mp_cpu.cpp -- the routed-expert chain on the host CPU.
//
// Integer dots with AVX-512 VNNI (vpdpbusd: unsigned weight codes x signed
// Q8_K values, no saturation) when the CPU has it, a portable path otherwise;
// both give identical results.  Per super-block the dot is an exact int32,
// and the fp32 steps run in row order exactly as the CPU reference chain
// (experiments/x2_cpu_expert_cost.cpp:115-156, ggml vec_dot_q4_K_q8_K /
// vec_dot_q6_K_q8_K) and the device kernels take them: acc + (d*dx)*sumi,
// then - (dmin*dx)*summ.  Built with -ffp-contract=off.
#include "mp_cpu.h"

#include <immintrin.h>
#include <math.h>
#include <string.h>
#include <sys/mman.h>
#include <unistd.h>

#include <algorithm>
#include <atomic>
#include <condition_variable>
#include <mutex>
#include <thread>
#include <vector>

#include "mp_format.h"

namespace mpc {

using mp::QK;
using mp::Q4K_BYTES;
using mp::Q6K_BYTES;
using mp::Q8K_BYTES;

static bool g_portable = false;     // set by the tests to pin the portable path

bool has_vnni() {
    static const bool v = __builtin_cpu_supports("avx512f") && __builtin_cpu_supports("avx512bw") &&
                          __builtin_cpu_supports("avx512vl") && __builtin_cpu_supports("avx512vnni");
    return v;
}

void set_portable(bool on) { g_portable = on; }

// canonical exp: Cody-Waite reduction by ln 2 in two parts, degree-7
// polynomial by Horner with fused multiply-adds, scale by 2^n (the device's
// canon_expf, step for step)
static inline float canon_expf(float x) {
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
    return p * mp::bits_f32(e << 23);
}

// the order-preserving unsigned image of a selection value, then the lower id first
static inline uint64_t sel_key(float v, int id) {
    v = v != v ? -INFINITY : v + 0.0f;
    uint32_t b;
    memcpy(&b, &v, 4);
    const uint32_t o = (b & 0x80000000u) ? ~b : (b | 0x80000000u);
    return ((uint64_t)o << 32) | (uint64_t)(0xffffffffu - (uint32_t)id);
}

void route_topk(const float *logits, int E, const float *prior, bool prior_on_logits, int K, int32_t *ids) {
    float m = logits[0];
    for (int e = 1; e < E; ++e) m = fmaxf(m, logits[e]);
    float ex[256], p[256];
    float sum = 0.0f;
    for (int c = 0; c < E / 64; ++c) {
        float t[64];
        for (int i = 0; i < 64; ++i) t[i] = ex[64 * c + i] = canon_expf(logits[64 * c + i] - m);
        for (int w = 1; w < 64; w *= 2)
            for (int i = 0; i < 64; i += 2 * w) t[i] = t[i] + t[i + w];
        sum = c == 0 ? t[0] : sum + t[0];
    }
    uint64_t key[256];
    for (int e = 0; e < E; ++e) {
        p[e] = ex[e] / sum;
        const float v = !prior ? p[e] : (prior_on_logits ? logits[e] + prior[e] : p[e] + prior[e]);
        key[e] = sel_key(v, e);
    }
    std::partial_sort(key, key + K, key + E, [](uint64_t a, uint64_t b) { return a > b; });
    for (int k = 0; k < K; ++k) ids[k] = (int32_t)(0xffffffffu - (uint32_t)key[k]);
}

void quant_q8k(const float *x, int n, uint8_t *out) {
    for (int b = 0; b < n / QK; ++b) {
        const float *v = x + (size_t)b * QK;
        uint8_t *o = out + (size_t)b * Q8K_BYTES;
        float amax = 0.0f, mx = 0.0f;
        for (int i = 0; i < QK; ++i) {
            const float a = fabsf(v[i]);
            if (a > amax) { amax = a; mx = v[i]; }     // first index of the largest magnitude
        }
        int8_t q[QK];
        float d = 0.0f;
        if (amax != 0.0f) {
            const float iscale = -127.0f / mx;
            for (int i = 0; i < QK; ++i) {
                const int t = (int)rintf(iscale * v[i]);
                q[i] = (int8_t)(t < 127 ? t : 127);
            }
            d = 1.0f / iscale;
        } else {
            memset(q, 0, sizeof q);
        }
        memcpy(o, &d, 4);
        memcpy(o + 4, q, QK);
        for (int g = 0; g < 16; ++g) {
            int s = 0;
            for (int i = 0; i < 16; ++i) s += q[16 * g + i];
            const int16_t s16 = (int16_t)s;
            memcpy(o + 4 + QK + 2 * g, &s16, 2);
        }
    }
}

static inline void q4k_scale_min(const uint8_t *s, int j, int &sc, int &m) {
    if (j < 4) {
        sc = s[j] & 63;
        m = s[j + 4] & 63;
    } else {
        sc = (s[j + 4] & 0xF) | ((s[j - 4] >> 6) << 4);
        m = (s[j + 4] >> 4) | ((s[j] >> 6) << 4);
    }
}

static inline float f32_at(const uint8_t *p) { float f; memcpy(&f, p, 4); return f; }
static inline uint16_t u16_at(const uint8_t *p) { uint16_t v; memcpy(&v, p, 2); return v; }
static inline int16_t i16_at(const uint8_t *p) { int16_t v; memcpy(&v, p, 2); return v; }

// ---- portable dots -----------------------------------------------------------
static float dot_q4k_port(const uint8_t *row, const uint8_t *q8, int nb) {
    float acc = 0.0f;
    for (int i = 0; i < nb; ++i, row += Q4K_BYTES, q8 += Q8K_BYTES) {
        const int8_t *qx = (const int8_t *)(q8 + 4);
        int32_t sumi = 0, summ = 0;
        for (int j = 0; j < 8; ++j) {
            int sc, m;
            q4k_scale_min(row + 4, j, sc, m);
            const uint8_t *qs = row + 16 + 32 * (j >> 1);
            const int sh = 4 * (j & 1);
            int32_t dot = 0;
            for (int l = 0; l < 32; ++l) dot += ((qs[l] >> sh) & 0xF) * qx[32 * j + l];
            sumi += sc * dot;
            summ += m * (i16_at(q8 + 4 + QK + 4 * j) + i16_at(q8 + 4 + QK + 4 * j + 2));
        }
        const float dx = f32_at(q8);
        const float d = mp::h2f(u16_at(row)) * dx, dm = mp::h2f(u16_at(row + 2)) * dx;
        acc = acc + d * (float)sumi;
        acc = acc - dm * (float)summ;
    }
    return acc;
}

static float dot_q6k_port(const uint8_t *row, const uint8_t *q8, int nb) {
    float acc = 0.0f;
    for (int i = 0; i < nb; ++i, row += Q6K_BYTES, q8 += Q8K_BYTES) {
        const uint8_t *ql = row, *qh = row + 128;
        const int8_t *sc = (const int8_t *)(row + 192);
        const int8_t *qx = (const int8_t *)(q8 + 4);
        int32_t sumi = 0;
        for (int h = 0; h < 2; ++h)
            for (int g = 0; g < 4; ++g)
                for (int s = 0; s < 2; ++s) {
                    int32_t dq = 0;
                    for (int l = 16 * s; l < 16 * s + 16; ++l) {
                        const uint8_t lo = ql[64 * h + 32 * (g & 1) + l];
                        const int low = g >= 2 ? (lo >> 4) : (lo & 0xF);
                        const int high = (qh[32 * h + l] >> (2 * g)) & 3;
                        dq += ((low | (high << 4)) - 32) * qx[128 * h + 32 * g + l];
                    }
                    sumi += sc[8 * h + 2 * g + s] * dq;
                }
        const float d = mp::h2f(u16_at(row + 208)) * f32_at(q8);
        acc = acc + d * (float)sumi;
    }
    return acc;
}

// ---- AVX-512 dots, NR rows at a time --------------------------------------------
// The rows share the activation loads; per super-block each row's integer sums
// are exact (u8 codes x s8 Q8_K values with maddubs: pairs stay below 2^15;
// dpwssd with 16-bit scales), the rows' sums are reduced together, and the fp32
// steps of every row run in the scalar order (scale term, then min term; no
// fused multiply-add), so each row's result is the portable dot's bit for bit.
#define MPC_AVX512 __attribute__((target("avx512f,avx512bw,avx512vl,avx512vnni,f16c")))

MPC_AVX512 static inline __m128i fold4(__m512i v) {
    const __m256i h = _mm256_add_epi32(_mm512_castsi512_si256(v), _mm512_extracti64x4_epi64(v, 1));
    return _mm_add_epi32(_mm256_castsi256_si128(h), _mm256_extracti128_si256(h, 1));
}

// [sum(a0), sum(a1), sum(a2), sum(a3)] of four 16-lane int32 vectors
MPC_AVX512 static inline __m128i hsum4(__m512i a0, __m512i a1, __m512i a2, __m512i a3) {
    const __m128i c0 = fold4(a0), c1 = fold4(a1), c2 = fold4(a2), c3 = fold4(a3);
    const __m128i u0 = _mm_add_epi32(_mm_unpacklo_epi32(c0, c1), _mm_unpackhi_epi32(c0, c1));   // c0 c1 c0 c1
    const __m128i u1 = _mm_add_epi32(_mm_unpacklo_epi32(c2, c3), _mm_unpackhi_epi32(c2, c3));   // c2 c3 c2 c3
    return _mm_add_epi32(_mm_unpacklo_epi64(u0, u1), _mm_unpackhi_epi64(u0, u1));
}

// the 8 six-bit scales and mins of a Q4_K super-block (12 bytes at s) as two
// 64-bit words of bytes: j < 4 from the low six bits of bytes j and j + 4;
// j >= 4 from the nibbles of byte j + 4 and the top two bits of bytes j - 4, j
static inline void q4k_scales8(const uint8_t *s, uint64_t &sc, uint64_t &mn) {
    uint32_t u0, u1, u2;
    memcpy(&u0, s, 4);
    memcpy(&u1, s + 4, 4);
    memcpy(&u2, s + 8, 4);
    const uint32_t sc_lo = u0 & 0x3f3f3f3fu, mn_lo = u1 & 0x3f3f3f3fu;
    const uint32_t sc_hi = (u2 & 0x0f0f0f0fu) | (((u0 >> 6) & 0x03030303u) << 4);
    const uint32_t mn_hi = ((u2 >> 4) & 0x0f0f0f0fu) | (((u1 >> 6) & 0x03030303u) << 4);
    sc = (uint64_t)sc_lo | ((uint64_t)sc_hi << 32);
    mn = (uint64_t)mn_lo | ((uint64_t)mn_hi << 32);
}

// Prefetch: the same super-block of the group of four rows two groups ahead
// (a row is only 6-18 lines, too short for the hardware's stream detection to
// run ahead), when the caller says such a group follows.  Two groups ahead
// measured ~4 % faster than one on the 48-layer decode (494-501 against
// 470-482 tok/s); a non-temporal hint was no better.
void prefetch_rows(int type, const uint8_t *row0, size_t stride, int nrows, int nb) {
    const size_t bytes = (size_t)nb * (type == mp::TYPE_Q6K ? Q6K_BYTES : Q4K_BYTES);
    for (int r = 0; r < nrows; ++r)
        for (size_t o = 0; o < bytes; o += 64) _mm_prefetch((const char *)(row0 + (size_t)r * stride + o), _MM_HINT_T0);
}

template <int NR>
MPC_AVX512 static void rows_q4k_vnni(const uint8_t *row0, size_t stride, const uint8_t *q8, int nb, float *out,
                                     bool more) {
    const __m512i m4 = _mm512_set1_epi8(0x0F);
    // int16 lane index of the scale for groups g: lanes 0-15 sub-block 2g, 16-31 sub-block 2g + 1
    __m512i gidx[4];
    for (int g = 0; g < 4; ++g)
        gidx[g] = _mm512_inserti64x4(_mm512_castsi256_si512(_mm256_set1_epi16((short)(2 * g))),
                                     _mm256_set1_epi16((short)(2 * g + 1)), 1);
    __m128 acc = _mm_setzero_ps();
    for (int i = 0; i < nb; ++i) {
        const uint8_t *qb = q8 + (size_t)i * Q8K_BYTES;
        __m512i xv[4];
        for (int g = 0; g < 4; ++g) xv[g] = _mm512_loadu_si512((const void *)(qb + 4 + 64 * g));
        const __m256i bs = _mm256_loadu_si256((const __m256i *)(qb + 4 + QK));   // 16 int16 block sums
        __m512i si[4], sm[4];
        alignas(16) uint16_t dh[8] = {0, 0, 0, 0, 0, 0, 0, 0}, mh[8] = {0, 0, 0, 0, 0, 0, 0, 0};
        for (int r = 0; r < NR; ++r) {
            const uint8_t *b = row0 + (size_t)r * stride + (size_t)i * Q4K_BYTES;
            uint64_t sc8, mn8;
            q4k_scales8(b + 4, sc8, mn8);
            const __m512i sc16 = _mm512_castsi128_si512(_mm_cvtepu8_epi16(_mm_cvtsi64_si128((long long)sc8)));
            const __m128i mn16 = _mm_cvtepu8_epi16(_mm_cvtsi64_si128((long long)mn8));
            const __m512i raw01 = _mm512_loadu_si512((const void *)(b + 16));        // groups 0, 1
            const __m512i raw23 = _mm512_loadu_si512((const void *)(b + 16 + 64));   // groups 2, 3
            const __m512i lo01 = _mm512_and_si512(raw01, m4), hi01 = _mm512_and_si512(_mm512_srli_epi16(raw01, 4), m4);
            const __m512i lo23 = _mm512_and_si512(raw23, m4), hi23 = _mm512_and_si512(_mm512_srli_epi16(raw23, 4), m4);
            const __m512i w[4] = {_mm512_shuffle_i64x2(lo01, hi01, 0x44), _mm512_shuffle_i64x2(lo01, hi01, 0xEE),
                                  _mm512_shuffle_i64x2(lo23, hi23, 0x44), _mm512_shuffle_i64x2(lo23, hi23, 0xEE)};
            __m512i a = _mm512_setzero_si512();
            for (int g = 0; g < 4; ++g)
                a = _mm512_dpwssd_epi32(a, _mm512_maddubs_epi16(w[g], xv[g]), _mm512_permutexvar_epi16(gidx[g], sc16));
            si[r] = a;
            if (more) {
                const char *pf = (const char *)(b + 8 * stride);
                _mm_prefetch(pf, _MM_HINT_T0);
                _mm_prefetch(pf + 64, _MM_HINT_T0);
                _mm_prefetch(pf + 128, _MM_HINT_T0);
            }
            // min term: m_j * (bs[2j] + bs[2j+1]) with each min on two int16 lanes
            const __m256i mn2 = _mm256_inserti128_si256(_mm256_castsi128_si256(_mm_unpacklo_epi16(mn16, mn16)),
                                                        _mm_unpackhi_epi16(mn16, mn16), 1);
            sm[r] = _mm512_zextsi256_si512(_mm256_madd_epi16(mn2, bs));
            dh[r] = u16_at(b);
            mh[r] = u16_at(b + 2);
        }
        for (int r = NR; r < 4; ++r) si[r] = sm[r] = _mm512_setzero_si512();
        const __m128 sumi = _mm_cvtepi32_ps(hsum4(si[0], si[1], si[2], si[3]));
        const __m128 summ = _mm_cvtepi32_ps(hsum4(sm[0], sm[1], sm[2], sm[3]));
        const __m128 dx = _mm_set1_ps(f32_at(qb));
        const __m128 d = _mm_mul_ps(_mm_cvtph_ps(_mm_load_si128((const __m128i *)dh)), dx);
        const __m128 dm = _mm_mul_ps(_mm_cvtph_ps(_mm_load_si128((const __m128i *)mh)), dx);
        acc = _mm_add_ps(acc, _mm_mul_ps(d, sumi));
        acc = _mm_sub_ps(acc, _mm_mul_ps(dm, summ));
    }
    alignas(16) float o[4];
    _mm_store_ps(o, acc);
    for (int r = 0; r < NR; ++r) out[r] = o[r];
}

// Q6_K: per 128-value half, quarters (0,1) and (2,3) of the six-bit codes as two
// 64-byte vectors; 16-value group c of the super-block has scale c; the -32
// offset is 32 * sum_c scale_c * bsum_c from the Q8_K block sums
template <int NR>
MPC_AVX512 static void rows_q6k_vnni(const uint8_t *row0, size_t stride, const uint8_t *q8, int nb, float *out,
                                     bool more) {
    const __m256i m4 = _mm256_set1_epi8(0x0F), m30 = _mm256_set1_epi8(0x30);
    __m512i cidx[4];           // chunk c (64 values): lanes 8t..8t+7 take scale 4c + t
    for (int c = 0; c < 4; ++c) {
        alignas(64) int16_t ix[32];
        for (int l = 0; l < 32; ++l) ix[l] = (int16_t)(4 * c + l / 8);
        cidx[c] = _mm512_load_si512((const void *)ix);
    }
    __m128 acc = _mm_setzero_ps();
    for (int i = 0; i < nb; ++i) {
        const uint8_t *qb = q8 + (size_t)i * Q8K_BYTES;
        __m512i xv[4];
        for (int c = 0; c < 4; ++c) xv[c] = _mm512_loadu_si512((const void *)(qb + 4 + 64 * c));
        const __m256i bs = _mm256_loadu_si256((const __m256i *)(qb + 4 + QK));
        __m512i si[4], so[4];
        alignas(16) uint16_t dh[8] = {0, 0, 0, 0, 0, 0, 0, 0};
        for (int r = 0; r < NR; ++r) {
            const uint8_t *b = row0 + (size_t)r * stride + (size_t)i * Q6K_BYTES;
            const __m256i sc16 = _mm256_cvtepi8_epi16(_mm_loadu_si128((const __m128i *)(b + 192)));
            const __m512i sc512 = _mm512_castsi256_si512(sc16);
            __m512i a = _mm512_setzero_si512();
            for (int h = 0; h < 2; ++h) {
                const __m256i ql0 = _mm256_loadu_si256((const __m256i *)(b + 64 * h));
                const __m256i ql1 = _mm256_loadu_si256((const __m256i *)(b + 64 * h + 32));
                const __m256i qh = _mm256_loadu_si256((const __m256i *)(b + 128 + 32 * h));
                const __m256i q0 = _mm256_or_si256(_mm256_and_si256(ql0, m4), _mm256_and_si256(_mm256_slli_epi16(qh, 4), m30));
                const __m256i q1 = _mm256_or_si256(_mm256_and_si256(ql1, m4), _mm256_and_si256(_mm256_slli_epi16(qh, 2), m30));
                const __m256i q2 = _mm256_or_si256(_mm256_and_si256(_mm256_srli_epi16(ql0, 4), m4), _mm256_and_si256(qh, m30));
                const __m256i q3 = _mm256_or_si256(_mm256_and_si256(_mm256_srli_epi16(ql1, 4), m4),
                                                   _mm256_and_si256(_mm256_srli_epi16(qh, 2), m30));
                const __m512i w0 = _mm512_inserti64x4(_mm512_castsi256_si512(q0), q1, 1);
                const __m512i w1 = _mm512_inserti64x4(_mm512_castsi256_si512(q2), q3, 1);
                const __m512i p0 = _mm512_maddubs_epi16(w0, xv[2 * h]);
                const __m512i p1 = _mm512_maddubs_epi16(w1, xv[2 * h + 1]);
                a = _mm512_dpwssd_epi32(a, p0, _mm512_permutexvar_epi16(cidx[2 * h], sc512));
                a = _mm512_dpwssd_epi32(a, p1, _mm512_permutexvar_epi16(cidx[2 * h + 1], sc512));
            }
            si[r] = a;
            so[r] = _mm512_zextsi256_si512(_mm256_madd_epi16(sc16, bs));      // sum_c scale_c * bsum_c
            dh[r] = u16_at(b + 208);
            if (more)
                for (int l = 0; l < 4; ++l) _mm_prefetch((const char *)(b + 8 * stride + 64 * l), _MM_HINT_T0);
        }
        for (int r = NR; r < 4; ++r) si[r] = so[r] = _mm512_setzero_si512();
        const __m128i sum_dot = hsum4(si[0], si[1], si[2], si[3]);
        const __m128i sum_off = hsum4(so[0], so[1], so[2], so[3]);
        const __m128 sumi = _mm_cvtepi32_ps(_mm_sub_epi32(sum_dot, _mm_slli_epi32(sum_off, 5)));
        const __m128 d = _mm_mul_ps(_mm_cvtph_ps(_mm_load_si128((const __m128i *)dh)), _mm_set1_ps(f32_at(qb)));
        acc = _mm_add_ps(acc, _mm_mul_ps(d, sumi));
    }
    alignas(16) float o[4];
    _mm_store_ps(o, acc);
    for (int r = 0; r < NR; ++r) out[r] = o[r];
}

MPC_AVX512 static void rows_vnni(int type, const uint8_t *row0, size_t stride, int nrows, const uint8_t *q8, int nb,
                                 float *out) {
    prefetch_rows(type, row0, stride, std::min(nrows, 8), nb);     // the first two groups; each group fetches the one two ahead
    int r = 0;
    for (; r + 4 <= nrows; r += 4)
        (type == mp::TYPE_Q6K ? rows_q6k_vnni<4> : rows_q4k_vnni<4>)(row0 + (size_t)r * stride, stride, q8, nb, out + r,
                                                                      r + 12 <= nrows);
    for (; r < nrows; ++r)
        (type == mp::TYPE_Q6K ? rows_q6k_vnni<1> : rows_q4k_vnni<1>)(row0 + (size_t)r * stride, stride, q8, nb, out + r,
                                                                      false);
}

float dot_q4k(const uint8_t *row, const uint8_t *q8, int nb) {
    if (g_portable || !has_vnni()) return dot_q4k_port(row, q8, nb);
    float y;
    rows_vnni(mp::TYPE_Q4K, row, 0, 1, q8, nb, &y);
    return y;
}

float dot_q6k(const uint8_t *row, const uint8_t *q8, int nb) {
    if (g_portable || !has_vnni()) return dot_q6k_port(row, q8, nb);
    float y;
    rows_vnni(mp::TYPE_Q6K, row, 0, 1, q8, nb, &y);
    return y;
}

void dot_rows(int type, const uint8_t *row0, size_t stride, int nrows, const uint8_t *q8, int nb, float *out) {
    if (!g_portable && has_vnni()) {
        rows_vnni(type, row0, stride, nrows, q8, nb, out);
        return;
    }
    for (int r = 0; r < nrows; ++r)
        out[r] = type == mp::TYPE_Q6K ? dot_q6k_port(row0 + (size_t)r * stride, q8, nb)
                                      : dot_q4k_port(row0 + (size_t)r * stride, q8, nb);
}

// ---- team --------------------------------------------------------------------
// Work is claimed item by item with a compare-and-swap on one word packing
// (generation, next item), so a worker that wakes late can never take an item
// of a newer job with an older job's function; the caller waits for the
// items to be done, not for every worker to check in (a worker the OS has
// descheduled holds nothing up unless it claimed an item).  Idle workers spin
// while the team is hot and for a grace period after, then sleep.
class Team {
  public:
    explicit Team(int n) {
        for (int i = 1; i < n; ++i) th_.emplace_back([this] { work(); });
    }
    ~Team() {
        {
            std::lock_guard<std::mutex> lk(mu_);
            quit_.store(true);
        }
        cv_.notify_all();
        for (auto &t : th_) t.join();
    }
    int size() const { return (int)th_.size() + 1; }
    void hot(bool on) {
        {
            std::lock_guard<std::mutex> lk(mu_);
            hot_.store(on);
        }
        if (on) cv_.notify_all();
    }
    // fn(ctx, item) for item in [0, n), spread over the team and the caller
    void run(int n, void (*fn)(void *, int), void *ctx) {
        if (n <= 0) return;
        const uint64_t g = ++gen_;
        Slot &sl = slot_[g & 1];
        sl.fn.store(fn, std::memory_order_relaxed);
        sl.ctx.store(ctx, std::memory_order_relaxed);
        sl.n.store(n, std::memory_order_relaxed);
        done_.store(0, std::memory_order_relaxed);
        {
            std::lock_guard<std::mutex> lk(mu_);
            state_.store(g << 32, std::memory_order_release);
        }
        if (!hot_.load(std::memory_order_relaxed)) cv_.notify_all();
        claim(g);
        while (done_.load(std::memory_order_acquire) < n) _mm_pause();
    }

  private:
    struct Slot {
        std::atomic<void (*)(void *, int)> fn{nullptr};
        std::atomic<void *> ctx{nullptr};
        std::atomic<int> n{0};
    };
    // take items of generation g until none is left or a newer job started
    void claim(uint64_t g) {
        const Slot &sl = slot_[g & 1];
        void (*fn)(void *, int) = sl.fn.load(std::memory_order_relaxed);
        void *ctx = sl.ctx.load(std::memory_order_relaxed);
        const uint32_t n = (uint32_t)sl.n.load(std::memory_order_relaxed);
        uint64_t st = state_.load(std::memory_order_acquire);
        for (;;) {
            if ((st >> 32) != g || (uint32_t)st >= n) return;
            if (state_.compare_exchange_weak(st, st + 1, std::memory_order_acq_rel, std::memory_order_acquire)) {
                fn(ctx, (int)(uint32_t)st);
                done_.fetch_add(1, std::memory_order_release);
                st = state_.load(std::memory_order_acquire);
            }
        }
    }
    void work() {
        uint64_t seen = 0;
        for (;;) {
            uint64_t g;
            int idle = 0;
            while ((g = state_.load(std::memory_order_acquire) >> 32) == seen) {
                if (quit_.load(std::memory_order_relaxed)) return;
                if (hot_.load(std::memory_order_relaxed) || ++idle < kGraceSpins) {
                    _mm_pause();
                    continue;
                }
                std::unique_lock<std::mutex> lk(mu_);
                cv_.wait(lk, [&] { return (state_.load() >> 32) != seen || quit_.load() || hot_.load(); });
                idle = 0;
            }
            seen = g;
            claim(g);
        }
    }
    static constexpr int kGraceSpins = 1 << 16;     // ~1-2 ms of pause instructions
    std::vector<std::thread> th_;
    std::mutex mu_;
    std::condition_variable cv_;
    uint64_t gen_ = 0;                               // the caller's job count
    alignas(64) std::atomic<uint64_t> state_{0};    // (generation << 32) | next item
    alignas(64) std::atomic<int> done_{0};
    alignas(64) Slot slot_[2];
    std::atomic<bool> quit_{false}, hot_{false};
};

namespace {
struct Touch {
    const volatile uint8_t *base;
    size_t n, page, per;
    std::atomic<unsigned> sink{0};
};
void touch_item(void *p, int item) {
    Touch &t = *(Touch *)p;
    unsigned s = 0;
    const size_t b = (size_t)item * t.per, e = std::min(t.n, b + t.per);
    for (size_t o = b; o < e; o += t.page) s += t.base[o];
    t.sink.fetch_add(s, std::memory_order_relaxed);
}
}  // namespace

#ifndef MADV_POPULATE_READ
#define MADV_POPULATE_READ 22
#endif

void prefault(Team *t, const void *p, size_t n) {
    if (!p || !n) return;
    const size_t page = (size_t)sysconf(_SC_PAGESIZE);
    const uintptr_t a = (uintptr_t)p / page * page;
    const size_t len = ((uintptr_t)p + n - a + page - 1) / page * page;
    if (madvise((void *)a, len, MADV_POPULATE_READ) == 0) return;
    Touch tc;                       // kernel without MADV_POPULATE_READ: read one byte per page
    tc.base = (const volatile uint8_t *)p;
    tc.n = n;
    tc.page = page;
    tc.per = 64 * page * 64;
    t->run((int)((n + tc.per - 1) / tc.per), touch_item, &tc);
}

Team *team_create(int n_threads) { return new Team(std::max(1, n_threads)); }
void team_destroy(Team *t) { delete t; }
int team_size(const Team *t) { return t->size(); }
void team_hot(Team *t, bool on) { t->hot(on); }

// ---- the chain -----------------------------------------------------------------
namespace {
// Rows per work item.  Measured on the 48-layer decode with 14 threads (the
// host's compute per layer is the critical path there): 8/16, 8/32, 16/16 ran
// 321-350 tok/s; 16/32 393-415; 32/64 451-479; 64/128 484-488; 64/64 475-495;
// 128/128 452-458 (6 up/gate items an expert leave threads idle).  Long runs
// of contiguous rows per thread read DRAM better than many short ones.
constexpr int UP_ROWS = 64;     // up/gate rows per work item
constexpr int DN_ROWS = 64;     // down rows per work item

struct Chain {
    const CpuExpert *e;
    int n, H, I, down_type;
    int n_up;                    // up/gate items of all experts; the down items follow
    float *h;
    uint8_t *q8h;
    alignas(64) std::atomic<int> left[16];    // up/gate items of expert k not finished yet
    alignas(64) std::atomic<int> ready[16];   // Q8_K of expert k's h written
};

// rows of up and gate; the item that finishes an expert's h quantizes it and
// lets the expert's down items go
void up_item(Chain &c, int item) {
    const int per = c.I / UP_ROWS;
    const int k = item / per, r0 = (item % per) * UP_ROWS;
    const size_t rb = (size_t)(c.H / QK) * Q4K_BYTES;
    const uint8_t *up = c.e[k].w, *gate = c.e[k].w + (size_t)c.I * rb;
    float *h = c.h + (size_t)k * c.I;
    float u[UP_ROWS], g[UP_ROWS];
    prefetch_rows(mp::TYPE_Q4K, up + r0 * rb, rb, 8, c.H / QK);       // the first two groups of both at once
    prefetch_rows(mp::TYPE_Q4K, gate + r0 * rb, rb, 8, c.H / QK);
    dot_rows(mp::TYPE_Q4K, up + r0 * rb, rb, UP_ROWS, c.e[k].q8x, c.H / QK, u);
    dot_rows(mp::TYPE_Q4K, gate + r0 * rb, rb, UP_ROWS, c.e[k].q8x, c.H / QK, g);
    for (int r = 0; r < UP_ROWS; ++r) h[r0 + r] = g[r] / (1.0f + canon_expf(-g[r])) * u[r];
    if (c.left[k].fetch_sub(1, std::memory_order_acq_rel) == 1) {
        quant_q8k(h, c.I, c.q8h + (size_t)k * (c.I / QK) * Q8K_BYTES);
        c.ready[k].store(1, std::memory_order_release);
    }
}

// rows of down, expert by expert.  Every up/gate item is claimed before the
// first down item (items go out in order) and none of them waits, so the wait
// for the expert's h always ends.
void down_item(const Chain &c, int item) {
    const int per = c.H / DN_ROWS;
    const int k = item / per, r0 = (item % per) * DN_ROWS;
    const size_t rb_in = (size_t)(c.H / QK) * Q4K_BYTES;
    const size_t rb = (size_t)(c.I / QK) * (c.down_type == mp::TYPE_Q6K ? Q6K_BYTES : Q4K_BYTES);
    const uint8_t *down = c.e[k].w + 2 * (size_t)c.I * rb_in;
    if (!c.ready[k].load(std::memory_order_acquire)) {
        // h is not ready yet: fetch this item's rows meanwhile (one expert a
        // layer leaves DRAM headroom while its up/gate items run)
        prefetch_rows(c.down_type, down + r0 * rb, rb, DN_ROWS, c.I / QK);
        while (!c.ready[k].load(std::memory_order_acquire)) _mm_pause();
    }
    const uint8_t *q = c.q8h + (size_t)k * (c.I / QK) * Q8K_BYTES;
    dot_rows(c.down_type, down + r0 * rb, rb, DN_ROWS, q, c.I / QK, c.e[k].y + r0);
}

void chain_item(void *p, int item) {
    Chain &c = *(Chain *)p;
    if (item < c.n_up)
        up_item(c, item);
    else
        down_item(c, item - c.n_up);
}
// groups of tokens sharing an expert: the same items, each token of the
// group in turn against rows that are already in the cache after the first
struct GChain {
    const CpuGroup *g;
    const uint8_t *const *q8x;
    float *const *y;
    int n, H, I, down_type;
    int n_up;
    float *h;                    // [token][I], tokens numbered as in q8x / y
    uint8_t *q8h;
    alignas(64) std::atomic<int> left[16];
    alignas(64) std::atomic<int> ready[16];
};

void gup_item(GChain &c, int item) {
    const int per = c.I / UP_ROWS;
    const int k = item / per, r0 = (item % per) * UP_ROWS;
    const CpuGroup &g = c.g[k];
    const size_t rb = (size_t)(c.H / QK) * Q4K_BYTES;
    const uint8_t *up = g.w, *gate = g.w + (size_t)c.I * rb;
    prefetch_rows(mp::TYPE_Q4K, up + r0 * rb, rb, 8, c.H / QK);
    prefetch_rows(mp::TYPE_Q4K, gate + r0 * rb, rb, 8, c.H / QK);
    for (int j = g.first; j < g.first + g.n; ++j) {
        float u[UP_ROWS], gg[UP_ROWS];
        dot_rows(mp::TYPE_Q4K, up + r0 * rb, rb, UP_ROWS, c.q8x[j], c.H / QK, u);
        dot_rows(mp::TYPE_Q4K, gate + r0 * rb, rb, UP_ROWS, c.q8x[j], c.H / QK, gg);
        float *h = c.h + (size_t)j * c.I;
        for (int r = 0; r < UP_ROWS; ++r) h[r0 + r] = gg[r] / (1.0f + canon_expf(-gg[r])) * u[r];
    }
    if (c.left[k].fetch_sub(1, std::memory_order_acq_rel) == 1) {
        for (int j = g.first; j < g.first + g.n; ++j)
            quant_q8k(c.h + (size_t)j * c.I, c.I, c.q8h + (size_t)j * (c.I / QK) * Q8K_BYTES);
        c.ready[k].store(1, std::memory_order_release);
    }
}

void gdown_item(const GChain &c, int item) {
    const int per = c.H / DN_ROWS;
    const int k = item / per, r0 = (item % per) * DN_ROWS;
    const CpuGroup &g = c.g[k];
    const size_t rb_in = (size_t)(c.H / QK) * Q4K_BYTES;
    const size_t rb = (size_t)(c.I / QK) * (c.down_type == mp::TYPE_Q6K ? Q6K_BYTES : Q4K_BYTES);
    const uint8_t *down = g.w + 2 * (size_t)c.I * rb_in;
    while (!c.ready[k].load(std::memory_order_acquire)) _mm_pause();
    for (int j = g.first; j < g.first + g.n; ++j)
        dot_rows(c.down_type, down + r0 * rb, rb, DN_ROWS, c.q8h + (size_t)j * (c.I / QK) * Q8K_BYTES, c.I / QK,
                 c.y[j] + r0);
}

void gchain_item(void *p, int item) {
    GChain &c = *(GChain *)p;
    if (item < c.n_up)
        gup_item(c, item);
    else
        gdown_item(c, item - c.n_up);
}
}  // namespace

void experts_grouped(Team *t, const CpuGroup *g, int n_groups, const uint8_t *const *q8x, float *const *y, int H,
                     int I, int down_type, float *h_scratch, uint8_t *q8h_scratch) {
    for (int b = 0; b < n_groups; b += 16) {  // at most 16 experts per pass
        GChain c;
        c.g = g + b; c.n = std::min(16, n_groups - b); c.H = H; c.I = I; c.down_type = down_type;
        c.q8x = q8x; c.y = y; c.h = h_scratch; c.q8h = q8h_scratch;
        c.n_up = c.n * (I / UP_ROWS);
        for (int k = 0; k < c.n; ++k) {
            c.left[k].store(I / UP_ROWS, std::memory_order_relaxed);
            c.ready[k].store(0, std::memory_order_relaxed);
        }
        t->run(c.n_up + c.n * (H / DN_ROWS), gchain_item, &c);
    }
}

// One team job per pass: up/gate of every expert, then down expert by expert;
// a down item waits only for its own expert's h, so the down rows of the first
// expert run while the last up/gate rows finish.
void experts(Team *t, const CpuExpert *e, int n, int H, int I, int down_type, float *h_scratch,
             uint8_t *q8h_scratch) {
    for (int b = 0; b < n; b += 16) {         // at most 16 experts per pass
        Chain c;
        c.e = e + b; c.n = std::min(16, n - b); c.H = H; c.I = I; c.down_type = down_type;
        c.n_up = c.n * (I / UP_ROWS);
        c.h = h_scratch + (size_t)b * I;
        c.q8h = q8h_scratch + (size_t)b * (I / QK) * Q8K_BYTES;
        for (int k = 0; k < c.n; ++k) {
            c.left[k].store(I / UP_ROWS, std::memory_order_relaxed);
            c.ready[k].store(0, std::memory_order_relaxed);
        }
        t->run(c.n_up + c.n * (H / DN_ROWS), chain_item, &c);
    }
}

}  // namespace mpc
