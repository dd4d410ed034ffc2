// Activations as two fp6 terms per value for the scaled MFMA (v_mfma_scale_f32_32x32x64_f8f6f4).
//
// A 32-value block v (one MX block of K) is stored as hi and lo codes in OCP fp6 e2m3 (sign,
// 2 exponent bits with bias 1, 3 mantissa bits; no inf or NaN, largest 7.5) with an e8m0
// scale byte s for hi and s - 5 for lo:
//   v_i ~= 2^(s - 127) (hi_i + 2^-5 lo_i).
// s puts the block's largest magnitude in [2, 4) (s = biased exponent of max|v| - 1), so hi
// rounds every value to a step of at most 1/4 and the remainder (at most 1/8) times 32 fits
// lo's range; lo rounds it to a step of at most 1/4, i.e. 2^-7 before the 2^-5: every value
// is kept to within 2^-8 of the block's scale (max|v| is 2^1..2^2 of it), which is the
// precision of bf16 relative to the block maximum. Zero blocks (and blocks whose maximum is
// below 2^-121) have zero codes and s = 127.
//
// Packed form: 32 codes of 6 bits in 6 dwords, code i at bit 6 i (the operand layout the
// MFMA reads for an fp6 lane: 32 consecutive K values).
#pragma once

#include "tsa_common.h"

namespace tsa {
namespace {

// e2m3 code of v rounded to nearest even (|v| <= 7.75), and the value of that code.
__device__ __forceinline__ uint32_t e2m3_code(float v, float& q) {
    const float a = __builtin_fabsf(v);
    int e = (int)((__float_as_uint(a) >> 23) & 255u) - 127;  // floor(log2 a) for a >= 1
    e = e < 0 ? 0 : e;                                         // below 1: the subnormal step 1/8
    const float m = __builtin_rintf(__builtin_amdgcn_ldexpf(a, 3 - e));  // 8..16 (0..8 below 1)
    q = __builtin_copysignf(__builtin_amdgcn_ldexpf(m, e - 3), v);
    return ((uint32_t)m + 8u * (uint32_t)e) | ((__float_as_uint(v) >> 26) & 0x20u);
}

template <int I>
__device__ __forceinline__ void pack6(uint32_t (&w)[6], uint32_t c) {
    constexpr int bit = 6 * I, d = bit >> 5, o = bit & 31;
    w[d] |= c << o;
    if constexpr (o > 26) w[d + 1] |= c >> (32 - o);
}

template <int I>
__device__ __forceinline__ void fp6_terms_from(const float (&v)[32], int sh, uint32_t (&hi)[6], uint32_t (&lo)[6]) {
    if constexpr (I < 32) {
        float qh, ql;
        const float u = __builtin_amdgcn_ldexpf(v[I], sh);
        pack6<I>(hi, e2m3_code(u, qh));
        pack6<I>(lo, e2m3_code(__builtin_amdgcn_ldexpf(u - qh, 5), ql));
        fp6_terms_from<I + 1>(v, sh, hi, lo);
    }
}

// hi and lo codes of a block and the hi scale byte (lo's is that minus 5).
__device__ __forceinline__ uint32_t fp6_terms(const float (&v)[32], uint32_t (&hi)[6], uint32_t (&lo)[6]) {
    uint32_t amax = 0u;  // the largest magnitude's bits (a NaN, if any, compares largest)
#pragma unroll
    for (int i = 0; i < 32; ++i) {
        const uint32_t m = __float_as_uint(v[i]) & 0x7FFFFFFFu;
        amax = m > amax ? m : amax;
    }
#pragma unroll
    for (int d = 0; d < 6; ++d) hi[d] = lo[d] = 0u;
    const int ef = (int)(amax >> 23);  // biased exponent of max|v|
    if (ef < 6) return 127u;           // zero (or negligible) block
    if (ef > 254) return 255u;         // inf / NaN: the e8m0 NaN scale
    fp6_terms_from<0>(v, 128 - ef, hi, lo);              // v * 2^-(s - 127), s = ef - 1
    return (uint32_t)(ef - 1);
}

}  // namespace
}  // namespace tsa
