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
// below 2^-120) have zero codes and s = 127.
//
// The codes come from v_cvt_scalef32_2xpk16_fp6_f32 (32 values divided by a power-of-two
// scale, rounded to nearest even onto the e2m3 grid: steps of 1/8 below 2, 1/4 in [2, 4),
// 1/2 above; checked on gfx950 against a software encoder on grid values, ties and the
// subnormal step) and hi's values back from v_cvt_scalef32_pk32_f32_fp6, two conversion
// instructions and 32 subtractions per block (a software encoder takes about 25 VALU
// instructions per value).
//
// Packed form: 32 codes of 6 bits in 6 dwords, code i at bit 6 i (the operand layout the
// MFMA reads for an fp6 lane: 32 consecutive K values).
#pragma once

#include "tsa_common.h"

namespace tsa {
namespace {

typedef float f32x16_t __attribute__((ext_vector_type(16)));
typedef float f32x32_t __attribute__((ext_vector_type(32)));
typedef uint32_t u32x6_t __attribute__((ext_vector_type(6)));

// e2m3 codes of v[i] / scale (a power of two), rounded to nearest even, code i at bit 6 i:
// the instruction packs its sources interleaved (a0, b0, a1, b1, ..), so a takes the even
// values and b the odd ones. Inline assembly with an early-clobbered result: ROCm 7.2's
// builtin for it may give the result registers that overlap the second source, which the
// instruction still reads after writing part of the result (the last two values of b came
// out wrong that way).
__device__ __forceinline__ u32x6_t fp6_codes32(const float (&v)[32], float scale) {
    f32x16_t a, b;
#pragma unroll
    for (int j = 0; j < 16; ++j) {
        a[j] = v[2 * j];
        b[j] = v[2 * j + 1];
    }
    u32x6_t c;
    asm volatile("v_cvt_scalef32_2xpk16_fp6_f32 %0, %1, %2, %3" : "=&v"(c) : "v"(a), "v"(b), "v"(scale));
    return c;
}

// The 32 values of codes c times scale, in code order (early-clobbered for the same reason).
__device__ __forceinline__ f32x32_t fp6_values32(u32x6_t c, float scale) {
    f32x32_t q;
    asm volatile("v_cvt_scalef32_pk32_f32_fp6 %0, %1, %2" : "=&v"(q) : "v"(c), "v"(scale));
    return q;
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
    if (ef < 7) return 127u;           // zero (or negligible) block: lo's scale 2^(s - 132) stays normal
    if (ef > 254) return 255u;         // inf / NaN: the e8m0 NaN scale
    const float sh = __builtin_amdgcn_ldexpf(1.0f, ef - 128);  // 2^(s - 127), s = ef - 1
    const u32x6_t ch = fp6_codes32(v, sh);
    const f32x32_t qh = fp6_values32(ch, sh);
    float r[32];  // what hi leaves, exact (hi's values are v rounded to a coarser step)
#pragma unroll
    for (int i = 0; i < 32; ++i) r[i] = v[i] - qh[i];
    const u32x6_t cl = fp6_codes32(r, __builtin_amdgcn_ldexpf(sh, -5));
#pragma unroll
    for (int d = 0; d < 6; ++d) {
        hi[d] = ch[d];
        lo[d] = cl[d];
    }
    return (uint32_t)(ef - 1);
}

}  // namespace
}  // namespace tsa
