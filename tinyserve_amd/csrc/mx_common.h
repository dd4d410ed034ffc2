// MX (OCP microscaling) helpers for the MFMA paths: fp32 <-> fp8 e4m3 and the
// multi-term block decomposition of activations.
//
// Activations enter the scaled MFMA (v_mfma_scale_f32_16x16x128_f8f6f4) as fp8 e4m3
// with one e8m0 scale per 32 values. One fp8 term carries ~4 significant bits, so an
// activation block is split into NTERM terms: term c holds the e4m3 rounding of the
// residual left by terms 0..c-1, each with its own block scale chosen so the block's
// largest residual scales into [128, 256). Three terms keep ~12 bits per element
// relative to the block maximum, which is more than bf16 carries. The terms ride in
// separate MFMA B columns, so they cost no extra MFMA issue; the columns are summed
// after the chain.
#pragma once

#include "tsa_common.h"

namespace tsa {

constexpr int NTERM = 3;

typedef int v8i __attribute__((ext_vector_type(8)));
typedef float v4f __attribute__((ext_vector_type(4)));
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

// float -> OCP fp8 e4m3 (bias 7, no inf), round to nearest even; requires |v| < 448.
__device__ __forceinline__ uint32_t f32_to_e4m3(float v) {
    const uint32_t u = __float_as_uint(v);
    const uint32_t s = (u >> 24) & 0x80u;
    const float a = fabsf(v);
    if (a < 0x1p-6f) return s | (uint32_t)rintf(a * 512.0f);  // subnormal step 2^-9 (8 -> 0x08 = 2^-6)
    uint32_t au = __float_as_uint(a);
    au += 0x7FFFFu + ((au >> 20) & 1u);
    const uint32_t e = (au >> 23) - 120u;  // (exp - 127) + 7
    return s | (e << 3) | ((au >> 20) & 7u);
}

__device__ __forceinline__ float e4m3_to_f32(uint32_t c) {
    const uint32_t e = (c >> 3) & 15u, m = c & 7u;
    const float v = e ? ldexpf((float)(8u + m), (int)e - 10) : ldexpf((float)m, -9);
    return (c & 0x80u) ? -v : v;
}

// Shared block exponent for a block whose largest magnitude is m: E with m / 2^E in
// [128, 256), clamped to the e8m0 range; 0 for an all-zero block.
__device__ __forceinline__ int mx_block_exp(float m) {
    if (!(m > 0.0f)) return 0;
    const int e = (int)((__float_as_uint(m) >> 23) & 255u) - 127;  // floor(log2 m) for normal m
    int E = e - 7;
    return E < -127 ? -127 : (E > 127 ? 127 : E);
}

}  // namespace tsa
