// Wave-cooperative row dot products over native weight rows (per-lane partial sums).
//
// A wave computes <row n of W, x> with its 64 lanes striding over the row: GGUF rows
// by 32-value units (flat index n*K + k, so rows may start inside a super-block),
// MXFP4 rows by 16-byte groups. The activations x are float32 in LDS. The caller
// reduces the partial with wave_sum.
#pragma once

#include "formats.h"

namespace tsa {

typedef float v2f __attribute__((ext_vector_type(2)));

template <int TYPE, int A>
__device__ __forceinline__ float gguf_row_partial(const uint8_t* __restrict__ w, int64_t n, int64_t K,
                                                  const float* __restrict__ xs, int lane) {
    using Tr = GgufTraits<TYPE>;
    const int64_t upr = K / 32;
    float acc = 0.0f;
    for (int64_t j = lane; j < upr; j += 64) {
        const int64_t U = n * upr + j;
        float v[32];
        decode_unit<TYPE, A>(w + (U / Tr::UPB) * Tr::TS, (int)(U % Tr::UPB), v);
        const float4* xv = reinterpret_cast<const float4*>(xs + 32 * j);
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const float4 q = xv[i];
            acc += v[4 * i] * q.x + v[4 * i + 1] * q.y + v[4 * i + 2] * q.z + v[4 * i + 3] * q.w;
        }
    }
    return acc;
}

// 16 bytes (32 e2m1 values) of one MXFP4 group dotted with 32 activations, unscaled.
__device__ __forceinline__ float mx16_dot(const uint32_t q[4], const float* __restrict__ xv) {
    float a = 0.0f;
#pragma unroll
    for (int d = 0; d < 4; ++d) {
        const float4* x4 = reinterpret_cast<const float4*>(xv + 8 * d);
        const float4 xa = x4[0], xb = x4[1];
        const v2f p0 = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(q[d], 1.0f, 0);
        const v2f p1 = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(q[d], 1.0f, 1);
        const v2f p2 = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(q[d], 1.0f, 2);
        const v2f p3 = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(q[d], 1.0f, 3);
        a += p0.x * xa.x + p0.y * xa.y + p1.x * xa.z + p1.y * xa.w;
        a += p2.x * xb.x + p2.y * xb.y + p3.x * xb.z + p3.y * xb.w;
    }
    return a;
}

template <int A>
__device__ __forceinline__ void ld16(const uint8_t* p, uint32_t q[4]) {
    if constexpr (A >= 16) {
        const uint4 v = *reinterpret_cast<const uint4*>(p);
        q[0] = v.x; q[1] = v.y; q[2] = v.z; q[3] = v.w;
    } else {
        __builtin_memcpy(q, p, 16);
    }
}

template <int A>
__device__ __forceinline__ float mx_row_partial(const uint8_t* __restrict__ blocks, const uint8_t* __restrict__ scales,
                                                int64_t n, int64_t G, const float* __restrict__ xs, int lane) {
    float acc = 0.0f;
    for (int64_t g = lane; g < G; g += 64) {
        const int64_t c = n * G + g;
        uint32_t q[4];
        ld16<A>(blocks + 16 * c, q);
        acc += mx16_dot(q, xs + 32 * g) * e8m0_to_f32(scales[c]);
    }
    return acc;
}

}  // namespace tsa
