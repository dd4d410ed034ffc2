// Operand helpers for the MXFP4 paths that run on v_mfma_f32_16x16x32_bf16 over the
// 16-row tile order of mx_tile.hip: fp4 -> bf16 expansion with the block scale folded in,
// and 4-row bias fetches that match the MFMA result layout (lane 16q + i holds rows
// 4q..4q+3 of a 16-row tile).
#pragma once

#include "tsa_common.h"
#include "formats.h"

namespace tsa {
namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float v4f __attribute__((ext_vector_type(4)));
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

// The lane's 16-byte MXFP4 block: dword u holds values 8u..8u+7, expanded with the
// block scale into the bf16 A operand of K-slice u. v_cvt_scalef32_pk_bf16_fp4 rounds
// to nearest even, so fp4 * 2^e is exact wherever bf16 can hold it. (A 0xFF scale byte,
// NaN in OCP E8M0, turns the whole block into NaN here.) The halves go through 32-bit
// words: extracting bf16 elements of the converted pairs miscompiles with this
// toolchain (both halves come out as the low one).
__device__ __forceinline__ bf16x8 expand(uint32_t w, float s) {
    u32x4 r;
    r[0] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(w, s, 0));
    r[1] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(w, s, 1));
    r[2] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(w, s, 2));
    r[3] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(w, s, 3));
    return __builtin_bit_cast(bf16x8, r);
}

// Bias rows r0..r0+3 of an n-row bias vector: the raw 16 bytes at row r0 (a bounded
// buffer load, so a 2-byte dtype may read past the last row without faulting), issued
// before the tile so that no dtype-dependent wait sits behind the tile loads, and
// converted once the tile is done.
__device__ __forceinline__ u32x4 bias_raw(const uint8_t* src, int dtype, int64_t n, int64_t r0) {
    const int es = dtype == TSA_F32 ? 4 : 2;
    const __amdgpu_buffer_rsrc_t r =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t*>(src), (short)0, (int)(n * es), 0x00020000);
    return __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(r, (int)(r0 * es), 0, 0));
}

__device__ __forceinline__ v4f bias_value(const u32x4& w, int dtype) {
    if (dtype == TSA_F32) return v4f{__uint_as_float(w[0]), __uint_as_float(w[1]), __uint_as_float(w[2]), __uint_as_float(w[3])};
    const uint32_t a0 = w[0] & 0xFFFFu, a1 = w[0] >> 16, a2 = w[1] & 0xFFFFu, a3 = w[1] >> 16;
    if (dtype == TSA_BF16)
        return v4f{bf16_bits_to_f32(a0), bf16_bits_to_f32(a1), bf16_bits_to_f32(a2), bf16_bits_to_f32(a3)};
    return v4f{f16_bits_to_f32(a0), f16_bits_to_f32(a1), f16_bits_to_f32(a2), f16_bits_to_f32(a3)};
}

}  // namespace
}  // namespace tsa
