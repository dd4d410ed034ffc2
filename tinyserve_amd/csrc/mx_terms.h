// Activations as the fp8 A operand of v_mfma_scale_f32_16x16x128_f8f6f4 against fp4 (MXFP4)
// weights: every 32-value block b of a bf16 vector v gets its own power-of-two scale
// s_b = 2^(7 - e_b), e_b the exponent of the block's largest |v|, and v s_b = hi + lo with
// hi = e4m3(v s_b), lo = e4m3(v s_b - hi). The instruction's A scale of block b is
// 1 / s_b (e8m0 byte 120 + e_b), so the matrix core undoes the scaling. For a bf16 v the
// pair is exact (hi keeps 4 significant bits, lo the remaining 4) unless v lies more than
// 2^9 below its block's maximum.
//
// Layouts (K positions as the instruction's fp8 operand takes them):
//   terms: hi [kp] bytes, then lo [kp] bytes, value k at byte k of each (zero past the
//          vector's end up to kp, a multiple of 128);
//   table: the vector's A-scale table, one e8m0 byte per block b at byte
//          4 (4 (b / 16) + b % 4) + (b % 16) / 4, so that dword 4g + q holds in byte j the
//          scale of block 16g + 4j + q, which is K block q of 128-wide piece 4g + j: lane
//          16q + r of a wave reads dword 4g + q for pieces 4g .. 4g + 3 and the opsel byte
//          m % 4 picks piece m's scale.
//   A operand of piece m: lane l holds row l % 16 of A, bytes 0..15 = K 16 (l / 16) .. + 15
//          and bytes 16..31 = K 64 + 16 (l / 16) .. + 15 of the piece; rows carrying
//          no term read zeros.
#pragma once

#include "mfma_tile.h"

namespace tsa {
namespace {

typedef int mxt_v8i __attribute__((ext_vector_type(8)));
typedef unsigned short mxt_us2 __attribute__((ext_vector_type(2)));

// 16 bytes from LDS (p points into LDS). Volatile: the read stays where it is written; the
// explicit address space keeps it a ds_read with an immediate offset (through a generic
// pointer the compiler precomputes a 64-bit flat address per read and runs out of registers).
typedef __attribute__((address_space(3))) const volatile u32x4 lds_u32x4;
__device__ __forceinline__ u32x4 lds16(const uint8_t* p) { return *(lds_u32x4*)(p); }
typedef __attribute__((address_space(3))) const volatile uint32_t lds_u32;

// Byte of block b in a vector's A-scale table.
__host__ __device__ __forceinline__ int ascale_byte(int b) { return 4 * (4 * (b >> 4) + (b & 3)) + ((b & 15) >> 2); }

// Two e4m3 terms of v * s: hi = RNE(v s), lo = RNE(v s - hi) (OCP e4m3; |v s| < 448).
__device__ __forceinline__ void fp8_terms(float v0, float v1, uint32_t& hi2, uint32_t& lo2) {
    const int h = __builtin_amdgcn_cvt_pk_fp8_f32(v0, v1, 0, false);
    const float r0 = v0 - __builtin_amdgcn_cvt_f32_fp8(h, 0), r1 = v1 - __builtin_amdgcn_cvt_f32_fp8(h, 1);
    hi2 = (uint32_t)h & 0xFFFFu;
    lo2 = (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(r0, r1, 0, false) & 0xFFFFu;
}

// Block-scaled terms of one 8-value chunk (v, bf16) of 32-value block b of a vector: the
// four chunks of a block are four consecutive lanes of one wave, all four active (the block
// maximum is taken by DPP across the quad). The block's largest magnitude has exponent e
// (clamped to [-120, 127]; 0 for an all-zero block); the lane writes its values' terms
// v 2^(7 - e) (largest in [128, 256)) as 8 bytes at hi and at lo (hi null: no write), and
// the lane with `first` set (one per quad) writes the block's A-scale byte 120 + e into the
// table.
__device__ __forceinline__ void block_terms(const u32x4& v, int b, bool first, uint8_t* hi, uint8_t* lo,
                                            uint8_t* table) {
    mxt_us2 mb = mxt_us2{0, 0};
#pragma unroll
    for (int d = 0; d < 4; ++d) mb = __builtin_elementwise_max(mb, __builtin_bit_cast(mxt_us2, v[d] & 0x7FFF7FFFu));
    // for non-negative bf16 the integer order of the bits is the order of the values
    int m = mb[0] > mb[1] ? mb[0] : mb[1];
    m = max(m, __builtin_amdgcn_mov_dpp(m, 0xB1, 0xF, 0xF, false));  // quad_perm [1,0,3,2]
    m = max(m, __builtin_amdgcn_mov_dpp(m, 0x4E, 0xF, 0xF, false));  // quad_perm [2,3,0,1]
    const int e = m ? min(max((m >> 7) - 127, -120), 127) : 0;
    const float s = __uint_as_float((uint32_t)(134 - e) << 23);  // 2^(7 - e)
    if (hi) {
        uint32_t hw[4], lw[4];
#pragma unroll
        for (int d = 0; d < 4; ++d)
            fp8_terms(bf16_bits_to_f32(v[d] & 0xFFFFu) * s, bf16_bits_to_f32(v[d] >> 16) * s, hw[d], lw[d]);
        *reinterpret_cast<uint2*>(hi) = uint2{hw[0] | (hw[1] << 16), hw[2] | (hw[3] << 16)};
        *reinterpret_cast<uint2*>(lo) = uint2{lw[0] | (lw[1] << 16), lw[2] | (lw[3] << 16)};
    }
    if (first) table[ascale_byte(b)] = (uint8_t)(120 + e);
}

}  // namespace
}  // namespace tsa
