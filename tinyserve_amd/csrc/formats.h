// Device-side decoders of the native weight formats (GGUF Q8_0/Q4_K/Q5_K/Q6_K, MXFP4).
//
// GGUF work is cut into 32-value "units": a Q8_0 block is one unit, a K-quant
// super-block (256 values) is eight. decode_unit<T, A>(block, u, v) writes the 32
// float32 values of unit u of the block at `block`; A is the byte alignment the
// caller guarantees for `block` (16 for Q4_K/Q5_K on a 16-aligned base, 2 for
// Q8_0/Q6_K, 1 for an unaligned base), which selects the widest safe loads.
//
// Bit-exactness: every product below is exact in float32 (Q8_0 <= 18, Q4_K <= 21,
// Q5_K <= 22, Q6_K <= 23 significant bits), so the only rounding is the single
// `a*q - c` subtraction of Q4_K/Q5_K, which is the same rounding whether or not the
// compiler fuses it into an FMA. The results therefore equal the reference's
// (tinyserve/gguf_dequant_torch.py:118-122,187-249) bit for bit.
#pragma once

#include "tsa_common.h"

namespace tsa {

template <int A>
__device__ __forceinline__ uint32_t ld_u32(const uint8_t* p) {
    uint32_t v;
    __builtin_memcpy(&v, __builtin_assume_aligned(p, A), 4);
    return v;
}

template <int A>
__device__ __forceinline__ uint32_t ld_u16(const uint8_t* p) {
    uint16_t v;
    __builtin_memcpy(&v, __builtin_assume_aligned(p, A < 2 ? A : 2), 2);
    return v;
}

// 32 bytes starting at p into w[8] (little-endian dwords).
template <int A>
__device__ __forceinline__ void ld_32bytes(const uint8_t* p, uint32_t w[8]) {
    if constexpr (A >= 16) {
        const uint4 a = *reinterpret_cast<const uint4*>(p);
        const uint4 b = *reinterpret_cast<const uint4*>(p + 16);
        w[0] = a.x; w[1] = a.y; w[2] = a.z; w[3] = a.w;
        w[4] = b.x; w[5] = b.y; w[6] = b.z; w[7] = b.w;
    } else {
#pragma unroll
        for (int i = 0; i < 8; ++i) w[i] = ld_u32<A>(p + 4 * i);
    }
}

__device__ __forceinline__ uint32_t byte_of(const uint32_t* w, int i) { return (w[i >> 2] >> (8 * (i & 3))) & 0xFFu; }

// 6-bit scale/min of sub-block j from the 12-byte K-quant field held in s[3] dwords
// (tinyserve/gguf_dequant_torch.py:101-111).
__device__ __forceinline__ void k_scale_min(const uint32_t s[3], int j, uint32_t& sc, uint32_t& m) {
    if (j < 4) {
        sc = byte_of(s, j) & 63u;
        m = byte_of(s, j + 4) & 63u;
    } else {
        sc = (byte_of(s, j + 4) & 15u) | ((byte_of(s, j - 4) >> 6) << 4);
        m = (byte_of(s, j + 4) >> 4) | ((byte_of(s, j) >> 6) << 4);
    }
}

template <int TYPE, int A>
__device__ __forceinline__ void decode_unit(const uint8_t* b, int u, float v[32]);

// Q8_0: fp16 d @0, int8 q[32] @2.
template <>
__device__ __forceinline__ void decode_unit<8, 1>(const uint8_t* b, int, float v[32]) {
    const float d = f16_bits_to_f32(ld_u16<1>(b));
#pragma unroll
    for (int i = 0; i < 32; ++i) v[i] = d * (float)(int8_t)b[2 + i];
}
template <>
__device__ __forceinline__ void decode_unit<8, 2>(const uint8_t* b, int, float v[32]) {
    const float d = f16_bits_to_f32(ld_u16<2>(b));
#pragma unroll
    for (int i = 0; i < 16; ++i) {
        const uint32_t h = ld_u16<2>(b + 2 + 2 * i);
        v[2 * i] = d * (float)(int8_t)(h & 0xFF);
        v[2 * i + 1] = d * (float)(int8_t)(h >> 8);
    }
}

// Q4_K: fp16 d @0, fp16 dmin @2, scales[12] @4, qs[128] @16; unit u uses the low
// (u even) or high (u odd) nibbles of qs[32*(u/2) .. +31].
template <int A>
__device__ __forceinline__ void decode_q4k(const uint8_t* b, int u, float v[32]) {
    uint32_t hd, s[3], q[8];
    if constexpr (A >= 4) {
        hd = ld_u32<4>(b);
        s[0] = ld_u32<4>(b + 4); s[1] = ld_u32<4>(b + 8); s[2] = ld_u32<4>(b + 12);
    } else {
        hd = ld_u32<A>(b);
        s[0] = ld_u32<A>(b + 4); s[1] = ld_u32<A>(b + 8); s[2] = ld_u32<A>(b + 12);
    }
    ld_32bytes<A>(b + 16 + 32 * (u >> 1), q);
    const float d = f16_bits_to_f32(hd & 0xFFFFu), dmin = f16_bits_to_f32(hd >> 16);
    uint32_t sc, m;
    k_scale_min(s, u, sc, m);
    const float a = d * (float)sc, c = dmin * (float)m;
    const int sh = (u & 1) * 4;
#pragma unroll
    for (int i = 0; i < 32; ++i) v[i] = a * (float)((byte_of(q, i) >> sh) & 15u) - c;
}
template <> __device__ __forceinline__ void decode_unit<12, 16>(const uint8_t* b, int u, float v[32]) { decode_q4k<16>(b, u, v); }
template <> __device__ __forceinline__ void decode_unit<12, 1>(const uint8_t* b, int u, float v[32]) { decode_q4k<1>(b, u, v); }

// Q5_K: as Q4_K with qh[32] @16 (bit u of qh[i] is bit 4 of element 32u+i), qs[128] @48.
template <int A>
__device__ __forceinline__ void decode_q5k(const uint8_t* b, int u, float v[32]) {
    uint32_t hd, s[3], q[8], h[8];
    hd = ld_u32<A < 4 ? A : 4>(b);
    s[0] = ld_u32<A < 4 ? A : 4>(b + 4); s[1] = ld_u32<A < 4 ? A : 4>(b + 8); s[2] = ld_u32<A < 4 ? A : 4>(b + 12);
    ld_32bytes<A>(b + 16, h);
    ld_32bytes<A>(b + 48 + 32 * (u >> 1), q);
    const float d = f16_bits_to_f32(hd & 0xFFFFu), dmin = f16_bits_to_f32(hd >> 16);
    uint32_t sc, m;
    k_scale_min(s, u, sc, m);
    const float a = d * (float)sc, c = dmin * (float)m;
    const int sh = (u & 1) * 4;
#pragma unroll
    for (int i = 0; i < 32; ++i) {
        const uint32_t qq = ((byte_of(q, i) >> sh) & 15u) | (((byte_of(h, i) >> u) & 1u) << 4);
        v[i] = a * (float)qq - c;
    }
}
template <> __device__ __forceinline__ void decode_unit<13, 16>(const uint8_t* b, int u, float v[32]) { decode_q5k<16>(b, u, v); }
template <> __device__ __forceinline__ void decode_unit<13, 1>(const uint8_t* b, int u, float v[32]) { decode_q5k<1>(b, u, v); }

// Q6_K: ql[128] @0, qh[64] @128, int8 sc[16] @192, fp16 d @208. Unit u = half h = u/4,
// quarter t = u%4: low 4 bits from ql[64h + 32(t&1) + i] >> 4(t>>1), high 2 bits from
// qh[32h + i] >> 2t; value = (d * sc[2u + i/16]) * (q - 32).
template <int A>
__device__ __forceinline__ void decode_q6k(const uint8_t* b, int u, float v[32]) {
    const int hh = u >> 2, t = u & 3;
    uint32_t ql[8], qh[8];
    ld_32bytes<A>(b + 64 * hh + 32 * (t & 1), ql);
    ld_32bytes<A>(b + 128 + 32 * hh, qh);
    const uint32_t scw = ld_u16<A>(b + 192 + 2 * u);
    const float d = f16_bits_to_f32(ld_u16<A>(b + 208));
    const float d0 = d * (float)(int8_t)(scw & 0xFF), d1 = d * (float)(int8_t)(scw >> 8);
    const int shl = 4 * (t >> 1), shh = 2 * t;
#pragma unroll
    for (int i = 0; i < 32; ++i) {
        const int q = (int)(((byte_of(ql, i) >> shl) & 15u) | (((byte_of(qh, i) >> shh) & 3u) << 4)) - 32;
        v[i] = (i < 16 ? d0 : d1) * (float)q;
    }
}
template <> __device__ __forceinline__ void decode_unit<14, 2>(const uint8_t* b, int u, float v[32]) { decode_q6k<2>(b, u, v); }
template <> __device__ __forceinline__ void decode_unit<14, 1>(const uint8_t* b, int u, float v[32]) { decode_q6k<1>(b, u, v); }

// Units per block and bytes per block as compile-time constants.
template <int TYPE> struct GgufTraits;
template <> struct GgufTraits<8>  { static constexpr int UPB = 1, TS = 34,  FAST_A = 2; };
template <> struct GgufTraits<12> { static constexpr int UPB = 8, TS = 144, FAST_A = 16; };
template <> struct GgufTraits<13> { static constexpr int UPB = 8, TS = 176, FAST_A = 16; };
template <> struct GgufTraits<14> { static constexpr int UPB = 8, TS = 210, FAST_A = 2; };

// ---------------------------------------------------------------- MXFP4
// e2m1 code -> float32 bits, from the format: sign bit 3, exponent bits 2..1, mantissa
// bit 0; codes 0/1 are 0 and the subnormal 0.5 (tinyserve/mxfp4.py:5-8).
__device__ __forceinline__ float e2m1_to_f32(uint32_t c) {
    const uint32_t s = (c & 8u) << 28, mag = c & 7u;
    uint32_t bits;
    if (mag == 0) bits = 0;
    else if (mag == 1) bits = 0x3F000000u;                                   // 0.5
    else bits = ((126u + (mag >> 1)) << 23) | ((mag & 1u) << 22);            // (1+m/2)*2^(e-1)
    return __uint_as_float(s | bits);
}

// e8m0 byte -> float32 2^(s-127): exact, s = 0 gives the subnormal 2^-127, s = 255 gives +inf
// (the float32 multiplier torch.ldexp uses in tinyserve/mxfp4.py:42).
__device__ __forceinline__ float e8m0_to_f32(uint32_t s) {
    return s == 0 ? __uint_as_float(0x00400000u) : __uint_as_float(s << 23);
}

}  // namespace tsa
