// Wave row-group dot products over native GGUF weight streams (Q8_0, Q4_K, Q5_K, Q6_K)
// against a bf16 vector held in LDS.
//
// Loads: a wave copies the contiguous byte range of its rows' super-blocks into its LDS
// area with coalesced 16-byte buffer-to-LDS loads (gq_stage_raw). Work unit: one lane then
// owns a whole quantisation unit of the stream (Q4_K / Q5_K: a 256-value super-block, 144
// / 176 bytes; Q6_K: half a super-block, 128 values: its 64 ql bytes, 32 qh bytes and 8
// scales; Q8_0: a 32-value block, 34 bytes) and reads it from LDS with 16-byte reads at
// 2-byte alignment (which gfx950 serves). Rows may start inside a unit (the flat stream at
// K = 2880), so results are attributed per 32-value sub-block to the unit's row or the
// next one.
//
// Arithmetic: a sub-block's dot product is sum_i (a q_i - c) x_i = a sum_i q_i x_i - c sum_i x_i
// with the block scales a, c factored out. The integer codes q (0..63 after offsetting)
// become the exact bf16 values 128 + q with one v_perm_b32 per pair (0x43 in the high
// byte makes 128 + q for q < 128), so v_dot2_f32_bf16 computes sum (128 + q_i) x_i with
// exact products in fp32, and 128 sum x_i, taken from a table of per-sub-block sums of the
// vector, is subtracted. x is the reference's bf16 activation, so no rounding happens
// before the fp32 accumulation.
//
// Semantics: tinyserve/gguf_dequant_torch.py:101-111,118-249 (formats), ggml_ops.cu:461-569
// (y = deq(W) x in fp32).
#pragma once

#include "formats.h"

namespace tsa {
namespace {

typedef short s16x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));

// bf16 pair (128 + b0, 128 + b1) from bytes b0 = byte s0, b1 = byte s1 of w (each < 128).
template <int S0, int S1>
__device__ __forceinline__ uint32_t q_pair(uint32_t w) {
    constexpr uint32_t sel = 0x04000400u | ((uint32_t)S0) | ((uint32_t)S1 << 16);
    return __builtin_amdgcn_perm(0x43434343u, w, sel);
}

__device__ __forceinline__ float dot2(uint32_t a, uint32_t b, float c) {
    return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, a), __builtin_bit_cast(bf16x2_t, b), c, false);
}

// sum over 4 codes (bytes of w, each < 128) of (128 + q) x for the 4 bf16 activations in
// xa (2 values) and xb (2 values).
__device__ __forceinline__ float dot4(uint32_t w, uint32_t xa, uint32_t xb, float c) {
    c = dot2(q_pair<0, 1>(w), xa, c);
    return dot2(q_pair<2, 3>(w), xb, c);
}

// sum over 32 codes, given as 8 words of 4 byte-codes, against 32 bf16 activations at xs.
__device__ __forceinline__ float dot32(const uint32_t q[8], const uint8_t* xs) {
    const u32x4 x0 = *reinterpret_cast<const u32x4*>(xs);
    const u32x4 x1 = *reinterpret_cast<const u32x4*>(xs + 16);
    const u32x4 x2 = *reinterpret_cast<const u32x4*>(xs + 32);
    const u32x4 x3 = *reinterpret_cast<const u32x4*>(xs + 48);
    float a = 0.0f, b = 0.0f;
    a = dot4(q[0], x0[0], x0[1], a);
    b = dot4(q[1], x0[2], x0[3], b);
    a = dot4(q[2], x1[0], x1[1], a);
    b = dot4(q[3], x1[2], x1[3], b);
    a = dot4(q[4], x2[0], x2[1], a);
    b = dot4(q[5], x2[2], x2[3], b);
    a = dot4(q[6], x3[0], x3[1], a);
    b = dot4(q[7], x3[2], x3[3], b);
    return a + b;
}

// 16 codes (4 words) against 16 activations.
__device__ __forceinline__ float dot16(const uint32_t* q, const uint8_t* xs) {
    const u32x4 x0 = *reinterpret_cast<const u32x4*>(xs);
    const u32x4 x1 = *reinterpret_cast<const u32x4*>(xs + 16);
    float a = dot4(q[0], x0[0], x0[1], 0.0f);
    float b = dot4(q[1], x0[2], x0[3], 0.0f);
    a = dot4(q[2], x1[0], x1[1], a);
    b = dot4(q[3], x1[2], x1[3], b);
    return a + b;
}

template <int TYPE> struct GqUnit;
// values per unit, super-block (or block) bytes, units per super-block
template <> struct GqUnit<8>  { static constexpr int V = 32,  SB = 34,  PER_SB = 1; };
template <> struct GqUnit<12> { static constexpr int V = 256, SB = 144, PER_SB = 1; };
template <> struct GqUnit<13> { static constexpr int V = 256, SB = 176, PER_SB = 1; };
template <> struct GqUnit<14> { static constexpr int V = 128, SB = 210, PER_SB = 2; };

__device__ __forceinline__ u32x4 ld16u(const uint8_t* p) { return *reinterpret_cast<const u32x4*>(p); }

typedef int gq_v4i __attribute__((ext_vector_type(4)));

// Copies bytes [a0, a0 + n) of the buffer (base, records) into LDS at dst (all 16-byte
// aligned; a0 may be "negative" as an unsigned wrap: those chunks read zero), 16 bytes per
// lane per instruction, one wave. Issued as inline assembly (the compiler would otherwise
// wait for every load before any later LDS read); the caller waits with gq_wait_dma.
__device__ __forceinline__ void gq_stage_raw(const uint8_t* base, uint32_t records, uint32_t a0, uint32_t n,
                                             uint32_t dst, int lane) {
    const uint64_t b = reinterpret_cast<uint64_t>(base);
    const gq_v4i r = gq_v4i{(int)(uint32_t)b, (int)(uint32_t)(b >> 32), (int)records, 0x00020000};
    for (uint32_t c = 0; c < n; c += 1024) {
        const uint32_t m0 = __builtin_amdgcn_readfirstlane(dst + c);
        if (c + 16 * lane < n)
            asm volatile("s_mov_b32 m0, %2\n\tbuffer_load_dwordx4 %0, %1, 0 offen lds" ::"v"(a0 + c + 16 * lane), "s"(r),
                         "s"(m0)
                         : "memory", "m0");
    }
}

// Copies the n bytes (a whole number of 16-byte chunks) of a bf16 vector at a0 of the
// buffer (base, records) into the padded vector layout at dst: one 256-byte run (16 lanes)
// per instruction.
__device__ __forceinline__ void gq_stage_vec_raw(const uint8_t* base, uint32_t records, uint32_t a0, uint32_t n,
                                                 uint32_t dst, int lane) {
    const uint64_t b = reinterpret_cast<uint64_t>(base);
    const gq_v4i r = gq_v4i{(int)(uint32_t)b, (int)(uint32_t)(b >> 32), (int)records, 0x00020000};
    for (uint32_t c = 0; c < n; c += 256) {
        const uint32_t m0 = __builtin_amdgcn_readfirstlane(dst + c + 16 * (c >> 8));
        if (lane < 16 && c + 16 * lane < n)
            asm volatile("s_mov_b32 m0, %2\n\tbuffer_load_dwordx4 %0, %1, 0 offen lds" ::"v"(a0 + c + 16 * lane), "s"(r),
                         "s"(m0)
                         : "memory", "m0");
    }
}

// This wave's loads (and LDS work) are complete; then its lanes may read what they staged.
__device__ __forceinline__ void gq_wait_dma() {
    asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)" ::: "memory");
    __builtin_amdgcn_wave_barrier();
}

// The vector in LDS: bf16 values and per-32-value and per-16-value sums (float), indexed by
// position along K. Every 128 values (256 bytes) are followed by 16 bytes of padding: the
// lanes of a wave read the vector at strides of 256 or 512 bytes (one unit each), which
// without the padding would put every lane's 16-byte read on the same four banks.
struct GqVec {
    const uint8_t* v;    // bf16 [K], padded
    const float* s32;    // [K / 32]
    const float* s16;    // [K / 16]
};

// Byte offset of value kk in the padded vector (kk a multiple of 8).
__host__ __device__ constexpr uint32_t gq_pad(uint32_t kk) { return 2 * kk + 16 * (kk >> 7); }
__device__ __forceinline__ const uint8_t* gq_x(const GqVec& x, uint32_t kk) { return x.v + gq_pad(kk); }

// Dot products of unit u (unit index in the flat stream) with the vector; b points at the
// unit's super-block (or block) in LDS. The unit's values start at column kk0 of some row
// (kk0 = (u V) % K, computed by the caller once per unit); 32-value sub-blocks whose flat
// value index g lies in [lo, hi) contribute to pa (still in that row) or pb (the next row,
// once kk reaches K; a unit spans at most two rows since K >= V). 32-bit indices
// (matrices below 2^31 values).
// WRAP = false: K is a multiple of the unit's values, so every unit lies inside one row
// and inside [lo, hi) (the caller's units are whole rows); the row checks compile away.
template <int TYPE, bool WRAP = true>
__device__ __forceinline__ void gq_unit(const uint8_t* __restrict__ b, uint32_t u, uint32_t kk0, uint32_t K, uint32_t lo,
                                        uint32_t hi, const GqVec& x, float& pa, float& pb) {
    using U = GqUnit<TYPE>;
    const uint32_t g0 = u * U::V;
    auto add = [&](uint32_t j, float part) {
        if (WRAP && kk0 + 32 * j >= K) pb += part;
        else pa += part;
    };
    auto col = [&](uint32_t j) {
        const uint32_t kk = kk0 + 32 * j;
        return WRAP && kk >= K ? kk - K : kk;
    };
    auto outside = [&](uint32_t g) { return WRAP && (g < lo || g >= hi); };
    if constexpr (TYPE == 8) {
        if (outside(g0)) return;
        const float d = f16_bits_to_f32(*reinterpret_cast<const uint16_t*>(b));
        const u32x4 a = ld16u(b + 2), c = ld16u(b + 18);
        uint32_t ql[8], qh[8];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const uint32_t wa = a[i] ^ 0x80808080u, wc = c[i] ^ 0x80808080u;  // q + 128
            ql[i] = wa & 0x0F0F0F0Fu;
            qh[i] = (wa >> 4) & 0x0F0F0F0Fu;
            ql[4 + i] = wc & 0x0F0F0F0Fu;
            qh[4 + i] = (wc >> 4) & 0x0F0F0F0Fu;
        }
        const uint32_t kk = kk0;
        const uint8_t* xs = gq_x(x, kk);
        const float sx = x.s32[kk / 32];
        // sum q x = sum (16 qh + ql - 128) x
        const float dl = dot32(ql, xs) - 128.0f * sx, dh = dot32(qh, xs) - 128.0f * sx;
        pa += d * (16.0f * dh + dl - 128.0f * sx);
    } else if constexpr (TYPE == 12 || TYPE == 13) {
        constexpr int QS = TYPE == 12 ? 16 : 48;
        const u32x4 hdr = ld16u(b);  // d, dmin | scales[12]
        u32x4 qv[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) qv[i] = ld16u(b + QS + 16 * i);
        u32x4 hv[2];
        if constexpr (TYPE == 13) {
            hv[0] = ld16u(b + 16);
            hv[1] = ld16u(b + 32);
        }
        const float d = f16_bits_to_f32(hdr[0] & 0xFFFFu), dmin = f16_bits_to_f32(hdr[0] >> 16);
        const uint32_t s[3] = {hdr[1], hdr[2], hdr[3]};
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            if (outside(g0 + 32 * j)) continue;
            uint32_t sc, m;
            k_scale_min(s, j, sc, m);
            uint32_t q[8];
            const int c = j >> 1, sh = 4 * (j & 1);
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                uint32_t n = (qv[2 * c + (i >> 2)][i & 3] >> sh) & 0x0F0F0F0Fu;
                if constexpr (TYPE == 13) n |= ((hv[i >> 2][i & 3] >> j) & 0x01010101u) << 4;
                q[i] = n;
            }
            const uint32_t kk = col(j);
            const float sx = x.s32[kk / 32];
            const float dq = dot32(q, gq_x(x, kk)) - 128.0f * sx;
            add(j, d * (float)sc * dq - dmin * (float)m * sx);
        }
    } else {  // Q6_K, half h of super-block u / 2: ql[64h, +64), qh[32h, +32), sc[8h, +8), d @208
        const uint32_t hh = u & 1;
        u32x4 l[4], qh[2];
#pragma unroll
        for (int i = 0; i < 4; ++i) l[i] = ld16u(b + 64 * hh + 16 * i);
        qh[0] = ld16u(b + 128 + 32 * hh);
        qh[1] = ld16u(b + 144 + 32 * hh);
        const uint2 scw = *reinterpret_cast<const uint2*>(b + 192 + 8 * hh);
        const float d = f16_bits_to_f32(*reinterpret_cast<const uint16_t*>(b + 208));
#pragma unroll
        for (int t = 0; t < 4; ++t) {  // 32-value quarter t of the half
            if (outside(g0 + 32 * t)) continue;
            uint32_t q[8];
            const int shl = 4 * (t >> 1), shh = 2 * t;
#pragma unroll
            for (int i = 0; i < 8; ++i)
                q[i] = ((l[2 * (t & 1) + (i >> 2)][i & 3] >> shl) & 0x0F0F0F0Fu) |
                       (((qh[i >> 2][i & 3] >> shh) & 0x03030303u) << 4);
            const uint32_t kk = col(t);
            const uint8_t* xs = gq_x(x, kk);
            const float s0 = x.s16[kk / 16], s1 = x.s16[kk / 16 + 1];
            const uint32_t sw = t < 2 ? scw.x : scw.y;
            const float sc0 = (float)(int8_t)((sw >> (16 * (t & 1))) & 0xFFu);
            const float sc1 = (float)(int8_t)((sw >> (16 * (t & 1) + 8)) & 0xFFu);
            // codes are q + 32 (0..63): sum (q) x = sum (128 + q + 32) x - 160 sum x
            const float a0 = dot16(q, xs) - 160.0f * s0, a1 = dot16(q + 4, xs + 32) - 160.0f * s1;
            add(t, d * (sc0 * a0 + sc1 * a1));
        }
    }
}

// Adds v to acc[r] for a row index r known only at run time (0 <= r < N; others dropped).
template <int N>
__device__ __forceinline__ void acc_add(float (&acc)[N], int r, float v) {
#pragma unroll
    for (int i = 0; i < N; ++i)
        if (r == i) acc[i] += v;
}

// Wave reduction (sum over the 64 lanes, result in every lane) via DPP.
__device__ __forceinline__ float gq_wave_sum(float v) { return wave_sum_u(v); }

}  // namespace
}  // namespace tsa
