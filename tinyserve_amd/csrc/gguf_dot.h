// Wave row-group dot products over native GGUF weight streams (Q8_0, Q4_K, Q5_K, Q6_K)
// against a bf16 vector held in LDS.
//
// Loads: a wave copies the contiguous byte range of its rows' super-blocks into its LDS
// area with coalesced 16-byte buffer-to-LDS loads (gq_stage_raw). Work unit: one lane then
// owns a quantisation unit of the stream (Q4_K / Q5_K: half a super-block, 128 values: its
// 64 qs bytes with the super-block's header and, for Q5_K, its 32 qh bytes; Q6_K: half a
// super-block: its 64 ql bytes, 32 qh bytes and 8 scales; Q8_0: a 32-value block, 34 bytes)
// and reads it from LDS with 16-byte reads at 2-byte alignment (which gfx950 serves). Rows may start inside a unit (the flat stream at
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

#include "fused_common.h"
#include "mfma_tile.h"

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

// dot32 / dot16 over the hi and lo halves of a split vector, sharing the code pairs.
__device__ __forceinline__ float dot32s(const uint32_t q[8], const uint8_t* xs, const uint8_t* xl) {
    float a = 0.0f, b = 0.0f;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const u32x4 h = *reinterpret_cast<const u32x4*>(xs + 16 * i);
        const u32x4 l = *reinterpret_cast<const u32x4*>(xl + 16 * i);
        a = dot4(q[2 * i], h[0], h[1], a);
        b = dot4(q[2 * i + 1], h[2], h[3], b);
        a = dot4(q[2 * i], l[0], l[1], a);
        b = dot4(q[2 * i + 1], l[2], l[3], b);
    }
    return a + b;
}
__device__ __forceinline__ float dot16s(const uint32_t* q, const uint8_t* xs, const uint8_t* xl) {
    float a = 0.0f, b = 0.0f;
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        const u32x4 h = *reinterpret_cast<const u32x4*>(xs + 16 * i);
        const u32x4 l = *reinterpret_cast<const u32x4*>(xl + 16 * i);
        a = dot4(q[2 * i], h[0], h[1], a);
        b = dot4(q[2 * i + 1], h[2], h[3], b);
        a = dot4(q[2 * i], l[0], l[1], a);
        b = dot4(q[2 * i + 1], l[2], l[3], b);
    }
    return a + b;
}

// A sub-block's 32 activations in registers (hi and, for split vectors, lo) with its sums.
struct GqXr {
    u32x4 h[4], l[4];
    float s[2];  // per-32 sum (Q4_K / Q5_K) or the two per-16 sums (Q6_K)
};
template <bool SPLIT>
__device__ __forceinline__ float dot16x(const uint32_t* q, const GqXr& r, int half) {
    float a = 0.0f, b = 0.0f;
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        const u32x4 h = r.h[2 * half + i];
        a = dot4(q[2 * i], h[0], h[1], a);
        b = dot4(q[2 * i + 1], h[2], h[3], b);
        if (SPLIT) {
            const u32x4 l = r.l[2 * half + i];
            a = dot4(q[2 * i], l[0], l[1], a);
            b = dot4(q[2 * i + 1], l[2], l[3], b);
        }
    }
    return a + b;
}
template <bool SPLIT>
__device__ __forceinline__ float dot32x(const uint32_t q[8], const GqXr& r) {
    return dot16x<SPLIT>(q, r, 0) + dot16x<SPLIT>(q + 4, r, 1);
}

// Values per unit: a Q8_0 block, or half a K-quant super-block (128 values: half the work
// per lane of a whole super-block, so a wave's compute after its copies arrive is half as
// long, and the same rows fill twice the lanes).
__host__ __device__ constexpr uint32_t gq_unit_values(int type) { return type == 8 ? 32u : 128u; }
template <int TYPE> struct GqUnit;
// values per unit, super-block (or block) bytes, units per super-block
template <> struct GqUnit<8>  { static constexpr int V = 32,  SB = 34,  PER_SB = 1; };
template <> struct GqUnit<12> { static constexpr int V = 128, SB = 144, PER_SB = 2; };
template <> struct GqUnit<13> { static constexpr int V = 128, SB = 176, PER_SB = 2; };
template <> struct GqUnit<14> { static constexpr int V = 128, SB = 210, PER_SB = 2; };

__device__ __forceinline__ u32x4 ld16u(const uint8_t* p) { return *reinterpret_cast<const u32x4*>(p); }

// N dwords of LDS data at byte address p, whatever its alignment. A ds_read_b128 / b64 off
// its natural alignment is split by the LDS into slow pieces (Q8_0 blocks of 34 bytes and
// Q6_K super-blocks of 210 sit off 16-byte boundaries), so whole dwords are read from the
// boundary at or below p and each pair is shifted into place (v_alignbyte_b32). The dword
// after the last is read only when p is off a dword boundary, when it holds data bytes.
template <int N>
__device__ __forceinline__ void lds_words(const uint8_t* p, uint32_t (&w)[N]) {
    const uint32_t ob = (uint32_t)reinterpret_cast<uintptr_t>(p) & 3u;
    const uint32_t* b = reinterpret_cast<const uint32_t*>(p - ob);
    uint32_t t[N + 1];
#pragma unroll
    for (int i = 0; i < N; ++i) t[i] = b[i];
    t[N] = ob ? b[N] : 0u;
#pragma unroll
    for (int i = 0; i < N; ++i) w[i] = __builtin_amdgcn_alignbyte(t[i + 1], t[i], ob);
}

typedef int gq_v4i __attribute__((ext_vector_type(4)));

// Buffer descriptor of (base, records) for the inline-assembly copies below, its words
// taken from the first lane: the "s" operand must sit in scalar registers, which the
// compiler only guarantees for values it can prove wave-uniform.
__device__ __forceinline__ gq_v4i gq_rsrc(const uint8_t* base, uint32_t records) {
    const uint64_t b = reinterpret_cast<uint64_t>(base);
    return gq_v4i{__builtin_amdgcn_readfirstlane((int)(uint32_t)b), __builtin_amdgcn_readfirstlane((int)(uint32_t)(b >> 32)),
                  __builtin_amdgcn_readfirstlane((int)records), 0x00020000};
}

// Records of a buffer that starts mis bytes below n bytes of data: whole 16-byte chunks, so
// the copy that holds the data's last bytes is not cut off by the range check (the rest of
// that chunk lies on the same page).
__device__ __forceinline__ uint32_t gq_records(uint64_t n, uint32_t mis) {
    const uint64_t r = (n + mis + 15) & ~(uint64_t)15;
    return r > 0xFFFFFFF0ull ? 0xFFFFFFF0u : (uint32_t)r;
}

// Copies bytes [a0, a0 + n) of the buffer (base, records) into LDS at dst (base + a0 and dst
// 16-byte aligned: an unaligned address would not be read as given), 16 bytes per
// lane per instruction, one wave. Issued as inline assembly (the compiler would otherwise
// wait for every load before any later LDS read); the caller waits with gq_wait_dma.
__device__ __forceinline__ void gq_stage_raw(const uint8_t* base, uint32_t records, uint32_t a0, uint32_t n,
                                             uint32_t dst, int lane) {
    const gq_v4i r = gq_rsrc(base, records);
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
    const gq_v4i r = gq_rsrc(base, records);
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
// fp32 / fp16 activations are held as two bf16 vectors, hi = bf16(x) and lo = bf16(x - hi)
// (hi + lo carries 16 significant bits, an fp16 value exactly); the dot products then run
// over both and the sums are of hi + lo.
struct GqVec {
    const uint8_t* v;    // bf16 [K], padded
    const uint8_t* lo;   // bf16 [K], padded, or null
    const float* s32;    // [K / 32]
    const float* s16;    // [K / 16]
};

// Byte offset of value kk in the padded vector (kk a multiple of 8).
__host__ __device__ constexpr uint32_t gq_pad(uint32_t kk) { return 2 * kk + 16 * (kk >> 7); }
__device__ __forceinline__ const uint8_t* gq_x(const GqVec& x, uint32_t kk) { return x.v + gq_pad(kk); }
__device__ __forceinline__ const uint8_t* gq_xl(const GqVec& x, uint32_t kk) { return x.lo + gq_pad(kk); }

// LDS bytes of a staged vector of n values (n % 32 == 0): padded bf16 values, then the
// per-32 and per-16 sums.
__host__ __device__ constexpr int gq_vec_vbytes(int n) { return (int)gq_pad((uint32_t)((n + 127) / 128 * 128)); }
__host__ __device__ constexpr int gq_vec_bytes(int n, bool split = false) {
    return gq_vec_vbytes(n) * (split ? 2 : 1) + 4 * (n / 32) + 4 * (n / 16);
}

// The LDS layout of a staged vector of n values at dst.
__device__ __forceinline__ GqVec gq_vec(uint8_t* dst, int n, bool split = false) {
    GqVec vec;
    vec.v = dst;
    vec.lo = split ? dst + gq_vec_vbytes(n) : nullptr;
    vec.s32 = reinterpret_cast<float*>(dst + gq_vec_vbytes(n) * (split ? 2 : 1));
    vec.s16 = vec.s32 + n / 32;
    return vec;
}

// One 8-value chunk of a vector as loaded: bf16 / fp16 values in a, fp32 values 0..3 in a
// and 4..7 in b.
struct GqRaw {
    u32x4 a, b;
};

// Chunk i of nv vectors of n values (cpv = n / 8 chunks each; vector jj from src (dtype) at
// element off0 + jj * src_stride): its loads (16 bytes for bf16 / fp16, 32 for fp32; rows
// 16-byte aligned, as the callers' are).
__device__ __forceinline__ GqRaw gq_chunk_load(const void* src, int dtype, int64_t off0, int64_t src_stride, int cpv,
                                               int i) {
    const int jj = i / cpv, c = i - jj * cpv;
    const int64_t e = off0 + jj * src_stride + 8 * (int64_t)c;  // first element of the chunk
    GqRaw r;
    if (dtype == TSA_F32) {
        r.a = *reinterpret_cast<const u32x4*>(static_cast<const float*>(src) + e);
        r.b = *reinterpret_cast<const u32x4*>(static_cast<const float*>(src) + e + 4);
    } else {
        r.a = *reinterpret_cast<const u32x4*>(static_cast<const uint16_t*>(src) + e);
        r.b = u32x4{0u, 0u, 0u, 0u};
    }
    return r;
}

// Chunk i (< cpv) of one vector of n values (cpv = n / 8), elements of es bytes (2 or 4) in
// the buffer rsrc (the vector's bytes; chunks past it read zero): straight-line buffer
// loads with no branch and no select on the loaded values, so that later loads issue
// before these return.
__device__ __forceinline__ GqRaw gq_chunk_load_buf(__amdgpu_buffer_rsrc_t rsrc, int es, int i) {
    const uint32_t off = (uint32_t)(8 * es) * (uint32_t)i;
    GqRaw r;
    r.a = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rsrc, off, 0, 0));
    r.b = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rsrc, es == 4 ? off + 16 : 0x80000000u, 0, 0));
    return r;
}

// Chunk i's values into the staged layout at dst0 + jj * dst_stride (as bf16, RNE; non-bf16
// sources as the hi / lo pair, the layout gq_vec(.., n, true) describes) with its share of
// the sums over every 32 and 16 consecutive positions, which come from neighbouring lanes
// by DPP: every lane of the wave calls, chunks in lane order (lanes 4m .. 4m + 3 hold four
// consecutive chunks of one vector, cpv % 4 == 0); invalid chunks (i past the last) write
// nothing.
__device__ __forceinline__ void gq_chunk_store(const GqRaw& r, bool valid, uint8_t* dst0, int dst_stride, int dtype,
                                               int n, int cpv, int i) {
    const bool split = dtype != TSA_BF16;
    const int jj = valid ? i / cpv : 0, c = valid ? i - jj * cpv : 0;
    uint32_t hw[4] = {0u, 0u, 0u, 0u}, lw[4] = {0u, 0u, 0u, 0u};
    float s8 = 0.0f;
    if (valid) {
        float f[8];
        if (dtype == TSA_BF16) {
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                hw[q] = r.a[q];
                s8 += bf16_bits_to_f32(r.a[q] & 0xFFFFu) + bf16_bits_to_f32(r.a[q] >> 16);
            }
        } else {
            if (dtype == TSA_F32) {
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    f[q] = __uint_as_float(r.a[q]);
                    f[4 + q] = __uint_as_float(r.b[q]);
                }
            } else {
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    f[2 * q] = f16_bits_to_f32(r.a[q] & 0xFFFFu);
                    f[2 * q + 1] = f16_bits_to_f32(r.a[q] >> 16);
                }
            }
#pragma unroll
            for (int q = 0; q < 8; ++q) {
                const uint32_t h = f32_to_bf16_bits(f[q]);
                const float hf = bf16_bits_to_f32(h);
                const uint32_t l = f32_to_bf16_bits(f[q] - hf);
                hw[q / 2] |= h << (16 * (q & 1));
                lw[q / 2] |= l << (16 * (q & 1));
                s8 += hf + bf16_bits_to_f32(l);  // hi + lo exactly: 16 significant bits
            }
        }
    }
    const float s16 = s8 + dpp_f<0xB1, 0xF, 0xF>(s8, 0.0f);    // quad_perm [1,0,3,2]
    const float s32 = s16 + dpp_f<0x4E, 0xF, 0xF>(s16, 0.0f);  // quad_perm [2,3,0,1]
    if (valid) {
        uint8_t* dst = dst0 + jj * dst_stride;
        const GqVec vec = gq_vec(dst, n, split);
        *reinterpret_cast<u32x4*>(dst + gq_pad(8 * c)) = u32x4{hw[0], hw[1], hw[2], hw[3]};
        if (split)
            *reinterpret_cast<u32x4*>(const_cast<uint8_t*>(vec.lo) + gq_pad(8 * c)) = u32x4{lw[0], lw[1], lw[2], lw[3]};
        if ((c & 1) == 0) const_cast<float*>(vec.s16)[c / 2] = s16;
        if ((c & 3) == 0) const_cast<float*>(vec.s32)[c / 4] = s32;
    }
}

// Stages nv vectors of n values (n % 32 == 0): vector jj from src (dtype) at element
// off0 + jj * src_stride into LDS at dst0 + jj * dst_stride (gq_chunk_store's layout).
// Threads tid of nthr (nthr a multiple of 64, whole waves calling) take 8-value chunks in
// lane order, so each load instruction reads one contiguous span.
__device__ void gq_stage_vecs(uint8_t* dst0, int dst_stride, const void* src, int dtype, int64_t off0,
                              int64_t src_stride, int n, int nv, int tid, int nthr) {
    const int cpv = n / 8, total = cpv * nv;  // chunks per vector (a multiple of 4)
    for (int base = 0; base < total; base += nthr) {
        const int i = base + tid;
        const bool valid = i < total;
        const GqRaw r = valid ? gq_chunk_load(src, dtype, off0, src_stride, cpv, i) : GqRaw{};
        gq_chunk_store(r, valid, dst0, dst_stride, dtype, n, cpv, i);
    }
}
__device__ void gq_stage(uint8_t* dst, const void* src, int dtype, int64_t off, int n, int tid, int nthr) {
    gq_stage_vecs(dst, 0, src, dtype, off, 0, n, 1, tid, nthr);
}

// The per-32 and per-16 sums of a bf16 vector already in LDS at vec (n values), one wave.
__device__ void gq_vec_sums(const GqVec& vec, int n, int lane) {
    float* s32 = const_cast<float*>(vec.s32);
    float* s16 = const_cast<float*>(vec.s16);
    for (int g = lane; g < n / 32; g += 64) {
        const u32x4* p4 = reinterpret_cast<const u32x4*>(gq_x(vec, 32 * g));
        float a = 0.0f, b = 0.0f;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const u32x4 w = p4[i];
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const float r = bf16_bits_to_f32(w[e] & 0xFFFFu) + bf16_bits_to_f32(w[e] >> 16);
                if (i < 2) a += r; else b += r;
            }
        }
        s16[2 * g] = a;
        s16[2 * g + 1] = b;
        s32[g] = a + b;
    }
}

// Super-blocks (or Q8_0 blocks) touched by the values [lo, hi) of a TYPE stream, and the
// LDS bytes a wave needs to stage them (16-byte aligned start, rounded up).
template <int TYPE>
__host__ __device__ constexpr uint32_t gq_sb_count(uint32_t lo, uint32_t hi) {
    constexpr uint32_t VS = TYPE == 8 ? 32 : 256;
    return (hi + VS - 1) / VS - lo / VS;
}
__host__ __device__ constexpr uint32_t gq_raw_bytes(uint32_t nsb, uint32_t sb) { return (nsb * sb + 15 + 15) / 16 * 16; }

// Host-side shape choice shared by the launches over unit streams. A wave that reduces
// `units` units (one per lane per round) takes ceil(units / 64) rounds; a SIMD issues its
// waves' rounds back to back when it holds several (throughput), while a lone wave waits
// on its own LDS and dot-product chains, measured at about 4x its issue time (latency).
// The cost is the larger of the two; the launchers pick the rows per wave with the least
// cost, and on a tie the most rows (fewer workgroups stage the activations).
__host__ inline double gq_cost(double units, double waves, int cus) {
    const double rounds = __builtin_ceil(units / 64.0), per_simd = waves / (4.0 * cus);
    return rounds * (per_simd > 4.0 ? per_simd : 4.0);
}
// Units a wave of `rows` rows of K values reduces (unit size v; rows that start inside a
// unit cost one more).
__host__ inline double gq_units(int rows, int64_t K, uint32_t v) {
    return K % v == 0 ? (double)rows * (double)(K / v) : __builtin_ceil((double)rows * (double)K / v) + 1.0;
}

// Dot products of unit u (unit index in the flat stream) with the vector; b points at the
// unit's super-block (or block) in LDS. The unit's values start at column kk0 of some row
// (kk0 = (u V) % K, computed by the caller once per unit); 32-value sub-blocks whose flat
// value index g lies in [lo, hi) contribute to pa (still in that row) or pb (the next row,
// once kk reaches K; a unit spans at most two rows since K >= V). 32-bit indices
// (matrices below 2^31 values).
// WRAP = false: K is a multiple of the unit's values, so every unit lies inside one row
// and inside [lo, hi) (the caller's units are whole rows); the row checks compile away.
template <int TYPE, bool WRAP = true, bool SPLIT = false>
__device__ __forceinline__ void gq_unit(const uint8_t* __restrict__ b, uint32_t u, uint32_t kk0, uint32_t K, uint32_t lo,
                                        uint32_t hi, const GqVec& x, float& pa, float& pb) {
    auto d32 = [&](const uint32_t q[8], uint32_t kk) {
        return SPLIT ? dot32s(q, gq_x(x, kk), gq_xl(x, kk)) : dot32(q, gq_x(x, kk));
    };

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
    // sub-block j's activations into r (issued a sub-block ahead of their use: the LDS
    // latency then overlaps the previous sub-block's arithmetic)
    auto ldx = [&](uint32_t j, GqXr& r) {
        const uint32_t kk = col(j);
        const uint8_t* ph = gq_x(x, kk);
#pragma unroll
        for (int i = 0; i < 4; ++i) r.h[i] = ld16u(ph + 16 * i);
        if (SPLIT) {
            const uint8_t* pl = gq_xl(x, kk);
#pragma unroll
            for (int i = 0; i < 4; ++i) r.l[i] = ld16u(pl + 16 * i);
        }
        if (TYPE == 14) {
            r.s[0] = x.s16[kk / 16];
            r.s[1] = x.s16[kk / 16 + 1];
        } else {
            r.s[0] = x.s32[kk / 32];
        }
    };
    if constexpr (TYPE == 8) {
        if (outside(g0)) return;
        const float d = f16_bits_to_f32(*reinterpret_cast<const uint16_t*>(b));
        uint32_t qw[8];
        lds_words<8>(b + 2, qw);
        uint32_t ql[8], qh[8];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const uint32_t wa = qw[i] ^ 0x80808080u, wc = qw[4 + i] ^ 0x80808080u;  // q + 128
            ql[i] = wa & 0x0F0F0F0Fu;
            qh[i] = (wa >> 4) & 0x0F0F0F0Fu;
            ql[4 + i] = wc & 0x0F0F0F0Fu;
            qh[4 + i] = (wc >> 4) & 0x0F0F0F0Fu;
        }
        const uint32_t kk = kk0;
        const float sx = x.s32[kk / 32];
        // sum q x = sum (16 qh + ql - 128) x
        const float dl = d32(ql, kk) - 128.0f * sx, dh = d32(qh, kk) - 128.0f * sx;
        pa += d * (16.0f * dh + dl - 128.0f * sx);
    } else if constexpr (TYPE == 12 || TYPE == 13) {
        // half hh of super-block u / 2: sub-blocks 4 hh .. 4 hh + 3, qs bytes [64 hh, + 64)
        // (32 bytes per pair of sub-blocks, low nibbles then high), all 32 qh bytes (Q5_K:
        // bit j of byte i is the fifth bit of value i of sub-block j), the 12 scale bytes
        constexpr int QS = TYPE == 12 ? 16 : 48;
        const uint32_t hh = u & 1;
        const u32x4 hdr = ld16u(b);  // d, dmin | scales[12]
        u32x4 qv[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) qv[i] = ld16u(b + QS + 64 * hh + 16 * i);
        u32x4 hv[2];
        if constexpr (TYPE == 13) {
            hv[0] = ld16u(b + 16);
            hv[1] = ld16u(b + 32);
#pragma unroll
            for (int i = 0; i < 2; ++i)
#pragma unroll
                for (int e = 0; e < 4; ++e) hv[i][e] >>= 4 * hh;  // bit jl: sub-block 4 hh + jl
        }
        const float d = f16_bits_to_f32(hdr[0] & 0xFFFFu), dmin = f16_bits_to_f32(hdr[0] >> 16);
        GqXr xr[2];
        ldx(0, xr[0]);
#pragma unroll
        for (int jl = 0; jl < 4; ++jl) {
            if (jl + 1 < 4) ldx(jl + 1, xr[(jl + 1) & 1]);
            __builtin_amdgcn_sched_barrier(0);
            if (outside(g0 + 32 * jl)) continue;
            // the 6-bit scale and min of sub-block j = 4 hh + jl (ggml's get_scale_min_k4):
            // j < 4 from bytes j, j + 4; j >= 4 from the low / high nibbles of byte j + 4 and
            // the top two bits of bytes j - 4, j
            const uint32_t b0 = (hdr[1] >> (8 * jl)) & 0xFFu, b1 = (hdr[2] >> (8 * jl)) & 0xFFu;
            const uint32_t b2 = (hdr[3] >> (8 * jl)) & 0xFFu;
            const uint32_t sc = hh ? ((b2 & 15u) | ((b0 >> 6) << 4)) : (b0 & 63u);
            const uint32_t m = hh ? ((b2 >> 4) | ((b1 >> 6) << 4)) : (b1 & 63u);
            uint32_t q[8];
            const int c = jl >> 1, sh = 4 * (jl & 1);
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                uint32_t n = (qv[2 * c + (i >> 2)][i & 3] >> sh) & 0x0F0F0F0Fu;
                if constexpr (TYPE == 13) n |= ((hv[i >> 2][i & 3] >> jl) & 0x01010101u) << 4;
                q[i] = n;
            }
            const float sx = xr[jl & 1].s[0];
            const float dq = dot32x<SPLIT>(q, xr[jl & 1]) - 128.0f * sx;
            add(jl, d * (float)sc * dq - dmin * (float)m * sx);
        }
    } else {  // Q6_K, half h of super-block u / 2: ql[64h, +64), qh[32h, +32), sc[8h, +8), d @208
        const uint32_t hh = u & 1;
        uint32_t lw[16], hw[8], sw2[2];
        lds_words<16>(b + 64 * hh, lw);
        lds_words<8>(b + 128 + 32 * hh, hw);
        lds_words<2>(b + 192 + 8 * hh, sw2);
        u32x4 l[4], qh[2];
#pragma unroll
        for (int i = 0; i < 4; ++i) l[i] = u32x4{lw[4 * i], lw[4 * i + 1], lw[4 * i + 2], lw[4 * i + 3]};
        qh[0] = u32x4{hw[0], hw[1], hw[2], hw[3]};
        qh[1] = u32x4{hw[4], hw[5], hw[6], hw[7]};
        const uint2 scw = make_uint2(sw2[0], sw2[1]);
        const float d = f16_bits_to_f32(*reinterpret_cast<const uint16_t*>(b + 208));
        GqXr xr[2];
        ldx(0, xr[0]);
#pragma unroll
        for (int t = 0; t < 4; ++t) {  // 32-value quarter t of the half
            if (t + 1 < 4) ldx(t + 1, xr[(t + 1) & 1]);
            __builtin_amdgcn_sched_barrier(0);
            if (outside(g0 + 32 * t)) continue;
            uint32_t q[8];
            const int shl = 4 * (t >> 1), shh = 2 * t;
#pragma unroll
            for (int i = 0; i < 8; ++i)
                q[i] = ((l[2 * (t & 1) + (i >> 2)][i & 3] >> shl) & 0x0F0F0F0Fu) |
                       (((qh[i >> 2][i & 3] >> shh) & 0x03030303u) << 4);
            const float s0 = xr[t & 1].s[0], s1 = xr[t & 1].s[1];
            const uint32_t sw = t < 2 ? scw.x : scw.y;
            const float sc0 = (float)(int8_t)((sw >> (16 * (t & 1))) & 0xFFu);
            const float sc1 = (float)(int8_t)((sw >> (16 * (t & 1) + 8)) & 0xFFu);
            // codes are q + 32 (0..63): sum (q) x = sum (128 + q + 32) x - 160 sum x
            const float a0 = dot16x<SPLIT>(q, xr[t & 1], 0) - 160.0f * s0;
            const float a1 = dot16x<SPLIT>(q + 4, xr[t & 1], 1) - 160.0f * s1;
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
