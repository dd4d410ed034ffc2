// GGUF matvec (y = deq(W) x for up to 8 tokens, Q8_0 / Q4_K / Q5_K / Q6_K) as a weight
// stream of 32-value sub-blocks.
//
// Work unit: one lane, one 32-value sub-block of a row (a Q8_0 block, or one eighth of a
// K-quant super-block). A row of K values has C = K / 32 sub-blocks and no sub-block
// straddles two rows, so a lane's work is always (row, column c). Lanes keep their columns
// for the whole launch: lane l takes column l (and l + 64 when C > 64), or, when C < 64,
// column l % C of every (64 / C)-th row, so the activations of a lane's columns sit in its
// registers for the whole stream.
//
// Activations: every workgroup quantises its token's vector once, per 32-value block, as two
// int8 terms, x ~= s (hi + lo / 254) with s = max|x| / 127 (at least 2^-126): hi = rint(x / s), lo =
// rint((x / s - hi) 254). |x - s (hi + lo / 254)| <= max|x| / (127 * 508) = 1.6e-5 max|x|:
// about 16 significant bits relative to the block's largest value. The exact sums of the
// block (and of its 16-value halves, for Q6_K) come along in fp32.
// Dot products: a sub-block's codes become 32 bytes (4 per dword; Q8_0 codes are already
// int8, the K-quants' 4..6-bit codes are unpacked to 0..63), v_dot4_i32_i8 sums codes x hi
// and codes x lo in int32 (exact), and the scales are applied once per sub-block:
//   Q4_K / Q5_K: d sc s (ihi + ilo / 254) - dmin m sum32(x)
//   Q6_K: d sum_h sc_h (s (ihi_h + ilo_h / 254) - 32 sum16_h(x))   (codes q + 32)
//   Q8_0: d s (ihi + ilo / 254)
// Loads: the token's activations (1 KB pieces dealt round the waves) and then the wave's rows of
// super-blocks are copied into LDS with contiguous buffer-to-LDS transfers; the wave waits
// for its activations with the weights still in flight, and starts on a row as soon as the
// transfers that hold it are complete (an exact vmcnt per row).
//
// Workgroup = 4..16 waves of one token (about one workgroup per CU), wave = RM rows.
//
// Semantics: tinyserve/gguf_dequant_torch.py:101-249 (formats), tinyserve/csrc/ggml_ops.cu:
// 461-569 (y = deq(W) x in fp32).
#include "fused_common.h"
#include "mfma_tile.h"
#include "gguf_dot.h"

namespace tsa {
namespace {

constexpr int GS_RD = 8;        // rows per wave, at most
constexpr int GS_MIN_WAVES = 4;  // waves per workgroup, at least (4 K / 32 <= 2 * 64 * 4 items)
constexpr int GS_MAX_WAVES = 16;
constexpr int GS_ITEMS = 2;     // activation quarters (8 values) a thread quantises, at most
constexpr int XQ_BYTES = 80;    // a quantised block in LDS: hi[8], lo[8] dwords, s, sum32, sum16 x 2

// A lane's quantised activation block.
struct XQ {
    uint32_t h[8], l[8];
    float s, s32, s16a, s16b;
};

__device__ __forceinline__ XQ xq_read(const uint8_t* p) {
    XQ x;
    const u32x4 a = ld16u(p), b = ld16u(p + 16), c = ld16u(p + 32), d = ld16u(p + 48), e = ld16u(p + 64);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        x.h[i] = a[i];
        x.h[4 + i] = b[i];
        x.l[i] = c[i];
        x.l[4 + i] = d[i];
    }
    x.s = __uint_as_float(e[0]);
    x.s32 = __uint_as_float(e[1]);
    x.s16a = __uint_as_float(e[2]);
    x.s16b = __uint_as_float(e[3]);
    return x;
}

// 8 raw activation values of one quarter-block, as loaded (bf16 / fp16: 4 dwords; fp32: 8).
struct XRaw {
    uint32_t w[8];
};
__device__ __forceinline__ void xraw_values(const XRaw& r, int dtype, float (&f)[8]) {
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        if (dtype == TSA_F32) {
            f[i] = __uint_as_float(r.w[i]);
        } else {
            const uint32_t b = (r.w[i >> 1] >> (16 * (i & 1))) & 0xFFFFu;
            f[i] = dtype == TSA_BF16 ? bf16_bits_to_f32(b) : f16_bits_to_f32(b);
        }
    }
}

// The activation items of one workgroup: nvec vectors of C blocks, item i = (vector i /
// (4C), block (i % 4C) / 4, quarter i % 4) for i = i0 + tid + nthr m, quantised by gs_quant.
struct XItems {
    XRaw r[GS_ITEMS];
};
// The items, read from a raw copy of the vectors in LDS (vectors back to back).
__device__ __forceinline__ void gs_items_lds(XItems& it, const uint8_t* raw, int dtype, int nvec, int C, int tid,
                                             int nthr, int i0 = 0) {
    const int total = nvec * 4 * C, es = dtype == TSA_F32 ? 4 : 2;
#pragma unroll
    for (int m = 0; m < GS_ITEMS; ++m) {
        const int i = i0 + tid + nthr * m;
        const int ii = i < total ? i : 0;
        const uint8_t* q = raw + 8 * es * ii;  // vectors back to back: item ii starts at value 8 ii
        const u32x4 a = ld16u(q);
        const u32x4 b = es == 4 ? ld16u(q + 16) : u32x4{0u, 0u, 0u, 0u};
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            it.r[m].w[e] = a[e];
            it.r[m].w[4 + e] = b[e];
        }
    }
}

// Quantises the loaded items into dst (block b = v C + c at dst + XQ_BYTES b). The four
// threads of a block are four consecutive lanes (4C items per vector): their maximum and
// sums come from DPP quad exchanges.
__device__ __forceinline__ void gs_quant(const XItems& it, uint8_t* dst, int dtype, int nvec, int C, int tid,
                                         int nthr, int i0 = 0) {
    const int total = nvec * 4 * C;
#pragma unroll
    for (int m = 0; m < GS_ITEMS; ++m) {
        const int i = i0 + tid + nthr * m;
        if (i0 + nthr * m >= total) break;  // workgroup-uniform: no thread has this item
        float f[8];
        xraw_values(it.r[m], dtype, f);
        float amax = 0.0f, sum = 0.0f;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            amax = __builtin_fmaxf(amax, __builtin_fabsf(f[e]));
            sum += f[e];
        }
        amax = __builtin_fmaxf(amax, dpp_f<0xB1, 0xF, 0xF>(amax, 0.0f));  // quad_perm [1,0,3,2]
        amax = __builtin_fmaxf(amax, dpp_f<0x4E, 0xF, 0xF>(amax, 0.0f));  // quad_perm [2,3,0,1]
        const float s16 = sum + dpp_f<0xB1, 0xF, 0xF>(sum, 0.0f);
        const float s32 = s16 + dpp_f<0x4E, 0xF, 0xF>(s16, 0.0f);
        // s = amax / 127 (at least 2^-126, so 1/s stays finite; an all-zero block then codes
        // as zeros); u = f / s in [-127, 127]. Adding 1.5 * 2^23 rounds u to the nearest
        // integer (ties to even) in the low mantissa bits, whose low byte is the two's
        // complement code; the remainder u - hi in [-1/2, 1/2] gives lo = rint(254 (u - hi)).
        const float s = __builtin_fmaxf(amax * (1.0f / 127.0f), 0x1p-126f);
        const float inv = __builtin_amdgcn_rcpf(s);
        constexpr float RND = 0x1.8p23f;
        uint32_t hb[8], lb[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            const float th = __builtin_fmaf(f[e], inv, RND);
            const float r = __builtin_fmaf(f[e], inv, -(th - RND));
            hb[e] = __float_as_uint(th);
            lb[e] = __float_as_uint(__builtin_fmaf(r, 254.0f, RND));
        }
        uint32_t hw[2], lw[2];
#pragma unroll
        for (int h = 0; h < 2; ++h) {  // low bytes of four words -> one word (v_perm_b32)
            hw[h] = __builtin_amdgcn_perm(__builtin_amdgcn_perm(hb[4 * h + 3], hb[4 * h + 2], 0x0C0C0400u),
                                          __builtin_amdgcn_perm(hb[4 * h + 1], hb[4 * h], 0x0C0C0400u), 0x05040100u);
            lw[h] = __builtin_amdgcn_perm(__builtin_amdgcn_perm(lb[4 * h + 3], lb[4 * h + 2], 0x0C0C0400u),
                                          __builtin_amdgcn_perm(lb[4 * h + 1], lb[4 * h], 0x0C0C0400u), 0x05040100u);
        }
        if (i < total) {
            const int b = i >> 2, q = i & 3;
            uint8_t* p = dst + XQ_BYTES * b;
            *reinterpret_cast<uint2*>(p + 8 * q) = make_uint2(hw[0], hw[1]);
            *reinterpret_cast<uint2*>(p + 32 + 8 * q) = make_uint2(lw[0], lw[1]);
            if (q == 0) *reinterpret_cast<float2*>(p + 64) = make_float2(s, s32);
            if ((q & 1) == 0) *reinterpret_cast<float*>(p + 72 + 2 * q) = s16;  // q 0: first half, q 2: second
        }
    }
}

// All nvec vectors (raw in LDS at raw, back to back) quantised into dst, in rounds of
// GS_ITEMS items per thread. The caller's barrier makes dst visible.
__device__ __forceinline__ void gs_quant_all(const uint8_t* raw, uint8_t* dst, int dtype, int nvec, int C, int tid,
                                             int nthr) {
    for (int i0 = 0; i0 < nvec * 4 * C; i0 += GS_ITEMS * nthr) {
        XItems xi;
        gs_items_lds(xi, raw, dtype, nvec, C, tid, nthr, i0);
        gs_quant(xi, dst, dtype, nvec, C, tid, nthr, i0);
    }
}

__device__ __forceinline__ int sdot4(uint32_t a, uint32_t b, int c) {
    return __builtin_amdgcn_sdot4((int)a, (int)b, c, false);
}

// sum over the block of code x activation, as s (hi + lo / 254), for the 8 code words q
// (dwords i0 .. i1 - 1).
template <int I0, int I1>
__device__ __forceinline__ float qdot(const uint32_t (&q)[8], const XQ& x) {
    int ih = 0, il = 0;
#pragma unroll
    for (int i = I0; i < I1; ++i) {
        ih = sdot4(q[i], x.h[i], ih);
        il = sdot4(q[i], x.l[i], il);
    }
    return x.s * ((float)ih + (float)il * (1.0f / 254.0f));
}

// k_scale_min for a sub-block index j that differs between lanes: both forms from the same
// three bytes, then a select (no divergent branch).
__device__ __forceinline__ void k_scale_min_lanes(const uint32_t s[3], int j, uint32_t& sc, uint32_t& m) {
    const uint32_t sh = 8u * (uint32_t)(j & 3);
    const uint32_t b0 = __builtin_amdgcn_ubfe(s[0], sh, 8), b1 = __builtin_amdgcn_ubfe(s[1], sh, 8);
    const uint32_t b2 = __builtin_amdgcn_ubfe(s[2], sh, 8);
    const bool lo = j < 4;
    sc = lo ? (b0 & 63u) : ((b2 & 15u) | ((b0 >> 6) << 4));
    m = lo ? (b1 & 63u) : ((b2 >> 4) | ((b1 >> 6) << 4));
}

// Sub-block j (0..7; 0 for Q8_0) of the super-block (block) at p in LDS, dotted with x.
template <int TY>
__device__ __forceinline__ float sb_dot(const uint8_t* p, int j, const XQ& x) {
    uint32_t q[8];
    if constexpr (TY == 8) {
        const float d = f16_bits_to_f32(*reinterpret_cast<const uint16_t*>(p));
        lds_words<8>(p + 2, q);
        return d * qdot<0, 8>(q, x);
    } else if constexpr (TY == 12 || TY == 13) {
        constexpr int QS = TY == 12 ? 16 : 48;
        const u32x4 hdr = ld16u(p);
        const u32x4 a = ld16u(p + QS + 32 * (j >> 1)), b = ld16u(p + QS + 32 * (j >> 1) + 16);
        const int sh = 4 * (j & 1);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            q[i] = (a[i] >> sh) & 0x0F0F0F0Fu;
            q[4 + i] = (b[i] >> sh) & 0x0F0F0F0Fu;
        }
        if constexpr (TY == 13) {
            const u32x4 ha = ld16u(p + 16), hb = ld16u(p + 32);
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                q[i] |= ((ha[i] >> j) & 0x01010101u) << 4;
                q[4 + i] |= ((hb[i] >> j) & 0x01010101u) << 4;
            }
        }
        const float d = f16_bits_to_f32(hdr[0] & 0xFFFFu), dmin = f16_bits_to_f32(hdr[0] >> 16);
        const uint32_t s[3] = {hdr[1], hdr[2], hdr[3]};
        uint32_t sc, m;
        k_scale_min_lanes(s, j, sc, m);
        return d * (float)sc * qdot<0, 8>(q, x) - dmin * (float)m * x.s32;
    } else {  // Q6_K: half h = j / 4, quarter t = j % 4 of it
        const int h = j >> 2, t = j & 3;
        uint32_t lw[8], hw[8];
        lds_words<8>(p + 64 * h + 32 * (t & 1), lw);
        lds_words<8>(p + 128 + 32 * h, hw);
        const int shl = 4 * (t >> 1), shh = 2 * t;
#pragma unroll
        for (int i = 0; i < 8; ++i) q[i] = ((lw[i] >> shl) & 0x0F0F0F0Fu) | (((hw[i] >> shh) & 0x03030303u) << 4);
        const uint32_t scw = *reinterpret_cast<const uint16_t*>(p + 192 + 2 * j);
        const float d = f16_bits_to_f32(*reinterpret_cast<const uint16_t*>(p + 208));
        const float sc0 = (float)(int8_t)(scw & 0xFFu), sc1 = (float)(int8_t)(scw >> 8);
        return d * (sc0 * (qdot<0, 4>(q, x) - 32.0f * x.s16a) + sc1 * (qdot<4, 8>(q, x) - 32.0f * x.s16b));
    }
}

template <int TY> struct GsType;
template <> struct GsType<8>  { static constexpr uint32_t SB = 34,  SPB = 1; };
template <> struct GsType<12> { static constexpr uint32_t SB = 144, SPB = 8; };
template <> struct GsType<13> { static constexpr uint32_t SB = 176, SPB = 8; };
template <> struct GsType<14> { static constexpr uint32_t SB = 210, SPB = 8; };

// A wave's staged range of one matrix: the super-blocks holding sub-blocks [f0, f1).
struct Range {
    uint32_t s0;     // first super-block
    uint32_t shift;  // the first super-block's offset in the LDS area (its address % 16)
    uint32_t bytes;  // bytes transferred (whole 16-byte chunks)
};
template <int TY>
__device__ __forceinline__ Range range_of(uint32_t off, uint32_t f0, uint32_t f1) {
    using G = GsType<TY>;
    Range r;
    r.s0 = f0 / G::SPB;
    const uint32_t s1 = (f1 + G::SPB - 1) / G::SPB;
    const uint32_t first = off + r.s0 * G::SB;
    r.shift = first & 15u;
    r.bytes = ((s1 - r.s0) * G::SB + r.shift + 15u) / 16u * 16u;
    return r;
}
// 1 KB transfers of the range that hold the sub-blocks before f_end.
template <int TY>
__device__ __forceinline__ uint32_t chunks_until(const Range& r, uint32_t f_end) {
    using G = GsType<TY>;
    const uint32_t s_end = (f_end + G::SPB - 1) / G::SPB;
    return ((s_end - r.s0) * G::SB + r.shift + 1023u) / 1024u;
}
__device__ __forceinline__ uint32_t chunks(const Range& r) { return (r.bytes + 1023u) / 1024u; }

// Waits until at most n of this wave's loads are outstanding (n above 31: 31, stricter).
#define GS_WAIT_CASE(n) \
    case n: asm volatile("s_waitcnt vmcnt(" #n ")" ::: "memory"); break;
__device__ __forceinline__ void gs_wait(int n) {
    switch (n) {
        GS_WAIT_CASE(0) GS_WAIT_CASE(1) GS_WAIT_CASE(2) GS_WAIT_CASE(3) GS_WAIT_CASE(4) GS_WAIT_CASE(5)
        GS_WAIT_CASE(6) GS_WAIT_CASE(7) GS_WAIT_CASE(8) GS_WAIT_CASE(9) GS_WAIT_CASE(10) GS_WAIT_CASE(11)
        GS_WAIT_CASE(12) GS_WAIT_CASE(13) GS_WAIT_CASE(14) GS_WAIT_CASE(15) GS_WAIT_CASE(16) GS_WAIT_CASE(17)
        GS_WAIT_CASE(18) GS_WAIT_CASE(19) GS_WAIT_CASE(20) GS_WAIT_CASE(21) GS_WAIT_CASE(22) GS_WAIT_CASE(23)
        GS_WAIT_CASE(24) GS_WAIT_CASE(25) GS_WAIT_CASE(26) GS_WAIT_CASE(27) GS_WAIT_CASE(28) GS_WAIT_CASE(29)
        GS_WAIT_CASE(30)
        default: asm volatile("s_waitcnt vmcnt(31)" ::: "memory"); break;
    }
    __builtin_amdgcn_wave_barrier();
}
#undef GS_WAIT_CASE

// A lane's place in a stream of rows of C sub-blocks: its columns c0 (and c0 + 64 when
// two), its row group g of G (rows g, g + G, ...), and whether it has any column.
struct Lanes {
    int c0, ncol, g, G;
};
__device__ __forceinline__ Lanes lanes_of(int C, int lane) {
    Lanes m;
    if (C >= 64) {
        m.c0 = lane;
        m.ncol = lane + 64 < C ? 2 : 1;
        m.g = 0;
        m.G = 1;
    } else {
        m.G = 64 / C;
        m.g = lane / C;
        m.c0 = lane - m.g * C;
        m.ncol = m.g < m.G ? 1 : 0;
    }
    return m;
}

template <int N>
__device__ __forceinline__ void acc_put(float (&acc)[N], int r, float v) {
#pragma unroll
    for (int i = 0; i < N; ++i)
        if (r == i) acc[i] += v;
}

struct GsMvParams {
    const uint8_t* w;
    uint32_t w_records;
    const void* x;
    uint32_t x_records;  // bytes of x
    int x_dtype;
    void* y;
    int y_dtype;
    int N, K, rm;
    int xq_off, xraw_off, raw_off, raw_stride;
};

template <int TY>
__global__ void __launch_bounds__(64 * GS_MAX_WAVES) gs_matvec_kernel(GsMvParams p) {
    extern __shared__ __align__(16) uint8_t smem[];
    using G = GsType<TY>;
    const int tid = threadIdx.x, lane = tid & 63, wave = uniform(tid >> 6);
    const int K = p.K, N = p.N, C = K / 32, t = blockIdx.y;
    const int nw = (int)(blockDim.x >> 6);
    const int n0 = ((int)blockIdx.x * nw + wave) * p.rm;
    const int nr = n0 >= N ? 0 : (N - n0 < p.rm ? N - n0 : p.rm);
    uint8_t* rbuf = smem + p.raw_off + wave * p.raw_stride;
    const uint32_t f0 = (uint32_t)n0 * C, f1 = (uint32_t)(n0 + nr) * C;
    // copies read 16-byte-aligned memory: the buffer starts at the boundary at or below w
    const uint32_t mis = (uint32_t)reinterpret_cast<uintptr_t>(p.w) & 15u;
    const Range rw = range_of<TY>(mis, f0, f1);
    // the token's activations (1 KB pieces dealt round the waves) and then the weight rows,
    // all as buffer-to-LDS copies, so the activations can be waited for with the weights
    // still out
    const uint32_t xbytes = (uint32_t)K * (p.x_dtype == TSA_F32 ? 4u : 2u);  // a multiple of 64
    for (uint32_t c = 1024u * wave; c < xbytes; c += 1024u * nw)
        gq_stage_raw(static_cast<const uint8_t*>(p.x), p.x_records, (uint32_t)t * xbytes + c,
                     xbytes - c < 1024u ? xbytes - c : 1024u,
                     (uint32_t)reinterpret_cast<uintptr_t>(smem + p.xraw_off) + c, lane);
    if (nr > 0)
        gq_stage_raw(p.w - mis, gq_records(p.w_records, mis), mis + rw.s0 * G::SB - rw.shift, rw.bytes,
                     (uint32_t)reinterpret_cast<uintptr_t>(rbuf), lane);
    const int total = nr > 0 ? (int)chunks(rw) : 0;
    gs_wait(total);
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    __syncthreads();  // every wave's pieces of the activations are in LDS
    XItems xi;
    gs_items_lds(xi, smem + p.xraw_off, p.x_dtype, 1, C, tid, 64 * nw);
    gs_quant(xi, smem + p.xq_off, p.x_dtype, 1, C, tid, 64 * nw);
    __syncthreads();
    if (nr == 0) return;
    const Lanes ln = lanes_of(C, lane);
    XQ x0 = xq_read(smem + p.xq_off + XQ_BYTES * ln.c0), x1 = x0;
    if (ln.ncol > 1) x1 = xq_read(smem + p.xq_off + XQ_BYTES * (ln.c0 + 64));
    float acc[8];
#pragma unroll
    for (int r = 0; r < 8; ++r) acc[r] = 0.0f;
    for (int r0 = 0; r0 < nr; r0 += ln.G) {
        const int rmax = r0 + ln.G - 1 < nr ? r0 + ln.G - 1 : nr - 1;
        gs_wait(total - (int)chunks_until<TY>(rw, f0 + (uint32_t)(rmax + 1) * C));
        const int r = r0 + ln.g;
        if (ln.ncol == 0 || r >= nr) continue;
        const uint8_t* area = rbuf + rw.shift;
        float part = 0.0f;
        {
            const uint32_t f = f0 + (uint32_t)r * C + ln.c0;
            part += sb_dot<TY>(area + (f / G::SPB - rw.s0) * G::SB, (int)(f % G::SPB), x0);
        }
        if (ln.ncol > 1) {
            const uint32_t f = f0 + (uint32_t)r * C + ln.c0 + 64;
            part += sb_dot<TY>(area + (f / G::SPB - rw.s0) * G::SB, (int)(f % G::SPB), x1);
        }
        acc_put(acc, r, part);
    }
    const float tot = wave_sum_rows<8>(acc, lane);
    const int r = lane >> 3;
    if ((lane & 7) == 0 && r < nr) store_out(p.y, p.y_dtype, (int64_t)t * N + n0 + r, tot);
}

// ---------------------------------------------------------------- expert decode
// Top-k GGUF expert decode as two launches over the same 32-value sub-block units:
//   gs_gate_up_kernel: workgroup = (row group of the intermediate dimension, (token, expert)
//     pair); each workgroup quantises its token's activations, each wave streams its rows of
//     gate and the same rows of up (per-row waits) and writes h = act(gate, up) as bf16, as
//     the super-block kernels do. Routed calls select the token's experts in the prologue
//     (the x copies are already out) and the first workgroup of each token writes the
//     selection for the down launch.
//   gs_down_kernel: workgroup = (row group of the hidden dimension, token); each workgroup
//     quantises the token's k h vectors, each wave streams its rows of every selected
//     expert's down in expert order and keeps sum_j w_j (row . h_j), so every output has one
//     writer and the sum runs in a fixed order.

constexpr int GS_MISC = 512;  // LDS: the routing tables (slots, weights) of the token group

struct GsDecParams {
    tsa_expert_layout L;
    const uint8_t* pool;
    int64_t n_slots;
    const int32_t* slots;        // [T, k]: given slots, or (down, routed) the selection gate_up made
    const float* wts;            // [T, k]
    const void* logits;          // gate_up, routed: [T, E] (slots unused)
    const int32_t* expert_slot;  // [E] (routed)
    int32_t* idx_out;            // [T, k] (routed, optional)
    float* w_out;
    int32_t* tab_slot;           // routed: the selection, for the down launch
    float* tab_w;
    int logits_dtype, route_mode, E;
    int T, k;
    const void* x;               // gate_up: x [T, H]; down: h [T k, I] (bf16)
    uint32_t x_records;
    int x_dtype;
    uint16_t* h;                 // gate_up: h [T k, I] (bf16)
    void* y;                     // down: y [T, H]
    int y_dtype;
    int rm;                      // rows per wave
    int xq_off, xraw_off, raw_off, raw_stride;
};

// Rows [n0, n0 + nr) of a matrix of C sub-blocks per row at mat (mat_bytes long) into LDS at
// dst: the buffer starts at the 16-byte boundary at or below mat, so every copy reads 16
// whole aligned bytes.
template <int TY>
__device__ __forceinline__ Range gs_issue_rows(const uint8_t* mat, uint32_t mat_bytes, int n0, int nr, int C,
                                               uint32_t dst, int lane) {
    using G = GsType<TY>;
    const uint32_t mis = (uint32_t)reinterpret_cast<uintptr_t>(mat) & 15u;
    const Range r = range_of<TY>(mis, (uint32_t)n0 * C, (uint32_t)(n0 + nr) * C);
    gq_stage_raw(mat - mis, gq_records(mat_bytes, mis), mis + r.s0 * G::SB - r.shift, r.bytes, dst, lane);
    return r;
}

__device__ __forceinline__ uint32_t lds_addr(const uint8_t* p) { return (uint32_t)reinterpret_cast<uintptr_t>(p); }

// n bytes of src from byte off into LDS at dst, in 1 KB pieces dealt round the waves.
__device__ __forceinline__ void gs_stage_vecs(const void* src, uint32_t records, uint32_t off, uint32_t n, uint8_t* dst,
                                              int wave, int nw, int lane) {
    for (uint32_t c = 1024u * wave; c < n; c += 1024u * nw)
        gq_stage_raw(static_cast<const uint8_t*>(src), records, off + c, n - c < 1024u ? n - c : 1024u, lds_addr(dst) + c,
                     lane);
}

template <int TY>
__global__ void __launch_bounds__(64 * GS_MAX_WAVES) gs_gate_up_kernel(GsDecParams p) {
    extern __shared__ __align__(16) uint8_t smem[];
    using G = GsType<TY>;
    const int tid = threadIdx.x, lane = tid & 63, wave = uniform(tid >> 6), nw = (int)(blockDim.x >> 6);
    const tsa_expert_layout& L = p.L;
    const int H = (int)L.hidden, I = (int)L.inter, k = p.k, C = H / 32;
    const int a = blockIdx.y, t = a / k, j = a - t * k;
    int* s_slot = reinterpret_cast<int*>(smem);
    float* s_w = reinterpret_cast<float*>(smem + 4 * FUSED_MAXT * FUSED_MAXK);
    // given slots: the pair's slot as a scalar load ahead of the copies (after them it would
    // be a vector load whose wait covers them)
    const int64_t given = p.logits ? -1 : uniform(p.slots[(int64_t)t * k + j]);
    const uint32_t xbytes = (uint32_t)H * (p.x_dtype == TSA_F32 ? 4u : 2u);  // a multiple of 64
    // the activation copies: every wave, or (routed) every wave but wave 0, which selects the
    // token's experts meanwhile (its logit loads would otherwise queue behind its copies)
    if (!p.logits) gs_stage_vecs(p.x, p.x_records, (uint32_t)t * xbytes, xbytes, smem + p.xraw_off, wave, nw, lane);
    else if (wave > 0)
        gs_stage_vecs(p.x, p.x_records, (uint32_t)t * xbytes, xbytes, smem + p.xraw_off, wave - 1, nw - 1, lane);
    int64_t slot;
    if (p.logits) {
        if (wave == 0) {
            int es[4];
#pragma unroll
            for (int q = 0; q < 4; ++q) es[q] = p.expert_slot[min(lane + 64 * q, p.E - 1)];
            const int sel = route_token(p, t, lane, es, s_slot, s_w);
            if (blockIdx.x == 0 && j == 0 && lane < k) {
                if (p.idx_out) {
                    p.idx_out[t * k + lane] = sel;
                    p.w_out[t * k + lane] = s_w[t * k + lane];
                }
                p.tab_slot[t * k + lane] = s_slot[t * k + lane];
                p.tab_w[t * k + lane] = s_w[t * k + lane];
            }
        }
        __syncthreads();
        slot = uniform(s_slot[t * k + j]);
    } else {
        slot = given;
    }
    const bool live = slot >= 0 && slot < p.n_slots;
    const int n0 = ((int)blockIdx.x * nw + wave) * p.rm;
    const int nr = !live || n0 >= I ? 0 : (I - n0 < p.rm ? I - n0 : p.rm);
    uint8_t* rbuf = smem + p.raw_off + wave * p.raw_stride;
    const uint32_t half = (uint32_t)p.raw_stride / 2;
    const uint8_t* base = p.pool + (live ? slot : 0) * L.slot_bytes;
    const uint32_t mat_bytes = (uint32_t)((int64_t)I * C / G::SPB * G::SB);
    Range rg{}, ru{};
    int cg = 0, cu = 0;
    if (nr > 0) {
        rg = gs_issue_rows<TY>(base + L.gate_off, mat_bytes, n0, nr, C, lds_addr(rbuf), lane);
        ru = gs_issue_rows<TY>(base + L.up_off, mat_bytes, n0, nr, C, lds_addr(rbuf) + half, lane);
        cg = (int)chunks(rg);
        cu = (int)chunks(ru);
    }
    gs_wait(cg + cu);  // this wave's activation pieces are in
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    __syncthreads();
    gs_quant_all(smem + p.xraw_off, smem + p.xq_off, p.x_dtype, 1, C, tid, 64 * nw);
    __syncthreads();
    if (nr == 0) return;  // a dead pair's h is never read
    const Lanes ln = lanes_of(C, lane);
    XQ x0 = xq_read(smem + p.xq_off + XQ_BYTES * ln.c0), x1 = x0;
    if (ln.ncol > 1) x1 = xq_read(smem + p.xq_off + XQ_BYTES * (ln.c0 + 64));
    float acc[8];  // gate rows 0..3, up rows 0..3
#pragma unroll
    for (int r = 0; r < 8; ++r) acc[r] = 0.0f;
    const uint32_t f0 = (uint32_t)n0 * C;
    for (int m = 0; m < 2; ++m) {
        const Range& rw = m ? ru : rg;
        const uint8_t* area = rbuf + (m ? half : 0u) + rw.shift;
        for (int r0 = 0; r0 < nr; r0 += ln.G) {
            const int rmax = r0 + ln.G - 1 < nr ? r0 + ln.G - 1 : nr - 1;
            const int done = (int)chunks_until<TY>(rw, f0 + (uint32_t)(rmax + 1) * C);
            gs_wait(m ? cu - done : cg - done + cu);
            const int r = r0 + ln.g;
            if (ln.ncol == 0 || r >= nr) continue;
            const uint32_t f = f0 + (uint32_t)r * C + ln.c0;
            float part = sb_dot<TY>(area + (f / G::SPB - rw.s0) * G::SB, (int)(f % G::SPB), x0);
            if (ln.ncol > 1)
                part += sb_dot<TY>(area + ((f + 64) / G::SPB - rw.s0) * G::SB, (int)((f + 64) % G::SPB), x1);
            acc_put(acc, 4 * m + r, part);
        }
    }
    const float tot = wave_sum_rows<8>(acc, lane);  // lane 8 i: gate row i (i < 4), up row i - 4
    // up row r (lane 32 + 8 r) beside gate row r: the swap's second half, lower lanes
    const float up = __uint_as_float(__builtin_amdgcn_permlane32_swap(__float_as_uint(tot), __float_as_uint(tot), false, false)[1]);
    const int r = lane >> 3;
    if ((lane & 7) == 0 && r < nr) {
        const float hv = L.act == TSA_ACT_SWIGLU_OAI ? swiglu_oai(L, tot, up) : tot * sigmoidf_(tot) * up;
        p.h[(int64_t)a * I + n0 + r] = f32_to_bf16_bits(hv);
    }
}

template <int TY>
__global__ void __launch_bounds__(64 * GS_MAX_WAVES) gs_down_kernel(GsDecParams p) {
    extern __shared__ __align__(16) uint8_t smem[];
    using G = GsType<TY>;
    const int tid = threadIdx.x, lane = tid & 63, wave = uniform(tid >> 6), nw = (int)(blockDim.x >> 6);
    const tsa_expert_layout& L = p.L;
    const int H = (int)L.hidden, I = (int)L.inter, k = p.k, C = I / 32, t = blockIdx.y;
    // the token's slots first, as scalar loads issued together (after the copies below they
    // would become vector loads that wait for those copies)
    int sl[FUSED_MAXK];
#pragma unroll
    for (int q = 0; q < FUSED_MAXK; ++q) sl[q] = uniform(p.slots[(int64_t)t * k + (q < k ? q : k - 1)]);
    const uint32_t vbytes = (uint32_t)k * (uint32_t)I * 2u;  // the token's k h vectors (bf16), back to back
    gs_stage_vecs(p.x, p.x_records, (uint32_t)t * vbytes, vbytes, smem + p.xraw_off, wave, nw, lane);
    const int n0 = ((int)blockIdx.x * nw + wave) * p.rm;
    const int nr = n0 >= H ? 0 : (H - n0 < p.rm ? H - n0 : p.rm);
    uint8_t* rbuf = smem + p.raw_off + wave * p.raw_stride;
    const uint32_t area = (uint32_t)p.raw_stride / (uint32_t)k;
    const uint32_t mat_bytes = (uint32_t)((int64_t)H * C / G::SPB * G::SB);
    int total = 0;
    if (nr > 0) {
#pragma unroll
        for (int j = 0; j < FUSED_MAXK; ++j) {  // every live expert's rows, in expert order
            if (j >= k) break;
            const int64_t slot = sl[j];
            if (slot < 0 || slot >= p.n_slots) continue;
            const Range rj = gs_issue_rows<TY>(p.pool + slot * L.slot_bytes + L.down_off, mat_bytes, n0, nr, C,
                                               lds_addr(rbuf) + area * (uint32_t)j, lane);
            total += (int)chunks(rj);
        }
    }
    gs_wait(total);  // this wave's pieces of the h vectors are in
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    __syncthreads();
    gs_quant_all(smem + p.xraw_off, smem + p.xq_off, TSA_BF16, k, C, tid, 64 * nw);
    __syncthreads();
    if (nr == 0) return;
    const Lanes ln = lanes_of(C, lane);
    float acc[8];
#pragma unroll
    for (int r = 0; r < 8; ++r) acc[r] = 0.0f;
    const uint32_t f0 = (uint32_t)n0 * C;
    int before = 0;
    for (int j = 0; j < k; ++j) {
        const int64_t slot = uniform(p.slots[(int64_t)t * k + j]);
        if (slot < 0 || slot >= p.n_slots) continue;
        const float wj = __int_as_float(uniform(__float_as_int(p.wts[(int64_t)t * k + j])));
        const uint8_t* mat = p.pool + slot * L.slot_bytes + L.down_off;
        const uint32_t mis = (uint32_t)reinterpret_cast<uintptr_t>(mat) & 15u;
        const Range rj = range_of<TY>(mis, f0, f0 + (uint32_t)nr * C);  // as issued
        const uint8_t* xqj = smem + p.xq_off + XQ_BYTES * j * C;
        XQ x0 = xq_read(xqj + XQ_BYTES * ln.c0), x1 = x0;
        if (ln.ncol > 1) x1 = xq_read(xqj + XQ_BYTES * (ln.c0 + 64));
        const uint8_t* ar = rbuf + area * (uint32_t)j + rj.shift;
        for (int r0 = 0; r0 < nr; r0 += ln.G) {
            const int rmax = r0 + ln.G - 1 < nr ? r0 + ln.G - 1 : nr - 1;
            gs_wait(total - before - (int)chunks_until<TY>(rj, f0 + (uint32_t)(rmax + 1) * C));
            const int r = r0 + ln.g;
            if (ln.ncol == 0 || r >= nr) continue;
            const uint32_t f = f0 + (uint32_t)r * C + ln.c0;
            float part = sb_dot<TY>(ar + (f / G::SPB - rj.s0) * G::SB, (int)(f % G::SPB), x0);
            if (ln.ncol > 1)
                part += sb_dot<TY>(ar + ((f + 64) / G::SPB - rj.s0) * G::SB, (int)((f + 64) % G::SPB), x1);
            acc_put(acc, r, wj * part);
        }
        before += (int)chunks(rj);
    }
    const float tot = wave_sum_rows<8>(acc, lane);
    const int r = lane >> 3;
    if ((lane & 7) == 0 && r < nr) store_out(p.y, p.y_dtype, (int64_t)t * H + n0 + r, tot);
}

template <int TY>
const void* gs_gu_fn() { return reinterpret_cast<const void*>(&gs_gate_up_kernel<TY>); }
template <int TY>
const void* gs_dn_fn() { return reinterpret_cast<const void*>(&gs_down_kernel<TY>); }
const void* gs_pick_dec(int t, bool gate_up) {
    switch (t) {
        case 8: return gate_up ? gs_gu_fn<8>() : gs_dn_fn<8>();
        case 12: return gate_up ? gs_gu_fn<12>() : gs_dn_fn<12>();
        case 13: return gate_up ? gs_gu_fn<13>() : gs_dn_fn<13>();
        case 14: return gate_up ? gs_gu_fn<14>() : gs_dn_fn<14>();
    }
    return nullptr;
}

const void* gs_pick(int t) {
    switch (t) {
        case 8: return reinterpret_cast<const void*>(&gs_matvec_kernel<8>);
        case 12: return reinterpret_cast<const void*>(&gs_matvec_kernel<12>);
        case 13: return reinterpret_cast<const void*>(&gs_matvec_kernel<13>);
        case 14: return reinterpret_cast<const void*>(&gs_matvec_kernel<14>);
    }
    return nullptr;
}

uint32_t gs_sb(int t) { return t == 8 ? 34u : t == 12 ? 144u : t == 13 ? 176u : 210u; }
uint32_t gs_spb(int t) { return t == 8 ? 1u : 8u; }

// LDS bytes of a staged range of `rows` rows of C sub-blocks (any alignment of the first
// row): the super-blocks they can touch, plus the 16-byte alignment slack.
size_t gs_raw_bytes(int t, int rows, int C) {
    const uint32_t spb = gs_spb(t);
    const uint32_t nsb = ((uint32_t)rows * C + spb - 1) / spb + 1;
    return ((size_t)nsb * gs_sb(t) + 15 + 15) / 16 * 16;
}

}  // namespace

// Whether the sub-block stream matvec covers a matrix: "" if it does.
const char* gs_unsupported(int type, int64_t K) {
    if (!gs_pick(type)) return "unsupported ggml type";
    if (K % 32) return "K must be a multiple of 32";
    if (K > 4096) return "K above 4096";
    return "";
}

int gs_matvec(int type, const uint8_t* w, int64_t w_bytes, const void* x, int x_dtype, int64_t T, int64_t K, void* y,
              int y_dtype, int64_t N, hipStream_t st) {
    GsMvParams p{};
    p.w = w;
    p.w_records = (uint32_t)(w_bytes < 0xFFFFFFF0ll ? w_bytes : 0xFFFFFFF0ll);
    p.x = x;
    p.x_dtype = x_dtype;
    p.y = y;
    p.y_dtype = y_dtype;
    p.N = (int)N;
    p.K = (int)K;
    const int C = (int)(K / 32), GM = C >= 64 ? 1 : 64 / C, cus = num_cus();
    p.rm = GS_RD / GM * GM;
    if (p.rm == 0) p.rm = GM;
    if (p.rm > GS_RD) p.rm = GS_RD;
    while (p.rm > GM && (double)((N + p.rm - 1) / p.rm) * T < 4.0 * cus) p.rm -= GM;
    const size_t xq = (size_t)XQ_BYTES * C, xraw = (size_t)K * (x_dtype == TSA_F32 ? 4 : 2);
    const size_t raw = gs_raw_bytes(type, p.rm, C);
    // about one workgroup per CU (every workgroup stages and quantises the activations once),
    // 4 to 16 waves, as LDS allows
    const double waves = (double)((N + p.rm - 1) / p.rm) * T;
    int nw = (int)((waves + cus - 1) / cus);
    nw = nw < GS_MIN_WAVES ? GS_MIN_WAVES : nw > GS_MAX_WAVES ? GS_MAX_WAVES : nw;
    while (nw > GS_MIN_WAVES && xq + xraw + (size_t)nw * raw > 160 * 1024) --nw;
    const size_t lds = xq + xraw + (size_t)nw * raw;
    TSA_REQUIRE(lds <= 160 * 1024, TSA_ERR_SHAPE, "GGUF matvec: LDS %zu bytes", lds);
    const int64_t xb = T * (int64_t)xraw;
    p.x_records = (uint32_t)(xb < 0xFFFFFFF0ll ? xb : 0xFFFFFFF0ll);
    p.xq_off = 0;
    p.xraw_off = (int)xq;
    p.raw_off = (int)(xq + xraw);
    p.raw_stride = (int)raw;
    const void* fn = gs_pick(type);
    TSA_HIP_CHECK(ensure_dynamic_lds(fn, (int)lds));
    void* args[] = {&p};
    const dim3 grid((unsigned)((N + (int64_t)nw * p.rm - 1) / ((int64_t)nw * p.rm)), (unsigned)T);
    TSA_HIP_CHECK(hipLaunchKernel(fn, grid, dim3(64 * nw), args, lds, st));
    return TSA_OK;
}

namespace {

// Launch shape of a decode launch: rows per wave (a multiple of the lane row group, at most
// rmax; fewer while the grid would hold under `target` waves per CU), waves per workgroup
// (about one workgroup per CU, 4..16, as LDS allows). rm == 0: the shape does not fit.
struct GsShape {
    int rm = 0, nw = 0;
    size_t raw = 0, lds = 0;
};

GsShape gs_shape(int type, int64_t rows, int64_t groups, int C, int rmax, size_t fixed, int areas, int cus,
                 double target) {
    GsShape s;
    const int GM = C >= 64 ? 1 : 64 / C;
    if (GM > rmax) return s;
    int rm = rmax / GM * GM;
    while (rm > GM && (double)((rows + rm - 1) / rm) * groups < target * cus) rm -= GM;
    const size_t raw = gs_raw_bytes(type, rm, C) * (size_t)areas;
    const double waves = (double)((rows + rm - 1) / rm) * groups;
    int nw = (int)((waves + cus - 1) / cus);
    nw = nw < GS_MIN_WAVES ? GS_MIN_WAVES : nw > GS_MAX_WAVES ? GS_MAX_WAVES : nw;
    while (nw > GS_MIN_WAVES && fixed + (size_t)nw * raw > 160 * 1024) --nw;
    if (fixed + (size_t)nw * raw > 160 * 1024) return s;
    s.rm = rm;
    s.nw = nw;
    s.raw = raw;
    s.lds = fixed + (size_t)nw * raw;
    return s;
}

}  // namespace

// Top-k GGUF expert decode on the sub-block stream kernels, with the same workspace layout
// as the super-block kernels (h as bf16 [T k, I], then the routed selection). Returns a
// positive value, having launched nothing, when the call is outside what these kernels
// cover (the caller then takes the super-block kernels).
int gs_decode(const tsa_expert_layout& L, const uint8_t* pool, int64_t n_slots, const int32_t* slots, const float* wts,
              const void* logits, int logits_dtype, int mode, const int32_t* expert_slot, int64_t E, int32_t* idx_out,
              float* w_out, int64_t T, int k, const void* x, int x_dtype, void* y, int y_dtype, uint8_t* ws,
              int64_t ws_bytes, hipStream_t st) {
    const int64_t H = L.hidden, I = L.inter;
    const int es = x_dtype == TSA_F32 ? 4 : 2;
    // One expert per token only: with several, each down wave walks every expert's rows in
    // turn and the super-block kernels (one expert per wave) measured faster (workload 4:
    // 29.6 against 18.7 us); one expert (workload 2): 15.1 against 16.6 us.
    if (k != 1 || L.format != TSA_EXPERT_GGUF || L.gate_type != L.up_type || !gs_pick_dec(L.gate_type, true) ||
        !gs_pick_dec(L.down_type, false) || H % 32 || I % 32 || H > 4096 || I > 4096 || k > FUSED_MAXK ||
        T * k > 65535 || (logits && (T > FUSED_MAXT || E > 256)) || (reinterpret_cast<uintptr_t>(x) & 15) ||
        T * H * es >= ((int64_t)1 << 32) - 16 || T * k * I * 2 >= ((int64_t)1 << 32) - 16)
        return 1;
    const int cus = num_cus();
    const int CA = (int)(H / 32), CB = (int)(I / 32);
    const size_t fixed_a = GS_MISC + (size_t)XQ_BYTES * CA + (size_t)H * es;
    const size_t fixed_b = GS_MISC + (size_t)XQ_BYTES * k * CB + (size_t)k * I * 2;
    // gate_up waves stream rm rows of gate and rm of up: one of each, 12 waves x 240
    // workgroups, measured 14.3 us for workload 2 against 15.6 at two of each (6 x 240);
    // the down launch's 2 rows x 6 waves and 1 x 12 measured the same
    const GsShape sa = gs_shape(L.gate_type, I, T * k, CA, 4, fixed_a, 2, cus, 8.0);
    const GsShape sb = gs_shape(L.down_type, H, T, CB, 8, fixed_b, k, cus, 4.0);
    if (!sa.rm || !sb.rm) return 1;
    const int64_t h_bytes = T * k * I * 2, tab_off = (h_bytes + 255) / 256 * 256;
    TSA_REQUIRE(ws_bytes >= tab_off + T * k * 8, TSA_ERR_WORKSPACE, "workspace too small for the GGUF decode");
    GsDecParams p{};
    p.L = L;
    p.pool = pool;
    p.n_slots = n_slots;
    p.slots = slots;
    p.wts = wts;
    p.logits = logits;
    p.expert_slot = expert_slot;
    p.idx_out = idx_out;
    p.w_out = w_out;
    p.tab_slot = reinterpret_cast<int32_t*>(ws + tab_off);
    p.tab_w = reinterpret_cast<float*>(ws + tab_off + T * k * 4);
    p.logits_dtype = logits_dtype;
    p.route_mode = mode;
    p.E = (int)E;
    p.T = (int)T;
    p.k = k;
    p.h = reinterpret_cast<uint16_t*>(ws);
    // gate_up
    p.x = x;
    p.x_records = (uint32_t)(T * H * es);
    p.x_dtype = x_dtype;
    p.rm = sa.rm;
    p.xq_off = GS_MISC;
    p.xraw_off = GS_MISC + XQ_BYTES * CA;
    p.raw_off = (int)fixed_a;
    p.raw_stride = (int)sa.raw;
    const void* fa = gs_pick_dec(L.gate_type, true);
    TSA_HIP_CHECK(ensure_dynamic_lds(fa, (int)sa.lds));
    void* args_a[] = {&p};
    TSA_HIP_CHECK(hipLaunchKernel(fa, dim3((unsigned)((I + (int64_t)sa.nw * sa.rm - 1) / ((int64_t)sa.nw * sa.rm)), (unsigned)(T * k)),
                                  dim3(64 * sa.nw), args_a, sa.lds, st));
    // down: the selection gate_up made (routed) or the given table
    GsDecParams q = p;
    if (logits) {
        q.logits = nullptr;
        q.slots = p.tab_slot;
        q.wts = p.tab_w;
    }
    q.x = ws;
    q.x_records = (uint32_t)h_bytes;
    q.x_dtype = TSA_BF16;
    q.y = y;
    q.y_dtype = y_dtype;
    q.rm = sb.rm;
    q.xq_off = GS_MISC;
    q.xraw_off = (int)(GS_MISC + (size_t)XQ_BYTES * k * CB);
    q.raw_off = (int)fixed_b;
    q.raw_stride = (int)sb.raw;
    const void* fb = gs_pick_dec(L.down_type, false);
    TSA_HIP_CHECK(ensure_dynamic_lds(fb, (int)sb.lds));
    void* args_b[] = {&q};
    TSA_HIP_CHECK(hipLaunchKernel(fb, dim3((unsigned)((H + (int64_t)sb.nw * sb.rm - 1) / ((int64_t)sb.nw * sb.rm)), (unsigned)T),
                                  dim3(64 * sb.nw), args_b, sb.lds, st));
    return TSA_OK;
}

}  // namespace tsa
