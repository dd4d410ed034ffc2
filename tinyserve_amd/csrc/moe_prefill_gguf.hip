// Batched (prefill) MoE over GGUF experts (Q8_0 / Q4_K / Q5_K / Q6_K slots in checkpoint
// order): grouped expert GEMMs on the bf16 matrix cores, the weights decoded on the fly.
//
// The reference's batched GGUF expert (tinyserve/ggml_forward.py:117-151,
// _fallback_forward) decodes each projection to fp32, casts it to the activations' dtype
// (bf16) and runs F.linear; here the same bf16 weights (decode_unit's bit-exact fp32 values,
// rounded to nearest even) are formed in registers piece by piece from the native blocks
// and never reach HBM.
//
// After group_kernel has sorted the (token, j) assignments expert-major, each resident
// expert's run of sorted rows is cut into tiles of up to 64 rows (by group_kernel too). Two
// launches then cover every (row tile, weight tile) pair, and a combine pass sums:
//   gate_up: h[i, n] = act(x[token(i)] . W_g[n], x[token(i)] . W_u[n]), bf16, sorted order;
//   down:    yk[a, n] = h[i] . W_d[n], bf16, by assignment a = perm[i];
//   combine: y[t] = sum_j w[t, j] yk[t k + j] in j order (one writer per output).
//
// Workgroup: 8 waves, a tile of 64 sorted rows x 128 weight rows (gate_up: 64 gate rows and
// the same 64 up rows, so the activation is formed in the workgroup). Wave (wr, kh) owns
// weight rows 32 wr .. + 31 and half the K values of every step: each lane decodes the values
// of its row that it feeds v_mfma_f32_32x32x16_bf16 as the A operand straight into registers
// (no row is decoded twice, no weight tile goes through LDS), the activations are the B
// operand from LDS, and the two halves' sums meet in LDS after the last step. The raw blocks
// (a 16-byte-aligned window per row) and the activations come in by buffer-to-LDS copies.
//
// gf_step_kernel (K-quants, K a multiple of 256): K in steps of 128 values, half a
// super-block of each row; a step's activations and the rows' half windows (the header and
// the codes that half reads) come in one step ahead into one of two tiles and areas, 77 KB
// of LDS at most, so two workgroups share a CU.
//
// gf_gemm_kernel (Q8_0, and K-quant rows that straddle super-blocks): K in pieces of 256
// values (one super-block of each row, or 8 Q8_0 blocks), up to 154 KB of LDS, one workgroup
// per CU: the activations into one of two tiles as the previous piece starts, the raw blocks
// into a ring of areas ahead of their piece. Where K is not a multiple of 256 (hidden 2880),
// a K-quant row starts inside a super-block (GGUF stores a matrix as one run of blocks) and a
// piece of it covers the end of one super-block and the start of the next: that variant keeps
// each row's super-blocks in a ring of areas, one new super-block per piece, and decodes
// every 32-value unit from whichever super-block holds it; the last piece of a row is
// partial, its units past K zeroed.
//
// Semantics: tinyserve/expert_pipeline.py:166-239 (group by expert, batched forward,
// weighted scatter), tinyserve/ggml_forward.py:117-151 (bf16 weights, F.linear,
// act_fn(gate) * up), tinyserve/gguf_dequant_torch.py:118-249 (block formats).
#include "fused_common.h"
#include "mfma_tile.h"

namespace tsa {

int launch_group_kernel(const int32_t* idx, int64_t n, int E, int32_t* counts, int32_t* offsets, int32_t* perm,
                        hipStream_t stream, const int32_t* expert_slot = nullptr, int64_t n_slots = 0,
                        int tile_rows = 0, int* n_entries = nullptr, void* table = nullptr);
int pf_combine(const uint16_t* yk, const int32_t* idx, const float* w, const int32_t* expert_slot, int64_t E,
               int64_t n_slots, int64_t T, int k, int H, void* y, int y_dtype, hipStream_t stream);

namespace {

constexpr int GF_THREADS = 512;
constexpr int GF_BM = 64;                  // sorted rows per tile
constexpr int GF_BN = 128;                 // weight rows per tile
constexpr int GF_KP = 256;                 // values per K piece
constexpr int GF_RS = 2 * GF_KP;           // an activation tile row: one piece of a sorted row (bf16), 32 chunks
constexpr int GF_XB = GF_BM * GF_RS;       // one activation tile; two of them
constexpr int GF_ROFF = 2 * GF_XB;         // then the raw areas
constexpr int GF_SS = GF_BN + 4;           // epilogue: fp32 stride of a sorted row's staged sums (per K half)
constexpr int GF_STAGE = 2 * GF_BM * GF_SS * 4;
constexpr int GF_MIN_ASSIGN = 64;          // fewer assignments take the decode kernels

typedef int v4i_t __attribute__((ext_vector_type(4)));
typedef float v16f_t __attribute__((ext_vector_type(16)));

struct GfEntry {
    int slot, row0, rows, pad;
};

// Raw bytes of one row's K piece (a raw group): a K-quant super-block, or 8 Q8_0 blocks.
template <int TY> struct GfType { static constexpr int PB = TY == 8 ? 272 : TY == 12 ? 144 : TY == 13 ? 176 : 210; };
// Alignment of a raw group in LDS, which keeps its global address modulo 16: the K-quant
// 4/5-bit super-blocks (144 / 176 bytes) stay 16-aligned, Q6_K / Q8_0 2-aligned (the host
// requires pool, slot size and offsets to keep that).
template <int TY> constexpr int gf_align() { return TY == 12 || TY == 13 ? 16 : 2; }
// 16-byte chunks of a group's window: from the boundary at or below the group (up to 14
// bytes before it when 2-aligned) to its end, rounded up to an odd count: the 32 rows a
// wave's lanes decode from then sit 4 (mod 8) dwords apart and spread over 16 bank groups
// (an even count halves that or worse: Q6_K's 14 chunks cost its kernel 8% against 15).
template <int TY> constexpr int gf_nch() { return ((GfType<TY>::PB + (gf_align<TY>() == 16 ? 0 : 14) + 15) / 16) | 1; }
// gf_gemm_kernel's raw areas, each the 128 rows' windows of one group. Plain (Q8_0): the
// piece in use and the next (three areas of its windows would not fit beside the activation
// tiles). Straddling (SD): a piece reads two groups of its row, and one or two more areas
// take the groups ahead (Q6_K: one; its windows leave room for three areas only).
template <int TY, bool SD> constexpr int gf_areas() { return SD ? (TY == 14 ? 3 : 4) : 2; }
template <int TY> constexpr int gf_raw() { return GF_BN * gf_nch<TY>() * 16; }
template <int TY, bool SD> constexpr int gf_lds() {
    return GF_ROFF + gf_areas<TY, SD>() * gf_raw<TY>() > GF_STAGE ? GF_ROFF + gf_areas<TY, SD>() * gf_raw<TY>()
                                                                  : GF_STAGE;
}
static_assert(gf_lds<8, false>() <= 160 * 1024 && gf_lds<12, true>() <= 160 * 1024 &&
                  gf_lds<13, true>() <= 160 * 1024 && gf_lds<14, true>() <= 160 * 1024,
              "LDS per workgroup");

struct GfGemm {
    const uint8_t* pool;
    int64_t slot_bytes;
    const int* n_entries;
    const GfEntry* table;
    const uint16_t* src;      // gate_up: x [T, K] (rows through perm / k); down: h [n, K] in sorted order
    int64_t src_bytes;
    const int32_t* perm;      // sorted position -> assignment id (token * k + j)
    int k;
    uint16_t* out;            // gate_up: h [n, N]; down: yk [T k, N]
    int N, K;                 // outputs per row (gate_up: inter; down: hidden), reduction length
    int64_t w_off, w2_off;    // slot offsets of the matrix (gate_up: gate, then up)
    int64_t w_bytes;          // bytes of one matrix (N rows)
    tsa_expert_layout L;
};

// One 1 KB copy: lane l's 16 bytes at buffer offset voff land at LDS byte lds + 16 l (the LDS
// address is the wave's, taken from the first lane).
__device__ __forceinline__ void gf_dma(const v4i_t& r, uint32_t voff, uint32_t lds) {
    asm volatile("s_mov_b32 m0, %2\n\tbuffer_load_dwordx4 %0, %1, 0 offen lds" ::"v"(voff), "s"(r),
                 "s"(__builtin_amdgcn_readfirstlane((int)lds))
                 : "memory", "m0");
}

__device__ __forceinline__ v4i_t gf_desc(const uint8_t* p, int64_t bytes) {
    const uint64_t a = reinterpret_cast<uint64_t>(p);
    const uint32_t n = bytes < 0xFFFFFFF0ll ? (uint32_t)bytes : 0xFFFFFFF0u;
    // words from the first lane: gf_dma's "s" operand must sit in scalar registers
    return v4i_t{__builtin_amdgcn_readfirstlane((int)(uint32_t)a), __builtin_amdgcn_readfirstlane((int)(uint32_t)(a >> 32)),
                 __builtin_amdgcn_readfirstlane((int)n), 0x00020000};
}

// Byte offset in its matrix of raw group q of weight row `row` (K = 32 KU values per row):
// Q8_0, blocks 8 q .. 8 q + 7 of the row; a K-quant, super-block q counted from the one the
// row starts in (the row's first value sits at unit (row KU) % 8 of that super-block).
template <int TY>
__device__ __forceinline__ uint32_t gf_group_byte(int row, int q, int KU) {
    if constexpr (TY == 8) return ((uint32_t)row * (uint32_t)KU + 8u * (uint32_t)q) * 34u;
    else return (((uint32_t)row * (uint32_t)KU >> 3) + (uint32_t)q) * (uint32_t)GfType<TY>::PB;
}

// Raw group q's windows of the tile's 128 weight rows into LDS: pair i = (row i / NCH,
// chunk i % NCH) lands at raw + 16 i, so one wave instruction fills 1 KB. The buffers start
// at the 16-byte boundary at or below each matrix (m0 / m1 bytes before it) and end at the
// boundary at or above its end, and a window starts at the boundary at or below its group,
// so every copy reads 16 whole aligned bytes; rows past the matrix read zero (buffer range).
template <int TY, bool GU>
__device__ __forceinline__ void gf_issue_raw(const v4i_t& r0, const v4i_t& r1, uint32_t m0, uint32_t m1, int n0,
                                             int p, int KU, uint32_t raw, int wave, int lane) {
    constexpr int NCH = gf_nch<TY>(), TOT = GF_BN * NCH;
    for (int ii = wave; 64 * ii < TOT; ii += GF_THREADS / 64) {
        const int q = 64 * ii + lane;
        if (q < TOT) {
            const int r = q / NCH, c = q - r * NCH;
            const bool up = GU && r >= 64;
            const int row = GU ? n0 + (r & 63) : n0 + r;
            const uint32_t m = up ? m1 : m0;
            const uint32_t voff = ((m + gf_group_byte<TY>(row, p, KU)) & ~15u) + 16u * (uint32_t)c;
            if (up) gf_dma(r1, voff, raw + 1024u * (uint32_t)ii);
            else gf_dma(r0, voff, raw + 1024u * (uint32_t)ii);
        }
    }
}

// The 16 values of unit u (32 values) of the block at sb (in LDS) that lane half g feeds
// the A operand with, values 8g .. 8g + 7 and 16 + 8g .. 16 + 8g + 7, as 8 packed bf16 words
// rounded to nearest even from the values decode_unit gives, four codes per dword: the
// 4-bit codes of four values come out of one shift and mask, their fifth (Q5_K) or fifth
// and sixth (Q6_K) bits out of another, and each byte converts to float in one instruction.
// The arithmetic per value is decode_unit's: Q4_K / Q5_K a*q - c (a*q exact, so one
// rounding, fused or not); Q6_K (d*sc) * (q - 32), here as (d*sc/4) times the signed byte
// 4 (q - 32) (q ^ 32 is q - 32 as a 6-bit two's-complement field, and two more bits to the
// left make the byte's sign), exact like the reference's product, signed zeros included.
// HALF: sb is a half window (gf_step_kernel) holding only what units 4h .. 4h + 3 (h = u / 4)
// read, at the offsets gf_half_chunk lays out: Q4_K / Q5_K keep the header (and Q5_K's high
// bits) and take the half's 64 bytes of codes right after; Q6_K's half window is the half's
// low codes (block bytes 64 h ..), high codes (128 + 32 h ..) at +80 and scales and d
// (192 ..) at -64, each from sb.
template <int TY, bool HALF = false>
__device__ __forceinline__ void gf_decode_a(const uint8_t* sb, int u, int g, uint32_t (&o)[8]) {
    if constexpr (TY == 12 || TY == 13) {  // sb is 16-byte aligned
        const u32x4 hdr = *reinterpret_cast<const u32x4*>(sb);
        const uint8_t* qs = sb + (TY == 12 ? 16 : 48) + 32 * (HALF ? (u >> 1) & 1 : u >> 1);
        const uint2 q0 = *reinterpret_cast<const uint2*>(qs + 8 * g), q1 = *reinterpret_cast<const uint2*>(qs + 16 + 8 * g);
        const uint32_t q[4] = {q0.x, q0.y, q1.x, q1.y};
        uint32_t hb[4] = {0u, 0u, 0u, 0u};
        if constexpr (TY == 13) {
            const uint2 h0 = *reinterpret_cast<const uint2*>(sb + 16 + 8 * g), h1 = *reinterpret_cast<const uint2*>(sb + 32 + 8 * g);
            hb[0] = h0.x; hb[1] = h0.y; hb[2] = h1.x; hb[3] = h1.y;
        }
        const float d = f16_bits_to_f32(hdr[0] & 0xFFFFu), dmin = f16_bits_to_f32(hdr[0] >> 16);
        const uint32_t s3[3] = {hdr[1], hdr[2], hdr[3]};
        uint32_t sc, m;
        k_scale_min(s3, u, sc, m);
        const float a = d * (float)sc, c = dmin * (float)m;
        const int sh = (u & 1) * 4;
#pragma unroll
        for (int w = 0; w < 4; ++w) {
            uint32_t qq = (q[w] >> sh) & 0x0F0F0F0Fu;
            if constexpr (TY == 13) qq |= ((hb[w] >> u) & 0x01010101u) << 4;
            o[2 * w] = pack_bf16x2(a * (float)(qq & 0xFFu) - c, a * (float)((qq >> 8) & 0xFFu) - c);
            o[2 * w + 1] = pack_bf16x2(a * (float)((qq >> 16) & 0xFFu) - c, a * (float)(qq >> 24) - c);
        }
    } else if constexpr (TY == 14) {
        // A Q6_K block sits 2 bytes off a dword boundary for half the rows: whole dwords from
        // the boundary below, each pair shifted into place (v_alignbyte_b32).
        const uint32_t ob = (uint32_t)reinterpret_cast<uintptr_t>(sb) & 3u;  // 0 or 2
        const uint32_t* wb = reinterpret_cast<const uint32_t*>(sb - ob);
        auto ld4 = [&](int off, uint32_t (&w)[4]) {  // dwords 2g, 2g + 1, 2g + 4, 2g + 5 of the 32 bytes at sb + off
            const int b0 = (off >> 2) + 2 * g;
            uint32_t t0, t1, t2, t4, t5, t6;  // at most the ninth: inside the block or half window
            if constexpr (HALF) {  // a half window starts at the dword of its block (wb), 16-byte aligned: 8-byte reads
                const uint2* w2 = reinterpret_cast<const uint2*>(wb + b0);
                const uint2 p0 = w2[0], p1 = w2[1], p2 = w2[2], p3 = w2[3];
                t0 = p0.x, t1 = p0.y, t2 = p1.x, t4 = p2.x, t5 = p2.y, t6 = p3.x;
            } else {
                t0 = wb[b0], t1 = wb[b0 + 1], t2 = wb[b0 + 2];
                t4 = wb[b0 + 4], t5 = wb[b0 + 5], t6 = wb[b0 + 6];
            }
            w[0] = __builtin_amdgcn_alignbyte(t1, t0, ob);
            w[1] = __builtin_amdgcn_alignbyte(t2, t1, ob);
            w[2] = __builtin_amdgcn_alignbyte(t5, t4, ob);
            w[3] = __builtin_amdgcn_alignbyte(t6, t5, ob);
        };
        auto ld16 = [&](int off) {  // the 2 bytes at sb + off (off even)
            const uint32_t a = ob + (uint32_t)off;
            return (wb[a >> 2] >> (8u * (a & 3u))) & 0xFFFFu;
        };
        const int hh = u >> 2, t = u & 3;
        uint32_t ql[4], qh[4];
        ld4(HALF ? 32 * (t & 1) : 64 * hh + 32 * (t & 1), ql);
        ld4(HALF ? 80 : 128 + 32 * hh, qh);
        const uint32_t scw = ld16((HALF ? 128 : 192) + 2 * u);
        const float d = f16_bits_to_f32(ld16(HALF ? 144 : 208));
        const float d0 = 0.25f * (d * (float)(int8_t)(scw & 0xFF)), d1 = 0.25f * (d * (float)(int8_t)(scw >> 8));
        const int shl = 4 * (t >> 1), shh = 2 * t;
#pragma unroll
        for (int w = 0; w < 4; ++w) {
            const uint32_t qq = ((ql[w] >> shl) & 0x0F0F0F0Fu) | (((qh[w] >> shh) & 0x03030303u) << 4);
            const uint32_t y = (qq ^ 0x20202020u) << 2;  // four signed bytes 4 (q - 32)
            const float dd = w < 2 ? d0 : d1;            // values below 16 take sc[2u], the rest sc[2u + 1]
            o[2 * w] = pack_bf16x2(dd * (float)(int8_t)(y & 0xFFu), dd * (float)(int8_t)((y >> 8) & 0xFFu));
            o[2 * w + 1] = pack_bf16x2(dd * (float)(int8_t)((y >> 16) & 0xFFu), dd * (float)(int8_t)(y >> 24));
        }
    } else {  // Q8_0: unit u is block u of the piece (34 bytes, 2-byte aligned)
        float v[32];
        decode_unit<8, 2>(sb + 34 * u, 0, v);
#pragma unroll
        for (int i = 0; i < 4; ++i) {  // constant indices and a select (a variable index would go through scratch)
            o[i] = g ? pack_bf16x2(v[8 + 2 * i], v[9 + 2 * i]) : pack_bf16x2(v[2 * i], v[2 * i + 1]);
            o[4 + i] = g ? pack_bf16x2(v[24 + 2 * i], v[25 + 2 * i]) : pack_bf16x2(v[16 + 2 * i], v[17 + 2 * i]);
        }
    }
}

// The epilogue of a tile: acc[t][4u + r] = tile row 32 wr + 8u + 4g + r, sorted row 32 t + rr,
// over K half kh (wave (wr, kh), lane (g, rr)). Both halves' sums into LDS (nothing may be in
// flight and every wave is here), stage[kh][sorted row][tile row], then each output adds its
// two halves: gate_up h = act(gate, up) rounded once to bf16 in sorted order, down one bf16
// row per assignment.
template <bool GU>
__device__ __forceinline__ void gf_store_tile(const GfGemm& p, const GfEntry& en, int n0, const v16f_t (&acc)[2],
                                              uint8_t* smem) {
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wr = wave & 3, kh = wave >> 2, g = lane >> 5, rr = lane & 31;
    const int N = p.N;
    __syncthreads();
    float* stage = reinterpret_cast<float*>(smem);
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
        for (int u = 0; u < 4; ++u)
            *reinterpret_cast<float4*>(stage + (kh * GF_BM + 32 * t + rr) * GF_SS + 32 * wr + 8 * u + 4 * g) =
                make_float4(acc[t][4 * u], acc[t][4 * u + 1], acc[t][4 * u + 2], acc[t][4 * u + 3]);
    __syncthreads();
    if constexpr (GU) {
        // h = act(gate, up) rounded once to bf16, 8 columns per thread (the sigmoid from
        // v_exp_f32 and v_rcp_f32: 64 values per thread and tile, far below the bf16 rounding)
        const int hr = tid >> 3, hc = 8 * (tid & 7);
        if (hr < en.rows && n0 + hc < N) {
            // 16-byte reads: the 16 lanes of a read (two rows 132 floats apart, eight column
            // groups) then cover the 64 banks once; single floats put four lanes on a bank
            const float4* s0 = reinterpret_cast<const float4*>(stage + hr * GF_SS + hc);
            const float4* s1 = reinterpret_cast<const float4*>(stage + (GF_BM + hr) * GF_SS + hc);
            float g8[8], u8[8];
#pragma unroll
            for (int i = 0; i < 2; ++i) {
                const float4 a = s0[i], b = s1[i], c = s0[16 + i], d = s1[16 + i];  // +16 float4: the up rows
                g8[4 * i] = a.x + b.x, g8[4 * i + 1] = a.y + b.y, g8[4 * i + 2] = a.z + b.z, g8[4 * i + 3] = a.w + b.w;
                u8[4 * i] = c.x + d.x, u8[4 * i + 1] = c.y + d.y, u8[4 * i + 2] = c.z + d.z, u8[4 * i + 3] = c.w + d.w;
            }
            float h[8];
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                const float gv = g8[i], uv = u8[i];
                h[i] = p.L.act == TSA_ACT_SWIGLU_OAI ? swiglu_oai_fast(p.L, gv, uv) : silu_mul_fast(gv, uv);
            }
            *reinterpret_cast<uint4*>(p.out + (int64_t)(en.row0 + hr) * N + n0 + hc) =
                make_uint4(pack_bf16x2(h[0], h[1]), pack_bf16x2(h[2], h[3]), pack_bf16x2(h[4], h[5]),
                           pack_bf16x2(h[6], h[7]));
        }
    } else {
        // 16 output rows per thread, bf16 per assignment
        const int hr = tid >> 3, hc = 16 * (tid & 7);
        if (hr < en.rows && n0 + hc < N) {  // N % 16 == 0
            const int64_t a = p.perm[en.row0 + hr];
            const float4* s0 = reinterpret_cast<const float4*>(stage + hr * GF_SS + hc);  // 16-byte reads, as above
            const float4* s1 = reinterpret_cast<const float4*>(stage + (GF_BM + hr) * GF_SS + hc);
            uint32_t o[8];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const float4 x = s0[i], y = s1[i];
                o[2 * i] = pack_bf16x2(x.x + y.x, x.y + y.y);
                o[2 * i + 1] = pack_bf16x2(x.z + y.z, x.w + y.w);
            }
            uint4* dst = reinterpret_cast<uint4*>(p.out + a * N + n0 + hc);
            dst[0] = make_uint4(o[0], o[1], o[2], o[3]);
            dst[1] = make_uint4(o[4], o[5], o[6], o[7]);
        }
    }
}

template <int TY, bool GU, bool SD>
__global__ void __launch_bounds__(GF_THREADS, 1) gf_gemm_kernel(GfGemm p) {
    extern __shared__ __align__(16) uint8_t smem[];
    // Work id w = (entry, column tile) of this workgroup. Workgroups are dealt round the 8
    // XCDs by linear id, so the ids are renumbered to give each XCD a run of consecutive
    // work: the column tiles of an entry (which gather the same activation rows) and the
    // tiles of an expert's consecutive entries (the same weight rows) then share one L2.
    const int tiles = (int)gridDim.x, nact = *p.n_entries * tiles;
    const int lin = (int)(blockIdx.y * gridDim.x + blockIdx.x);
    if (lin >= nact) return;  // workgroup-uniform
    const int xcd = lin & 7, q8 = nact >> 3, rem = nact & 7;
    const int wid = xcd * q8 + (xcd < rem ? xcd : rem) + (lin >> 3);  // a bijection of [0, nact)
    const int en_i = wid / tiles, tile = wid - en_i * tiles;
    const GfEntry en = p.table[en_i];
    const int tid = threadIdx.x, lane = tid & 63, wave = uniform(tid >> 6);
    const int wr = wave & 3, kh = wave >> 2, g = lane >> 5, rr = lane & 31;
    const int K = p.K, KU = K / 32, P = (KU + 7) / 8;
    const int n0 = tile * (GU ? GF_BN / 2 : GF_BN);  // first output column of the tile
    const uint8_t* base = p.pool + (int64_t)en.slot * p.slot_bytes;
    const uint8_t* mat0 = base + p.w_off;
    const uint8_t* mat1 = base + (GU ? p.w2_off : p.w_off);
    const uint32_t mis0 = (uint32_t)reinterpret_cast<uintptr_t>(mat0) & 15u;
    const uint32_t mis1 = (uint32_t)reinterpret_cast<uintptr_t>(mat1) & 15u;
    const v4i_t rs0 = gf_desc(mat0 - mis0, (p.w_bytes + mis0 + 15) & ~15ll),
                rs1 = gf_desc(mat1 - mis1, (p.w_bytes + mis1 + 15) & ~15ll);
    const uint32_t lds0 = (uint32_t)reinterpret_cast<uintptr_t>(smem);
    const uint32_t raw = lds0 + GF_ROFF;
    constexpr int RA = gf_areas<TY, SD>(), RAW = gf_raw<TY>();
    // raw groups per row (a straddling piece also reads the next group) and how many of the
    // newest may still fly when a piece starts
    const int NG = SD ? P + 1 : P;
    constexpr int OUT = RA - 2 - (SD ? 1 : 0);
    static_assert(OUT == 0 || OUT == 1, "raw groups in flight at a piece's start");

    // Activation tiles: row r holds sorted row r's piece as 32 chunks of 16 bytes, chunk c in
    // slot c ^ (r % 32), so the 32 rows of an MFMA operand read fall on distinct banks. They
    // arrive by buffer-to-LDS copies: wave w's copy i fills rows 8w + 2i and 8w + 2i + 1 (1 KB,
    // lane l: row 8w + 2i + l / 32, slot l % 32, so it reads chunk (l % 32) ^ row % 32).
    // Rows past the tile's read zeros (an offset past the buffer's end).
    // Columns past K (the last piece of a row when K % 256 != 0) read zeros as well. Only the
    // straddling variants and Q8_0 can have such a piece (a plain K-quant kernel has K % 256 == 0).
    constexpr bool TAILS = SD || TY == 8;
    const v4i_t rx = gf_desc(reinterpret_cast<const uint8_t*>(p.src), p.src_bytes);
    uint32_t xo[4];
    int xc[4];  // the first column of this lane's chunk in piece 0
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int r = 8 * wave + 2 * i + (lane >> 5);
        xo[i] = 0x80000000u;
        xc[i] = 8 * ((lane & 31) ^ (r & 31));
        if (r < en.rows) {
            const int a = p.perm[en.row0 + r];
            const int64_t xrow = GU ? (int64_t)(a / p.k) : (int64_t)(en.row0 + r);
            xo[i] = (uint32_t)(xrow * K * 2) + 2u * (uint32_t)xc[i];
        }
    }
    auto issue_x = [&](int pc) {
        const uint32_t t = lds0 + (uint32_t)(pc & 1) * GF_XB + (uint32_t)(8 * wave) * GF_RS;
        const bool tail = TAILS && (K & (GF_KP - 1)) && pc == P - 1;  // wave-uniform
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const uint32_t o = tail && GF_KP * pc + xc[i] >= K ? 0x80000000u : xo[i] + (uint32_t)pc * (2 * GF_KP);
            gf_dma(rx, o, t + (uint32_t)(2 * i) * GF_RS);
        }
    };
    // this wave's raw copies per piece: instructions ii = wave, wave + 8, .. below NI
    constexpr int NI = (GF_BN * gf_nch<TY>() + 63) / 64, RWA = (NI + 7) / 8, RWB = NI / 8;
    const bool rw_more = wave < NI % 8;

    // This lane's weight row: tile row 32 wr + rr (gate_up: rows 64.. are the up rows).
    const int trow = 32 * wr + rr;
    const int drow = GU ? n0 + (trow & 63) : n0 + trow;
    constexpr int NCH = gf_nch<TY>();
    const uint32_t dmis = GU && trow >= 64 ? mis1 : mis0;
    const int ph = SD ? (int)(((uint32_t)drow * (uint32_t)KU) & 7u) : 0;  // the row's first unit in its super-block

    v16f_t acc[2];
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
        for (int i = 0; i < 16; ++i) acc[t][i] = 0.0f;

    // Piece pc's activations sit in tile pc % 2 and raw group q in area q % RA. As piece pc
    // starts, the copies of piece pc + 1's activations and then of group pc + RA - 1 go out
    // (into the area group pc - 1 left), so a group flies for RA - 2 pieces (plain) or
    // RA - 3 (straddling: piece pc reads groups pc and pc + 1). A tile or area is rewritten
    // one piece after it was last read, with the barrier of the piece between. Every load
    // here is an inline-assembly copy (the compiler counts none of them), so the waits are
    // explicit: at the top of piece pc everything must have landed but the newest OUT groups
    // (the RWA or RWB instructions per group of this wave).
    issue_x(0);
    for (int q = 0; q < RA - 1 && q < NG; ++q)
        gf_issue_raw<TY, GU>(rs0, rs1, mis0, mis1, n0, q, KU, raw + (uint32_t)q * RAW, wave, lane);
    for (int pc = 0; pc < P; ++pc) {
        const uint8_t* xt = smem + (pc & 1) * GF_XB;
        if (OUT == 1 && pc + RA - 2 < NG) {
            if (rw_more) asm volatile("s_waitcnt vmcnt(%0)" ::"n"(RWA) : "memory");
            else asm volatile("s_waitcnt vmcnt(%0)" ::"n"(RWB) : "memory");
        } else {
            asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        }
        __syncthreads();  // piece pc's raw groups and activations are in LDS; tile (pc + 1) % 2 and area (pc - 1) % RA are free
        if (pc + 1 < P) issue_x(pc + 1);
        if (pc + RA - 1 < NG)
            gf_issue_raw<TY, GU>(rs0, rs1, mis0, mis1, n0, pc + RA - 1, KU, raw + (uint32_t)((pc + RA - 1) % RA) * RAW,
                                 wave, lane);
        // unit uu of the half, then its two K steps (the next unit's decode can issue while
        // these MFMAs run); step j: K 16 j .. + 15 of the half, lane half g holds K 16 j + 8 g .. + 7
        const uint8_t* xr0 = xt + rr * GF_RS;  // sorted row rr (t = 0) and 32 + rr (t = 1): same swizzle
        // this lane's window of group pc (and, straddling, of group pc + 1)
        const uint8_t* sb0 = smem + GF_ROFF + (pc % RA) * RAW + 16 * NCH * trow +
                             ((dmis + gf_group_byte<TY>(drow, pc, KU)) & 15u);
        const uint8_t* sb1 = SD ? smem + GF_ROFF + ((pc + 1) % RA) * RAW + 16 * NCH * trow +
                                      ((dmis + gf_group_byte<TY>(drow, pc + 1, KU)) & 15u)
                                : sb0;
        const bool tail = TAILS && (KU & 7) && pc == P - 1;  // wave-uniform: the row's last, partial piece
#pragma unroll
        for (int uu = 0; uu < 4; ++uu) {
            const int j = 4 * kh + uu;  // unit of the piece
            const int v = ph + j;       // straddling: unit v % 8 of group pc + v / 8
            uint32_t av[8];
            gf_decode_a<TY>(SD && v >= 8 ? sb1 : sb0, SD ? v & 7 : j, g, av);
            if (tail && 8 * pc + j >= KU) {  // past the row's end: another row's values or zeros
#pragma unroll
                for (int i = 0; i < 8; ++i) av[i] = 0u;
            }
#pragma unroll
            for (int s2 = 0; s2 < 2; ++s2) {
                const int j2 = 2 * uu + s2;
                const bf16x8 A = __builtin_bit_cast(bf16x8, u32x4{av[4 * s2], av[4 * s2 + 1], av[4 * s2 + 2], av[4 * s2 + 3]});
#pragma unroll
                for (int t = 0; t < 2; ++t) {
                    const int c = (16 * kh + 2 * j2 + g) ^ rr;  // chunk of K 128 kh + 16 j2 + 8 g
                    const bf16x8 B = *reinterpret_cast<const bf16x8*>(xr0 + 32 * t * GF_RS + 16 * c);
                    acc[t] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(A, B, acc[t], 0, 0, 0);
                }
            }
        }
    }

    gf_store_tile<GU>(p, en, n0, acc, smem);
}

// ---- gf_step_kernel: the plain K-quant matrices (K % 256 == 0), K in steps of 128 values

constexpr int GF_KS = 128;               // values per step: half a super-block of each row
constexpr int GF_SRS = 2 * GF_KS;        // a step's activation row: 256 bytes, 16 chunks
constexpr int GF_SXB = GF_BM * GF_SRS;   // one step activation tile; two of them
constexpr int GF_SROFF = 2 * GF_SXB;     // then two raw areas

// 16-byte chunks of a row's half window (odd, as gf_nch): Q4_K header + 4 of codes; Q5_K
// header, high bits + 4 of codes; Q6_K 5 of low codes, 3 of high codes, 2 of scales and d
// (+1 unused). A Q6_K window's chunks are counted from the dword at or below its block (0
// or 2 bytes before it: the copies read 16 bytes at dword-aligned offsets), so the block
// sits 0 or 2 bytes into a 16-byte-aligned window and its decode reads aligned 8-byte pairs
// (on distinct banks for the 16 rows of a read, where single dwords 44 apart pair up rows r
// and r + 16).
template <int TY> constexpr int gf_half_nch() { return TY == 12 ? 5 : TY == 13 ? 7 : 11; }
template <int TY> constexpr int gf_half_raw() { return GF_BN * gf_half_nch<TY>() * 16; }
template <int TY> constexpr int gf_step_lds() {
    return GF_SROFF + 2 * gf_half_raw<TY>() > GF_STAGE ? GF_SROFF + 2 * gf_half_raw<TY>() : GF_STAGE;
}
static_assert(gf_step_lds<12>() <= 80 * 1024 && gf_step_lds<13>() <= 80 * 1024 && gf_step_lds<14>() <= 80 * 1024,
              "two workgroups per CU");

// Source chunk of half window slot c in half h, counted from the window's base (Q4_K 9
// chunks, Q5_K 11; a Q6_K block covers chunks 0 .. 13).
template <int TY> __device__ __forceinline__ int gf_half_chunk(int c, int h) {
    if constexpr (TY == 12) return c == 0 ? 0 : c + 4 * h;
    else if constexpr (TY == 13) return c < 3 ? c : c + 4 * h;
    else return c < 5 ? 4 * h + c : c < 8 ? 3 + 2 * h + c : c < 10 ? 4 + c : 13;
}

// The same tile as gf_gemm_kernel (64 sorted rows x 128 weight rows, wave (wr, kh) decoding
// the A operands of its 32 rows), with K in steps of 128 values: a step's activations (16 KB)
// and the half windows of its 128 rows' super-blocks come in one step ahead into one of two
// tiles and areas, so a workgroup holds at most 77 KB of LDS and two share a CU (what one
// workgroup's barrier, copy waits, prologue and epilogue leave idle, the other fills). Step s
// is half s % 2 of piece s / 2; wave kh decodes units 4 h + 2 kh and 4 h + 2 kh + 1 of it, and
// the steps of a piece are unrolled and the two kh branches written out, so every unit index
// and shift is a constant and the LDS addresses of the B operands and windows are fixed per lane.
template <int TY, bool GU>
__global__ void __launch_bounds__(GF_THREADS, 2) gf_step_kernel(GfGemm p) {
    extern __shared__ __align__(16) uint8_t smem[];
    const int tiles = (int)gridDim.x, nact = *p.n_entries * tiles;
    const int lin = (int)(blockIdx.y * gridDim.x + blockIdx.x);
    if (lin >= nact) return;  // workgroup-uniform
    const int xcd = lin & 7, q8 = nact >> 3, rem = nact & 7;
    const int wid = xcd * q8 + (xcd < rem ? xcd : rem) + (lin >> 3);  // as gf_gemm_kernel
    const int en_i = wid / tiles, tile = wid - en_i * tiles;
    const GfEntry en = p.table[en_i];
    const int tid = threadIdx.x, lane = tid & 63, wave = uniform(tid >> 6);
    const int wr = wave & 3, kh = wave >> 2, g = lane >> 5, rr = lane & 31;
    const int K = p.K, KU = K / 32, P = K / GF_KP;
    const int n0 = tile * (GU ? GF_BN / 2 : GF_BN);
    const uint8_t* base = p.pool + (int64_t)en.slot * p.slot_bytes;
    const uint8_t* mat0 = base + p.w_off;
    const uint8_t* mat1 = base + (GU ? p.w2_off : p.w_off);
    const uint32_t mis0 = (uint32_t)reinterpret_cast<uintptr_t>(mat0) & 15u;
    const uint32_t mis1 = (uint32_t)reinterpret_cast<uintptr_t>(mat1) & 15u;
    const v4i_t rs0 = gf_desc(mat0 - mis0, (p.w_bytes + mis0 + 15) & ~15ll),
                rs1 = gf_desc(mat1 - mis1, (p.w_bytes + mis1 + 15) & ~15ll);
    const uint32_t lds0 = (uint32_t)reinterpret_cast<uintptr_t>(smem);
    constexpr int RAW = gf_half_raw<TY>(), NCH = gf_half_nch<TY>(), PB = GfType<TY>::PB;
    constexpr uint32_t WA = TY == 14 ? 3u : 15u;  // a window's base: the dword (Q6_K) or 16 bytes at or below the block
    // a step's raw copies: 128 NCH chunks = 2 NCH wave instructions (ii = wave, wave + 8, ..)
    constexpr int RI = (2 * NCH + 7) / 8;

    // Activation tiles: row r holds sorted row r's step as 16 chunks, chunk c in slot c ^ (r % 16);
    // wave w's copy i fills rows 8w + 4i .. 8w + 4i + 3 (lane l: row 8w + 4i + l / 16, slot l % 16).
    // Rows past the tile read zeros (an offset past the buffer's end).
    const v4i_t rx = gf_desc(reinterpret_cast<const uint8_t*>(p.src), p.src_bytes);
    uint32_t xo[2];
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        const int r = 8 * wave + 4 * i + (lane >> 4);
        xo[i] = 0x80000000u;
        if (r < en.rows) {
            const int a = p.perm[en.row0 + r];
            const int64_t xrow = GU ? (int64_t)(a / p.k) : (int64_t)(en.row0 + r);
            xo[i] = (uint32_t)(xrow * K * 2) + 16u * (uint32_t)((lane & 15) ^ (r & 15));
        }
    }
    // Raw areas: pair q = (row q / NCH, slot q % NCH) of the 128 rows' half windows at 16 q.
    // Per copy instruction i of this wave: its lane's row's first super-block (byte offset from
    // the buffer base, the matrix's misalignment included) and its chunk in half 0 and half 1.
    // 128 NCH is a multiple of 64, so every instruction is whole, and its rows are all gate or
    // all up rows (ii < NCH: rows 0 .. 63).
    uint32_t rg[RI], rc0[RI], rc1[RI];
#pragma unroll
    for (int i = 0; i < RI; ++i) {
        const int q = 64 * (wave + 8 * i) + lane, r = q / NCH, c = q - r * NCH;
        const int row = GU ? n0 + (r & 63) : n0 + r;
        rg[i] = (GU && r >= 64 ? mis1 : mis0) + gf_group_byte<TY>(row, 0, KU);
        rc0[i] = 16u * (uint32_t)gf_half_chunk<TY>(c, 0);
        rc1[i] = 16u * (uint32_t)gf_half_chunk<TY>(c, 1);
    }
    auto issue = [&](int s) {  // step s's activations and half windows, into tile and area s % 2
        const int pc = s >> 1, h = s & 1;
        const uint32_t t = lds0 + (uint32_t)h * GF_SXB + (uint32_t)(8 * wave) * GF_SRS;
#pragma unroll
        for (int i = 0; i < 2; ++i) gf_dma(rx, xo[i] + (uint32_t)s * (2 * GF_KS), t + (uint32_t)(4 * i) * GF_SRS);
        const uint32_t ra = lds0 + GF_SROFF + (uint32_t)h * RAW;
#pragma unroll
        for (int i = 0; i < RI; ++i) {
            const int ii = wave + 8 * i;
            if (ii < 2 * NCH) {  // wave-uniform
                const uint32_t voff = ((rg[i] + (uint32_t)pc * PB) & ~WA) + (h ? rc1[i] : rc0[i]);
                gf_dma(GU && ii >= NCH ? rs1 : rs0, voff, ra + 1024u * (uint32_t)ii);
            }
        }
    };

    // this lane's weight row (tile row 32 wr + rr) and its half window; the B operands: K steps
    // j2 = 4 kh + j (j = 0 .. 3) of a step, lane half g reading chunk 2 j2 + g of sorted row rr
    const int trow = 32 * wr + rr;
    const int drow = GU ? n0 + (trow & 63) : n0 + trow;
    const uint32_t dg = (GU && trow >= 64 ? mis1 : mis0) + gf_group_byte<TY>(drow, 0, KU);
    const uint8_t* win = smem + GF_SROFF + 16 * NCH * trow;
    const uint8_t* xa[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) xa[j] = smem + rr * GF_SRS + 16 * ((2 * (4 * kh + j) + g) ^ (rr & 15));

    v16f_t acc[2];
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
        for (int i = 0; i < 16; ++i) acc[t][i] = 0.0f;

    // units 4 h + 2 khc + uu of the step in tile / area h: each decoded straight into the A
    // operands of its two K steps, each times sorted rows 0 .. 31 and 32 .. 63
    auto units = [&](const uint8_t* sb, int h, int khc) {
#pragma unroll
        for (int uu = 0; uu < 2; ++uu) {
            uint32_t av[8];
            gf_decode_a<TY, true>(sb, 4 * h + 2 * khc + uu, g, av);
#pragma unroll
            for (int s2 = 0; s2 < 2; ++s2) {
                const bf16x8 A = __builtin_bit_cast(bf16x8, u32x4{av[4 * s2], av[4 * s2 + 1], av[4 * s2 + 2], av[4 * s2 + 3]});
#pragma unroll
                for (int t = 0; t < 2; ++t) {
                    const bf16x8 B = *reinterpret_cast<const bf16x8*>(xa[2 * uu + s2] + h * GF_SXB + 32 * t * GF_SRS);
                    acc[t] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(A, B, acc[t], 0, 0, 0);
                }
            }
        }
    };

    // Step s waits for everything this wave copied (step s's data: nothing newer flies), then
    // the barrier: every wave's copies of step s have landed and tile / area (s + 1) % 2, last
    // read in step s - 1, is free for step s + 1's copies.
    issue(0);
    for (int pc = 0; pc < P; ++pc) {
        const uint8_t* sbp = win + ((dg + (uint32_t)pc * PB) & WA);  // the block's place in its window
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
            __syncthreads();
            if (h == 0 || pc + 1 < P) issue(2 * pc + h + 1);
            if (kh == 0) units(sbp + h * RAW, h, 0);
            else units(sbp + h * RAW, h, 1);
        }
    }
    gf_store_tile<GU>(p, en, n0, acc, smem);
}

template <int TY, bool GU, bool SD>
const void* gf_fn() { return reinterpret_cast<const void*>(&gf_gemm_kernel<TY, GU, SD>); }

// gf_gemm_kernel runs Q8_0 (plain) and the K-quants' straddling rows
const void* gf_pick(int t, bool gu) {
    switch (t) {
        case 8: return gu ? gf_fn<8, true, false>() : gf_fn<8, false, false>();
        case 12: return gu ? gf_fn<12, true, true>() : gf_fn<12, false, true>();
        case 13: return gu ? gf_fn<13, true, true>() : gf_fn<13, false, true>();
        case 14: return gu ? gf_fn<14, true, true>() : gf_fn<14, false, true>();
    }
    return nullptr;
}

template <int TY, bool GU>
const void* gf_step_fn() { return reinterpret_cast<const void*>(&gf_step_kernel<TY, GU>); }

const void* gf_step_pick(int t, bool gu) {
    switch (t) {
        case 12: return gu ? gf_step_fn<12, true>() : gf_step_fn<12, false>();
        case 13: return gu ? gf_step_fn<13, true>() : gf_step_fn<13, false>();
        case 14: return gu ? gf_step_fn<14, true>() : gf_step_fn<14, false>();
    }
    return nullptr;
}

int gf_step_lds_of(int t) { return t == 12 ? gf_step_lds<12>() : t == 13 ? gf_step_lds<13>() : gf_step_lds<14>(); }

int gf_lds_of(int t) {
    return t == 8 ? gf_lds<8, false>() : t == 12 ? gf_lds<12, true>() : t == 13 ? gf_lds<13, true>() : gf_lds<14, true>();
}

int64_t gf_al256(int64_t v) { return (v + 255) / 256 * 256; }

struct GfWs {
    int64_t counts, offsets, perm, nent, table, h, yk, total;
};

GfWs gf_ws_layout(const tsa_expert_layout& L, int64_t T, int k, int64_t E) {
    const int64_t n = T * k;
    GfWs w;
    int64_t o = 0;
    w.counts = o; o += gf_al256(4 * E);
    w.offsets = o; o += gf_al256(4 * (E + 1));
    w.perm = o; o += gf_al256(4 * n);
    w.nent = o; o += 256;
    w.table = o; o += gf_al256((int64_t)sizeof(GfEntry) * (n / GF_BM + E + 1));
    w.h = o; o += gf_al256(2 * n * L.inter);
    w.yk = o; o += gf_al256(2 * n * L.hidden);
    w.total = o;
    return w;
}

bool gf_type_ok(int t, int64_t slot_bytes, int64_t off) {
    if (t != 8 && t != 12 && t != 13 && t != 14) return false;
    const int a = (t == 12 || t == 13) ? 16 : 2;
    return slot_bytes % a == 0 && off % a == 0;
}

}  // namespace

// Whether the grouped GGUF GEMMs cover a prefill call (else the decode kernels run over
// token chunks): GGUF slots whose gate and up share a type, hidden and inter multiples of
// 32 (K-quant rows may start inside a super-block), bf16 activations, block alignment kept
// by the slot size and offsets, and at least GF_MIN_ASSIGN assignments.
bool gf_supported(const tsa_expert_layout& L, int x_dtype, int64_t T, int k) {
    const int64_t n = T * k;
    return L.format == TSA_EXPERT_GGUF && L.gate_type == L.up_type && x_dtype == TSA_BF16 && L.hidden % 32 == 0 &&
           L.inter % 32 == 0 && L.gate_bias_off < 0 && L.down_bias_off < 0 && n >= GF_MIN_ASSIGN &&
           n / GF_BM + 1024 < 65535 && 2 * n * L.inter < ((int64_t)1 << 31) &&
           2 * n * L.hidden < ((int64_t)1 << 31) && gf_type_ok(L.gate_type, L.slot_bytes, L.gate_off) &&
           gf_type_ok(L.up_type, L.slot_bytes, L.up_off) && gf_type_ok(L.down_type, L.slot_bytes, L.down_off);
}

int64_t gf_workspace_bytes(const tsa_expert_layout& L, int64_t T, int k, int64_t E) {
    return gf_ws_layout(L, T, k, E).total;
}

int gf_prefill(const tsa_expert_layout& L, const uint8_t* pool, int64_t n_slots, const int32_t* expert_slot, int64_t E,
               const int32_t* idx, const float* weights, int64_t T, int k, const uint16_t* x, void* y, int y_dtype,
               uint8_t* ws, hipStream_t stream) {
    TSA_REQUIRE((reinterpret_cast<uintptr_t>(pool) & 15u) == 0 && (reinterpret_cast<uintptr_t>(x) & 15u) == 0,
                TSA_ERR_INVALID_ARG, "GGUF grouped prefill: pool and x must be 16-byte aligned");
    const GfWs w = gf_ws_layout(L, T, k, E);
    int32_t* counts = reinterpret_cast<int32_t*>(ws + w.counts);
    int32_t* offsets = reinterpret_cast<int32_t*>(ws + w.offsets);
    int32_t* perm = reinterpret_cast<int32_t*>(ws + w.perm);
    int* nent = reinterpret_cast<int*>(ws + w.nent);
    GfEntry* table = reinterpret_cast<GfEntry*>(ws + w.table);
    uint16_t* h = reinterpret_cast<uint16_t*>(ws + w.h);
    uint16_t* yk = reinterpret_cast<uint16_t*>(ws + w.yk);
    const int H = (int)L.hidden, I = (int)L.inter;
    const int64_t n = T * k;

    static_assert(sizeof(GfEntry) == 16, "the grouping kernel writes the tile table as int4 entries");
    int rc = launch_group_kernel(idx, n, (int)E, counts, offsets, perm, stream, expert_slot, n_slots, GF_BM, nent, table);
    if (rc) return rc;

    // a K-quant matrix whose K is a multiple of 256 takes gf_step_kernel; one whose K is not,
    // the straddling variant of gf_gemm_kernel; Q8_0 its plain variant
    const bool sd_gu = L.gate_type != 8 && L.hidden % GF_KP != 0, sd_dn = L.down_type != 8 && L.inter % GF_KP != 0;
    const bool st_gu = L.gate_type != 8 && !sd_gu, st_dn = L.down_type != 8 && !sd_dn;
    const void* f_gu = st_gu ? gf_step_pick(L.gate_type, true) : gf_pick(L.gate_type, true);
    const void* f_dn = st_dn ? gf_step_pick(L.down_type, false) : gf_pick(L.down_type, false);
    const int lds_gu = st_gu ? gf_step_lds_of(L.gate_type) : gf_lds_of(L.gate_type),
              lds_dn = st_dn ? gf_step_lds_of(L.down_type) : gf_lds_of(L.down_type);
    for (auto [f, b] : {std::pair<const void*, int>{f_gu, lds_gu}, std::pair<const void*, int>{f_dn, lds_dn}}) {
        const hipError_t e = ensure_dynamic_lds(f, b);
        TSA_REQUIRE(e == hipSuccess, TSA_ERR_HIP, "hipFuncSetAttribute(LDS %d): %s", b, hipGetErrorString(e));
    }
    const unsigned max_entries = (unsigned)(n / GF_BM + (E < n ? E : n) + 1);
    auto mat_bytes = [](int t, int64_t rows, int64_t K) {  // rows K values as one run of blocks
        return t == 8 ? rows * K / 32 * 34 : rows * K / GF_KP * (t == 12 ? 144 : t == 13 ? 176 : 210);
    };

    GfGemm g{};
    g.pool = pool;
    g.slot_bytes = L.slot_bytes;
    g.n_entries = nent;
    g.table = table;
    g.perm = perm;
    g.k = k;
    g.L = L;
    // gate_up: x [T, H] -> h [n, I]
    g.src = x;
    g.src_bytes = T * L.hidden * 2;
    g.out = h;
    g.N = I;
    g.K = H;
    g.w_off = L.gate_off;
    g.w2_off = L.up_off;
    g.w_bytes = mat_bytes(L.gate_type, I, H);
    void* args[] = {&g};
    TSA_HIP_CHECK(hipLaunchKernel(f_gu, dim3((unsigned)((I + GF_BN / 2 - 1) / (GF_BN / 2)), max_entries),
                                  dim3(GF_THREADS), args, lds_gu, stream));
    // down: h [n, I] -> yk [n, H] by assignment id
    g.src = h;
    g.src_bytes = n * L.inter * 2;
    g.out = yk;
    g.N = H;
    g.K = I;
    g.w_off = L.down_off;
    g.w2_off = L.down_off;
    g.w_bytes = mat_bytes(L.down_type, H, I);
    TSA_HIP_CHECK(hipLaunchKernel(f_dn, dim3((unsigned)((H + GF_BN - 1) / GF_BN), max_entries),
                                  dim3(GF_THREADS), args, lds_dn, stream));
    return pf_combine(yk, idx, weights, expert_slot, E, n_slots, T, k, H, y, y_dtype, stream);
}

}  // namespace tsa
