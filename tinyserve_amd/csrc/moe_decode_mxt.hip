// MoE decode over MXFP4 experts stored in the 16-row tile order (mx_tile.hip): routing,
// gate_up, clamped SwiGLU, down and the weighted top-k sum in two launches, each a pure
// weight stream. Every weight byte is read by contiguous 1 KB wave loads and fed to the
// matrix cores as it arrives, still in fp4.
//
// Arithmetic. One 1 KB piece m of a 16-row tile is the fp4 (e2m1) B operand of one
// v_mfma_scale_f32_16x16x128_f8f6f4, as loaded: lane 16q+i holds block 4m+q of row i, which
// is exactly that instruction's fp4 operand layout (column i, K = 32q..32q+31), and byte m%4
// of the lane's scale word m/4 is the e8m0 scale of that block, which the instruction takes
// as the lane's B scale: the block scales are applied by the matrix core. The A operand
// carries the activation vector v (x for gate_up, h for down) as two fp8 e4m3 terms in
// rows 0 and 1 (rows 2..15 zero), so D[r][i] accumulates sum_k W[i][k] term_r(k) over the
// pieces and lane i adds rows 0 and 1 at the end. Every 32-value block b of v has its own
// power-of-two scale s_b = 2^(7 - e_b), e_b the exponent of the block's largest |v|, and the
// terms are v s_b = hi + lo with hi = e4m3(v s_b) and lo = e4m3(v s_b - hi); the A scale of
// block b is 1 / s_b (e8m0), so the matrix core undoes the scaling. For a bf16 v the pair is
// exact (hi keeps 4 significant bits, lo the remaining 4) unless v is more than 2^9 below
// its block's maximum, so the products are those of the reference's bf16 arithmetic whatever
// the magnitude of v and however it varies across blocks.
//
// Launch 1 (gate_up): workgroup (kb, pair) multiplies 32 gate_up rows of the pair's expert
//   (one 16-row tile per wave) by x of the pair's token; bias, clamped SwiGLU, h rounded to
//   bf16 (the reference runs its experts in bf16) and written to the workspace. A routed
//   launch selects the experts in every workgroup (one wave, from the token's logits); the
//   first workgroup of each token also writes the selection.
// Launch 2 (down): workgroup (token, 16 output rows): wave j multiplies expert j's 16-row
//   down tile by h(token, j), which it turns into block-scaled terms while its tile streams
//   in; the waves' weighted rows are summed in a fixed order in LDS (one writer per output,
//   deterministic).
// No workgroup waits for another: stream order between the launches is the only
// synchronisation, so the grid needs no co-residency and the workspace carries no state
// from one call to the next.
//
// Semantics: tinyserve/_model_hooks.py:380-394 (MXFP4 expert with biases, clamped
// SwiGLU), :456-473 (routing), tinyserve/csrc/expert_loop.cpp:83-121 (weighted sum).
#include "fused_common.h"
#include "mfma_tile.h"
#include "mx_terms.h"

namespace tsa {

int64_t mx_tile_groups(int64_t K);
int64_t mx_tile_scale_bytes(int64_t K);

namespace {

constexpr int MAXT = FUSED_MAXT;
constexpr int MAXK = FUSED_MAXK;
constexpr int WAVES = 4;
constexpr int MISC_LDS = 1024;  // down launch: weighted rows [WAVES][16] floats, then the waves' A-scale tables
constexpr int VCH = 3072 / 8 / 64;  // 8-value chunks per lane when a wave holds a whole vector (length <= 3072)
constexpr int ASC_BYTES = 16 * VCH;  // A-scale table of one vector: one e8m0 byte per 32-value block (<= 96 blocks)

typedef int v8i __attribute__((ext_vector_type(8)));

struct MxtParams {
    tsa_expert_layout L;
    const uint8_t* pool;
    int64_t n_slots;
    int32_t* sel_slot;           // [T, k] slot per pair: the caller's (unrouted) or the workspace's (routed)
    float* sel_w;                // [T, k] weights, likewise
    const void* logits;          // [T, E] (routed) or null
    const int32_t* expert_slot;  // [E] (routed)
    int32_t* idx_out;            // [T, k] (routed, optional)
    float* w_out;                // [T, k] (routed, optional)
    int logits_dtype, route_mode, E;
    int T, k;
    const uint16_t* x;  // bf16 [T, H]
    void* y;
    int y_dtype;
    uint16_t* h;  // [T k][I] bf16
    int64_t gu_tile, gu_stile, dn_tile, dn_stile;  // bytes per 16-row tile: blocks, scale words
    struct MxtSync* sync;  // one-launch form: the workspace's sync area
    uint8_t* hterm;        // one-launch form: h as the down dot's terms, pair_term_bytes(I) per pair
    uint32_t wait_limit;   // one-launch form: polls before a wait gives up
    int n_gu;              // one-launch form: workgroups [0, n_gu) run gate_up
};

// A wave's 16-row tile: MM pieces of 1 KB and the scale words (byte m%4 of word m/4) as
// loaded; words >= w (past the row end) are masked where they are used (a select right
// after the load would make the wave wait for the scales before it issues the pieces).
// Buffer resources span exactly the tile, so pieces past a short row (K < 128 MM) read
// zero without touching memory.
template <int MM>
struct Tile {
    static constexpr int MS = (MM + 3) / 4;
    static constexpr int CHUNKS = (MS + 3) / 4;  // scale loads
    u32x4 q[MM];
    uint32_t sc[MS];
    int w;
};

// The scale words (w per lane, w = stile_bytes / 256 <= MS) come in lane-major chunks of
// up to 4 words: one 16-byte load per chunk, bounded to the tile's scale area. A load
// wider than a lane's part of a chunk picks up the next lane's words, which the mask at
// use removes. Issues exactly CHUNKS + MM buffer loads, in that order.
template <int MM>
__device__ __forceinline__ void tile_load(Tile<MM>& tl, const uint8_t* blocks, int64_t tile_bytes,
                                          const uint8_t* scales, int64_t stile_bytes, int lane) {
    const __amdgpu_buffer_rsrc_t rb =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t*>(blocks), (short)0, (int)tile_bytes, 0x00020000);
    const __amdgpu_buffer_rsrc_t rs =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t*>(scales), (short)0, (int)stile_bytes, 0x00020000);
    const int W = (int)(stile_bytes >> 8);
    tl.w = W;
#pragma unroll
    for (int c = 0; c < Tile<MM>::CHUNKS; ++c) {
        const int wc = W - 4 * c < 4 ? (W - 4 * c > 0 ? W - 4 * c : 0) : 4;  // this chunk's words per lane
        const u32x4 v = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rs, 4 * wc * lane, 1024 * c, 0));
#pragma unroll
        for (int d = 0; d < 4 && 4 * c + d < Tile<MM>::MS; ++d) tl.sc[4 * c + d] = v[d];
    }
    __builtin_amdgcn_sched_barrier(0);
    // Every piece is issued, in order, before any is used: left alone the scheduler sinks
    // loads into the MFMA loop to save registers or reorders them so that the first MFMA
    // waits for nearly the whole tile.
#pragma unroll
    for (int m = 0; m < MM; ++m) {  // nt: streamed once, keep it out of the caches' way
        tl.q[m] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rb, 16 * lane, 1024 * m, 2));
        __builtin_amdgcn_sched_barrier(0);
    }
}

// The tile's B-scale words moved to LDS (word g of lane l at st + 4 (64 g + l)), freeing their
// registers for the dot; waits for the scale loads only (the pieces, issued after them, stay
// in flight).
template <int MM>
__device__ __forceinline__ void tile_stash(const Tile<MM>& tl, uint8_t* st, int lane) {
#pragma unroll
    for (int g = 0; g < Tile<MM>::MS; ++g) *reinterpret_cast<uint32_t*>(st + 4 * (64 * g + lane)) = tl.sc[g];
}

// ---- checkpoint order ([N, G, 16] blocks, [N, G] scales, G = K / 32): the same MFMA operands,
// loaded lane by lane. Lane 16q + i loads, for piece m, the 16 bytes of the tile's row i,
// block 4m + q (its fp4 operand for column i, K block q), so a wave instruction reads 64
// contiguous bytes of each of the 16 rows; blocks past G read zero. The tile's scale bytes
// (16 G contiguous bytes, 16-byte aligned) come first as two 16-byte loads per lane into
// `scr`, for tile_stash_ck. CK_STAGE: LDS bytes of a wave's scale staging area.
constexpr int CK_STAGE = 2048;  // 16 G <= 2048 (G <= 96)
template <int MM>
__device__ __forceinline__ void tile_load_ck(Tile<MM>& tl, u32x4 (&scr)[2], const uint8_t* blocks,
                                             const uint8_t* scales, int G, int lane) {
    const __amdgpu_buffer_rsrc_t rb =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t*>(blocks), (short)0, 256 * G, 0x00020000);
    const __amdgpu_buffer_rsrc_t rs =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t*>(scales), (short)0, 16 * G, 0x00020000);
    tl.w = Tile<MM>::MS;  // scales past the row are masked in the stash
#pragma unroll
    for (int c = 0; c < 2; ++c)
        scr[c] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rs, 16 * (lane + 64 * c), 0, 0));
    __builtin_amdgcn_sched_barrier(0);
    const int i = lane & 15, q = lane >> 4;
#pragma unroll
    for (int m = 0; m < MM; ++m) {  // nt: streamed once
        const int g = 4 * m + q;
        const int off = g < G ? 16 * (i * G + g) : 256 * G;  // past the buffer: zero
        tl.q[m] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rb, off, 0, 2));
        __builtin_amdgcn_sched_barrier(0);
    }
}

// The scale bytes of a checkpoint-order tile rearranged into tile_stash's word layout (word
// g of lane 16q + i: byte j = scale of row i, block 16g + 4j + q; 127, a unit scale, past the
// row) through the wave's staging area; waits for the scale loads only.
template <int MM>
__device__ __forceinline__ void tile_stash_ck(const u32x4 (&scr)[2], uint8_t* stage, uint8_t* st, int G, int lane) {
    *reinterpret_cast<u32x4*>(stage + 16 * lane) = scr[0];
    *reinterpret_cast<u32x4*>(stage + 16 * (lane + 64)) = scr[1];
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");  // the wave reads what its lanes wrote
    const int i = lane & 15, q = lane >> 4;
    const uint8_t* row = stage + i * G;
#pragma unroll
    for (int g = 0; g < Tile<MM>::MS; ++g) {
        uint32_t w = 0;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int b = 16 * g + 4 * j + q;
            w |= (uint32_t)(b < G ? row[b] : 127) << (8 * j);
        }
        *reinterpret_cast<uint32_t*>(st + 4 * (64 * g + lane)) = w;
    }
}

// The bias of row r as one dword load bounded to the n-element bias vector (n * element
// size is a multiple of 4 here; a 2-byte element is the half of its dword that r & 1
// selects). A zero-size bound (no bias) reads 0. One register, so no reuse of a pending
// load's registers makes the wave wait for it early.
__device__ __forceinline__ uint32_t bias_word(const uint8_t* src, int dtype, int64_t n, int64_t r) {
    const int es = dtype == TSA_F32 ? 4 : 2;
    const __amdgpu_buffer_rsrc_t rb =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t*>(src), (short)0, (int)(n * es), 0x00020000);
    return __builtin_amdgcn_raw_buffer_load_b32(rb, (int)((r * es) & ~3ll), 0, 0);
}
__device__ __forceinline__ float bias_word_value(uint32_t w, int dtype, int64_t r) {
    if (dtype == TSA_F32) return __uint_as_float(w);
    const uint32_t h = (r & 1) ? (w >> 16) : (w & 0xFFFFu);
    return dtype == TSA_BF16 ? bf16_bits_to_f32(h) : f16_bits_to_f32(h);
}

// One scaled MFMA: D = A * B (+ C) with both operands' block scales taken per lane: lane
// 16q + r supplies the e8m0 scale of A row r, K block q, as byte OP of sa, and lane 16q + i
// that of B column i, K block q, as byte OP of sb.
template <int OP>
__device__ __forceinline__ v4f mfma_fp8_fp4(const v8i& A, const v8i& B, const v4f& C, int sa, int sb) {
    return __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(A, B, C, 0, 4, OP, sa, OP, sb);
}

// sum over the tile's K of W[i][k] v(k) in lane i < 16, W the wave's 16-row tile and v a
// vector held in LDS as two fp8 terms per value with per-block scales (chunk_terms). Piece m
// is one v_mfma_scale_f32_16x16x128_f8f6f4 (fp8 e4m3 A, cbsz 0; fp4 e2m1 B, blgp 4): A row r
// is term r over the piece's 128 K (rows 2..15 zero), B is the piece as loaded, and the block
// scales of both operands are applied by the instruction: lane 16q + i holds the scale word
// of (row i, blocks 4m' + q), so byte m % 4 of its word m / 4 is exactly its B scale for
// piece m, and byte m % 4 of the lane's word of the A-scale table is the A scale of block q of piece m. The
// MFMA accumulates across pieces. src: the lane's A-operand source (a_source). The A operands
// of the next two pieces are read ahead of each MFMA (sched barriers keep them there: left
// alone the scheduler moves the reads next to their use and the MFMAs wait for LDS, and
// the reads are volatile so that no earlier pass hoists them all to the top).
template <int MM, int PD = 2>
__device__ __forceinline__ float tile_dot(const Tile<MM>& tl, const uint8_t* src, const uint8_t* table, int lane,
                                         const uint8_t* bst = nullptr) {
    v4f acc = v4f{0.0f, 0.0f, 0.0f, 0.0f};
    u32x4 lo[PD + 1], hi[PD + 1];
    // the lane's A-scale word of pieces 4g .. 4g + 3 (the table's layout above), read one group
    // ahead; likewise its B-scale word from the tile's stash (tile_stash) when there is one
    const uint8_t* aw = table + 4 * (lane >> 4);
    uint32_t asc_cur = *(lds_u32*)(aw), asc_next = MM > 4 ? *(lds_u32*)(aw + 16) : 0u;
    const uint8_t* bw = bst + 4 * lane;
    uint32_t bsc_cur = bst ? *(lds_u32*)(bw) : 0u, bsc_next = bst && MM > 4 ? *(lds_u32*)(bw + 256) : 0u;
#pragma unroll
    for (int i = 0; i <= PD && i < MM; ++i) {
        lo[i] = lds16(src + 128 * i);
        hi[i] = lds16(src + 128 * i + 64);
    }
#pragma unroll
    for (int m = 0; m < MM; ++m) {
        const int b = m % (PD + 1);
        const v8i A = {(int)lo[b][0], (int)lo[b][1], (int)lo[b][2], (int)lo[b][3],
                       (int)hi[b][0], (int)hi[b][1], (int)hi[b][2], (int)hi[b][3]};
        const v8i B = {(int)tl.q[m][0], (int)tl.q[m][1], (int)tl.q[m][2], (int)tl.q[m][3], 0, 0, 0, 0};
        if (m % 4 == 0 && m > 0) {
            asc_cur = asc_next;
            if (m + 4 < MM) asc_next = *(lds_u32*)(aw + 16 * (m / 4 + 1));
            if (bst) {
                bsc_cur = bsc_next;
                if (m + 4 < MM) bsc_next = *(lds_u32*)(bw + 256 * (m / 4 + 1));
            }
        }
        // past the row end: any finite scale
        const int sb = m / 4 < tl.w ? (int)(bst ? bsc_cur : tl.sc[m / 4]) : 0x7F7F7F7F;
        const int sa = (int)asc_cur;
        switch (m & 3) {
            case 0: acc = mfma_fp8_fp4<0>(A, B, acc, sa, sb); break;
            case 1: acc = mfma_fp8_fp4<1>(A, B, acc, sa, sb); break;
            case 2: acc = mfma_fp8_fp4<2>(A, B, acc, sa, sb); break;
            default: acc = mfma_fp8_fp4<3>(A, B, acc, sa, sb); break;
        }
        asm volatile("" : "+v"(acc));  // piece m's MFMA stays ahead of the next reads
        if (m + PD + 1 < MM) {
            lo[b] = lds16(src + 128 * (m + PD + 1));
            hi[b] = lds16(src + 128 * (m + PD + 1) + 64);
        }
        __builtin_amdgcn_sched_barrier(0);
    }
    return acc[0] + acc[1];  // lanes 0..15: rows 0 and 1 of D, column = lane
}

// The lane's A-operand source for a vector whose two terms start at `terms` (term r at
// terms + r * kp, zero past the vector's end): lane l holds row l % 16 of A, bytes 0..15 =
// K 16 (l / 16) .. + 15 and bytes 16..31 = K 64 + 16 (l / 16) .. + 15 of each piece (read at
// src + 128 m and src + 128 m + 64); rows 2..15 read a zero area of kp bytes instead.
__device__ __forceinline__ const uint8_t* a_source(const uint8_t* terms, const uint8_t* zero, int kp, int lane) {
    const int row = lane & 15, kq = lane >> 4;
    return row < 2 ? terms + row * kp + 16 * kq : zero;
}

// Block-scaled fp8 terms of chunk set i of a bf16 vector (mx_terms.h): lane l holds chunk
// c = l + 64 i (8 values, zero past the vector's end), so a lane quad holds block 16 i + l / 4.
// (All lanes read an A-scale word: rows 2..15 of A are zero, and every table byte is a
// finite scale.)
__device__ __forceinline__ void chunk_terms(const u32x4& v, int i, int lane, uint8_t* terms, int kp, uint8_t* table) {
    const int c = lane + 64 * i;
    block_terms(v, c >> 2, (lane & 3) == 0, 8 * c < kp ? terms + 8 * c : nullptr, terms + kp + 8 * c, table);
}

// Zero bytes [from, to) of an LDS area (16-byte multiples), spread over nthr threads.
__device__ __forceinline__ void lds_zero(uint8_t* a, int from, int to, int me, int nthr) {
    for (int o = from + 16 * me; o < to; o += 16 * nthr) *reinterpret_cast<u32x4*>(a + o) = u32x4{0u, 0u, 0u, 0u};
}

constexpr int GU_WAVES = 2;  // waves per workgroup of the gate_up launch (one 16-row tile each)

// The token's routing from its logits (all k rounds): lane r < k ends with the r-th selected
// expert id and slot and its weight (softmax over the k selected logits, or the unnormalised
// mode's softmax over all E).
template <class P>
__device__ float route_weights(const P& p, int lane, const float lg[4], const int es[4], int k, int& mysel,
                               int& myslot) {
    uint32_t myk;
    select_topk(p, lane, lg, es, k, myk, mysel, myslot);
    const float myval = route_key_value(myk);
    const float top = route_key_value((uint32_t)__builtin_amdgcn_readfirstlane((int)myk));
    if (p.route_mode == TSA_ROUTE_SOFTMAX_TOPK) {
        float sum = 0.0f;
#pragma unroll
        for (int j = 0; j < 4; ++j)
            if (lane + 64 * j < p.E) sum += __expf(lg[j] - top);
        const float z = wave_sum_u(sum);
        return lane < k ? __expf(myval - top) / z : 0.0f;
    }
    const float ex = lane < k ? __expf(myval - top) : 0.0f;
    return ex / row16_sum(ex);
}

// ---- launch 1 of the two-launch form: workgroup b of NW waves multiplies 16 NW gate_up rows
// of one (token, expert) pair by x of the token; bias, clamped SwiGLU, h rounded to bf16 into
// the workspace. Pair b % (T k), row block b / (T k) (pair-major, so neighbouring workgroups
// stream different experts).
//
// Each wave selects the token's experts itself and issues its tile's loads as soon as it
// knows the slot. Each wave also loads all of x; in the shadow of the tile loads the waves
// convert interleaved 512-value chunk sets of x into the shared block-scaled terms and meet
// at the workgroup's barrier before the dot.
template <int MM, int NW, bool CK = false>
__device__ __forceinline__ void gate_up_body(const MxtParams& p, int b) {
    extern __shared__ __align__(16) uint8_t smem[];
    constexpr int KP = 128 * MM;  // padded vector length
    const int tid = threadIdx.x, lane = tid & 63, wave = uniform(tid >> 6);
    const tsa_expert_layout& L = p.L;
    const int H = (int)L.hidden, I = (int)L.inter, k = p.k;
    const int pairs = p.T * k;
    const int kb = b / pairs, pr = b % pairs, t = pr / k, jj = pr % k;
    uint8_t* vec = smem;  // x terms [2][KP], a zero area [KP], then x's A-scale table
    uint8_t* zero = vec + 2 * KP;
    uint8_t* table = zero + KP;
    const bool routed = p.logits != nullptr;

    // ---- loads, all issued before any is used: x of token t, then the routing inputs
    u32x4 xr[VCH];
    const uint16_t* xt = p.x + (int64_t)t * H;
#pragma unroll
    for (int i = 0; i < VCH; ++i) {
        const int c = lane + 64 * i;
        xr[i] = c < H / 8 ? *reinterpret_cast<const u32x4*>(xt + 8 * c) : u32x4{0u, 0u, 0u, 0u};
    }
    float lg[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    int es[4] = {0, 0, 0, 0};
    int64_t slot = -1;
    int mysel = -1, myslot = -1;
    if (routed) {
        uint32_t myk;
#pragma unroll
        for (int j = 0; j < 4; ++j) es[j] = p.expert_slot[min(lane + 64 * j, p.E - 1)];
        load4(p.logits, p.logits_dtype, (int64_t)t * p.E, p.E, lane, lg);
        select_topk(p, lane, lg, es, jj + 1, myk, mysel, myslot);  // the pair's selection is round jj
        slot = __builtin_amdgcn_readlane(myslot, jj);
    } else {
        slot = uniform(p.sel_slot[pr]);
    }

    // the token's first workgroup publishes the selection (all k rounds)
    auto publish = [&]() {
        const float w = route_weights(p, lane, lg, es, k, mysel, myslot);
        if (lane < k) {
            p.sel_slot[t * k + lane] = myslot;
            p.sel_w[t * k + lane] = w;
            if (p.idx_out) {
                p.idx_out[t * k + lane] = mysel;
                p.w_out[t * k + lane] = w;
            }
        }
    };
    const bool publisher = routed && kb == 0 && jj == 0 && wave == 0;
    const bool live = slot >= 0 && slot < p.n_slots;
    if (!live) {  // a dead pair's h is never read
        if (publisher) publish();
        return;
    }

    // ---- the wave's gate_up tile: rows row0 .. row0 + 15 of the pair's expert, after its bias
    const int64_t row0 = (int64_t)kb * 16 * NW + 16 * wave;
    const uint8_t* base = p.pool + slot * L.slot_bytes;
    const bool hbias = L.gate_bias_off >= 0;
    const int64_t brow = row0 + (lane & 15);
    const uint32_t bw = bias_word(base + (hbias ? L.gate_bias_off : 0), L.bias_dtype, hbias ? 2 * (int64_t)I : 0, brow);
    Tile<MM> tl;
    u32x4 scr[2];
    const int G = H / 32;
    if constexpr (CK)
        tile_load_ck<MM>(tl, scr, base + L.gate_off + row0 * 16 * G, base + L.gate_scales_off + row0 * G, G, lane);
    else
        tile_load<MM>(tl, base + L.gate_off + (row0 / 16) * p.gu_tile, p.gu_tile,
                      base + L.gate_scales_off + (row0 / 16) * p.gu_stile, p.gu_stile, lane);
    if (publisher) publish();  // while the tile streams in

    // ---- x as block-scaled terms (chunk sets i = wave, wave + NW, ...; past H they are zero)
#pragma unroll
    for (int i = 0; i < VCH; ++i)
        if (i % NW == wave) chunk_terms(xr[i], i, lane, vec, KP, table);
    lds_zero(zero, 0, KP, tid, 64 * NW);
    uint8_t* stash = table + ASC_BYTES + wave * (CK_STAGE + 256 * Tile<MM>::MS) + CK_STAGE;
    if constexpr (CK) tile_stash_ck<MM>(scr, stash - CK_STAGE, stash, G, lane);
    __syncthreads();  // every pair is live or dead for all waves: all get here or none

    const float a = CK ? tile_dot<MM>(tl, a_source(vec, zero, KP, lane), table, lane, stash)
                       : tile_dot<MM>(tl, a_source(vec, zero, KP, lane), table, lane);
    const float bias = bias_word_value(bw, L.bias_dtype, brow);  // 0 without a bias
    const float tot = a + bias;  // lanes 0..15: row row0 + lane
    // rows alternate gate, up: lane 2r holds h[row0 / 2 + r]; lanes 0, 4, 8, 12 store two
    // values each (their own and lane + 2's, by quad_perm [2,3,2,3])
    const float up = __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(tot), 0xB1, 0xF, 0xF, false));
    const int hb = (int)f32_to_bf16_bits(swiglu_oai(L, tot, up));
    const int hb2 = __builtin_amdgcn_mov_dpp(hb, 0xEE, 0xF, 0xF, false);
    if (lane < 16 && (lane & 3) == 0)
        *reinterpret_cast<uint32_t*>(p.h + (int64_t)pr * I + row0 / 2 + (lane >> 1)) =
            ((uint32_t)hb & 0xFFFFu) | ((uint32_t)hb2 << 16);
}

template <int MM, bool CK>
__global__ void __launch_bounds__(64 * GU_WAVES) mxt_gate_up_kernel(MxtParams p) {
    gate_up_body<MM, GU_WAVES, CK>(p, (int)blockIdx.x);
}

// ---- launch 2 of the two-launch form: workgroup d (token d / (H / 16), output rows
// 16 (d % (H / 16)) .. + 15) runs the down tiles of every selected expert of its token, wave
// j = expert j (further experts take further rounds), and sums the waves' weighted rows in a
// fixed order in LDS (one writer per output, deterministic). Each wave turns its pair's h
// into block-scaled terms while its tile streams in.
template <int MM, bool CK>
__global__ void __launch_bounds__(256, 2) mxt_down_kernel(MxtParams p) {
    extern __shared__ __align__(16) uint8_t smem[];
    constexpr int KP = 128 * MM;  // padded vector length
    const int tid = threadIdx.x, lane = tid & 63, wave = uniform(tid >> 6);
    const tsa_expert_layout& L = p.L;
    const int H = (int)L.hidden, I = (int)L.inter, k = p.k;
    const int RB = H / 16;
    const int d = (int)blockIdx.x;
    const int t = d / RB;
    const int64_t n0 = (int64_t)(d % RB) * 16;
    float* s_y = reinterpret_cast<float*>(smem);             // [WAVES][16]
    uint8_t* table = smem + 64 * WAVES + ASC_BYTES * wave;  // this wave's h A-scale table
    uint8_t* hs = smem + MISC_LDS + wave * 2 * KP;          // this wave's h terms [2][KP]
    uint8_t* zero = smem + MISC_LDS + WAVES * 2 * KP;
    uint8_t* stash = zero + KP + wave * (CK_STAGE + 256 * Tile<MM>::MS) + CK_STAGE;  // checkpoint order
    const int G = I / 32;
    const bool hbias = L.down_bias_off >= 0;
    const int rounds = (k + WAVES - 1) / WAVES;

    // the first round's selection as scalar loads, ahead of every vector load (inside the loop
    // they would be vector loads whose wait covers the h loads issued before them)
    const int j0 = wave < k ? wave : k - 1;
    const int64_t slot0 = uniform(p.sel_slot[t * k + j0]);
    const float w0 = __int_as_float(uniform(__float_as_int(p.sel_w[t * k + j0])));
    lds_zero(zero, 0, KP, tid, 256);
    __syncthreads();  // the only barrier before the weighted sum: the waves stream independently
    float yv = 0.0f;  // lanes 0..15: row n0 + lane, this wave's weighted experts
#pragma unroll 1
    for (int rd = 0; rd < rounds; ++rd) {
        const int j = rd * WAVES + wave;
        if (j >= k) break;
        // h(t, j) in 8-value chunks into registers (bounded to the vector: zero past its end),
        // then the bias and the tile
        const int64_t slot = rd == 0 ? slot0 : uniform(p.sel_slot[t * k + j]);
        const float w = rd == 0 ? w0 : __int_as_float(uniform(__float_as_int(p.sel_w[t * k + j])));
        const __amdgpu_buffer_rsrc_t rh = __builtin_amdgcn_make_buffer_rsrc(
            const_cast<uint16_t*>(p.h + (int64_t)(t * k + j) * I), (short)0, 2 * I, 0x00020000);
        u32x4 hr[VCH];
#pragma unroll
        for (int i = 0; i < VCH; ++i)
            hr[i] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rh, 16 * (lane + 64 * i), 0, 0));
        __builtin_amdgcn_sched_barrier(0);
        if (slot < 0 || slot >= p.n_slots) continue;  // contributes nothing
        const uint8_t* base = p.pool + slot * L.slot_bytes;
        Tile<MM> tl;
        const int64_t brow = n0 + (lane & 15);
        const uint32_t bw = bias_word(base + (hbias ? L.down_bias_off : 0), L.bias_dtype, hbias ? (int64_t)H : 0, brow);
        u32x4 scr[2];
        if constexpr (CK)
            tile_load_ck<MM>(tl, scr, base + L.down_off + n0 * 16 * G, base + L.down_scales_off + n0 * G, G, lane);
        else
            tile_load<MM>(tl, base + L.down_off + (n0 / 16) * p.dn_tile, p.dn_tile,
                          base + L.down_scales_off + (n0 / 16) * p.dn_stile, p.dn_stile, lane);
        // h as block-scaled terms while the tile streams in (the h loads are the oldest)
#pragma unroll
        for (int i = 0; i < VCH; ++i) chunk_terms(hr[i], i, lane, hs, KP, table);
        if constexpr (CK) tile_stash_ck<MM>(scr, stash - CK_STAGE, stash, G, lane);
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");  // the wave's own terms and table are in LDS
        const float a = CK ? tile_dot<MM>(tl, a_source(hs, zero, KP, lane), table, lane, stash)
                           : tile_dot<MM>(tl, a_source(hs, zero, KP, lane), table, lane);
        const float bias = bias_word_value(bw, L.bias_dtype, brow);  // 0 without a bias
        yv += w * (a + bias);
    }
    if (lane < 16) s_y[wave * 16 + lane] = yv;
    __syncthreads();
    if (wave == 0 && lane < 16) {
        float sum = 0.0f;
#pragma unroll
        for (int w = 0; w < WAVES; ++w) sum += s_y[w * 16 + lane];
        store_out(p.y, p.y_dtype, (int64_t)t * H + n0 + lane, sum);
    }
}

// =====================================================================================
// The one-launch form (k <= 4 experts per token, inter a multiple of 64). Workgroups of 8
// waves (two per SIMD, so they pack four to a CU): workgroups [0, n_gu) run gate_up (128 rows
// of one pair, eight 16-row tiles: two 32-value blocks of h), the rest run down (16 output
// rows of one token: waves 0..3 compute, wave j on expert j; waves 4..7 are helpers, helper
// 4 + j fetching pair j's h). Down workgroups come after every gate_up workgroup in dispatch
// order, so a waiting workgroup's producers have all been dispatched: they run whether or not
// the whole grid is resident.
//
// Hand-over. A gate_up workgroup writes its blocks of h as the down dot's operands: the two
// fp8 terms of each value and the block's A-scale byte (at its place in the down wave's scale
// table), at agent scope (sc1: coherent across the XCDs' L2 caches). A sync area at the
// start of the workspace holds a call counter (gen) and one flag per workgroup. One wave of
// each workgroup reads gen = g when it starts; a gate_up workgroup sets its flag to next(g)
// once its stores are complete, a down workgroup sets its flag to next(g) as soon as it has
// read g. Each down helper waits for the flags of its pair and copies the pair's terms into
// LDS while the compute waves' tiles stream in (a helper has no tile loads in flight, so its
// polls return at once; a compute wave's poll would wait behind its tile). The last down
// workgroup first waits for every flag of the call (so every workgroup has read g) and
// advances gen to next(g): a flag never holds next(g) before the call writes it, provided
// every word of the area held one value before the first call (zero it, or fill it with any
// one byte). Waits are bounded: a helper that gives up makes its workgroup write NaN and sets
// gen to GEN_POISON, after which every call on the workspace writes NaN until the area is
// cleared again.
constexpr int F_WAVES = 2 * WAVES;          // eight waves per workgroup
constexpr int F_MISC = 1024;                // slots, weights, block maxima, status, weighted rows
constexpr uint32_t GEN_POISON = MXT_GEN_POISON;
struct MxtSync {
    uint32_t gen;
    uint32_t pad[63];
    uint32_t gflag[MXT_SYNC_GFLAGS];  // gate_up workgroup (pair pr, block pair m): pr * (I / 64) + m
    uint32_t dflag[MXT_SYNC_DFLAGS];  // down workgroup (token t, row block rb): t * (H / 16) + rb
    uint32_t relay[MAXT][8][32];      // per token and XCD (one 128-byte line each): its pairs are complete
};
static_assert(sizeof(MxtSync) <= MXT_SYNC_BYTES, "sync area");

// The terms of one pair in the workspace: hi [I] bytes, lo [I] bytes, then the A-scale table
// (ASC_BYTES, in the A-scale table's order), padded to 256 bytes.
__host__ __device__ __forceinline__ int64_t pair_term_bytes(int64_t I) { return (2 * I + ASC_BYTES + 255) / 256 * 256; }

__device__ __forceinline__ uint32_t next_gen(uint32_t g) { return g + 1 == GEN_POISON ? g + 2 : g + 1; }
__device__ __forceinline__ uint32_t load_agent(const uint32_t* a) {
    return __hip_atomic_load(const_cast<uint32_t*>(a), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void store_agent(uint32_t* a, uint32_t v) {
    __hip_atomic_store(a, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void poison(MxtSync* s) {
    __hip_atomic_exchange(&s->gen, GEN_POISON, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
// Whole-wave bounded wait until words [0, n) of f all equal v: polls (agent-scope loads) with
// a short sleep between them, at most `limit` times (0: give up at once). True if they did.
__device__ bool wait_flags(const uint32_t* f, int n, uint32_t v, uint32_t limit, int lane) {
    for (uint32_t it = 0; it < limit; ++it) {
        bool ok = true;
        for (int i = lane; i < n; i += 64) ok = ok && load_agent(f + i) == v;
        if (__builtin_amdgcn_ballot_w64(!ok) == 0) return true;
        __builtin_amdgcn_s_sleep(2);
    }
    return false;
}

// The down helper's wait for every pair of token t (all flags equal want, bounded). Each round
// reads the token's relay word for this XCD at XCD scope (sc0: past the CU's L1, an L2 hit, no
// memory traffic); one round in four, staggered by workgroup, polls the flags themselves at
// agent scope and, once they are complete, sets the relay for the other workgroups on the XCD
// (so a flag line is polled by a quarter of the workgroups at a time, not all of them). The
// relay only ever says what a poll of the flags saw, so its XCD index need not be exact.
__device__ bool wait_token(const MxtParams& p, int t, uint32_t want, int lane, int d) {
    const int n = p.k * (int)(p.L.inter / 64);
    const uint32_t* f = &p.sync->gflag[t * n];
    const int xcc = __builtin_amdgcn_s_getreg((20) | (0 << 6) | (3 << 11)) & 7;  // HW_REG_XCC_ID
    const __amdgpu_buffer_rsrc_t rr =
        __builtin_amdgcn_make_buffer_rsrc(&p.sync->relay[t][xcc][0], (short)0, 4, 0x00020000);
    for (uint32_t it = 0; it < p.wait_limit; ++it) {
        if (__builtin_amdgcn_raw_buffer_load_b32(rr, 0, 0, 1) == want) return true;
        if (((it + (uint32_t)d) & 3) == 0) {
            bool ok = true;
            for (int i = lane; i < n; i += 64) ok = ok && load_agent(f + i) == want;
            if (__builtin_amdgcn_ballot_w64(!ok) == 0) {
                if (lane == 0) __builtin_amdgcn_raw_buffer_store_b32(want, rr, 0, 0, 1);
                return true;
            }
        }
        __builtin_amdgcn_s_sleep(2);
    }
    return false;
}

// 16 bytes per lane at buffer offset voff, at agent scope (sc1), straight into LDS at
// lds + 16 lane (one 1 KB wave transfer); 4 bytes per lane (256 B) for the dword form.
// Issued from inline assembly: the caller waits for them with its own s_waitcnt.
__device__ __forceinline__ void lds_dma16_agent(const __amdgpu_buffer_rsrc_t& r, uint32_t voff, uint32_t lds) {
    asm volatile("s_mov_b32 m0, %2\n\tbuffer_load_dwordx4 %0, %1, 0 offen sc1 lds" ::"v"(voff), "s"(r), "s"(lds)
                 : "memory", "m0");
}
__device__ __forceinline__ void lds_dma4_agent(const __amdgpu_buffer_rsrc_t& r, uint32_t voff, uint32_t lds) {
    asm volatile("s_mov_b32 m0, %2\n\tbuffer_load_dword %0, %1, 0 offen sc1 lds" ::"v"(voff), "s"(r), "s"(lds)
                 : "memory", "m0");
}

template <int MM>
__device__ __forceinline__ void fused_gate_up(const MxtParams& p, int b) {
    extern __shared__ __align__(16) uint8_t smem[];
    constexpr int KP = 128 * MM;
    const int tid = threadIdx.x, lane = tid & 63, wave = uniform(tid >> 6);
    const tsa_expert_layout& L = p.L;
    const int H = (int)L.hidden, I = (int)L.inter, k = p.k;
    const int pairs = p.T * k;
    const int m = b / pairs, pr = b % pairs, t = pr / k, jj = pr % k;
    const int kb = 2 * m + (wave >> 2);                    // the wave's block of h
    const int64_t row0 = (int64_t)m * 128 + 16 * wave;     // the wave's 16 gate_up rows
    float* s_max = reinterpret_cast<float*>(smem + 128);  // [8]
    uint8_t* vec = smem + F_MISC;                          // x terms [2][KP], zero [KP], x's table
    uint8_t* zero = vec + 2 * KP;
    uint8_t* table = zero + KP;
    uint8_t* stash = table + 128 + wave * (256 * Tile<MM>::MS);  // the wave's B-scale words
    uint8_t* terms = p.hterm + pr * pair_term_bytes(I);
    // gen as a plain load: the previous call's update is visible across kernel boundaries, and
    // agent-scope loads of one word by every workgroup would queue at its memory channel
    const uint32_t g = wave == 0 ? p.sync->gen : 0u;

    // ---- loads, all issued before any is used: the wave's chunk set of x, then the routing inputs
    u32x4 xr = u32x4{0u, 0u, 0u, 0u};
    const int xc = lane + 64 * wave;
    if (wave < VCH && xc < H / 8) xr = *reinterpret_cast<const u32x4*>(p.x + (int64_t)t * H + 8 * xc);
    float lg[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    int es[4] = {0, 0, 0, 0};
    int64_t slot = -1;
    int mysel = -1, myslot = -1;
    if (p.logits) {
        uint32_t myk;
#pragma unroll
        for (int j = 0; j < 4; ++j) es[j] = p.expert_slot[min(lane + 64 * j, p.E - 1)];
        load4(p.logits, p.logits_dtype, (int64_t)t * p.E, p.E, lane, lg);
        select_topk(p, lane, lg, es, jj + 1, myk, mysel, myslot);  // the pair's selection is round jj
        slot = __builtin_amdgcn_readlane(myslot, jj);
    } else {
        slot = uniform(p.sel_slot[pr]);
    }
    const bool publisher = p.logits && m == 0 && jj == 0 && wave == 0;
    if (wave == 0 && g == GEN_POISON) slot = -1;  // a poisoned workspace: no work, no flag
    // every wave reaches B0 (the poisoned check is wave 0's): the slot as wave 0 sees it
    int* s_live = reinterpret_cast<int*>(smem);
    if (tid == 0) *s_live = slot >= 0 && slot < p.n_slots;
    __syncthreads();  // B0
    if (!uniform(*s_live)) {  // a dead pair: nothing to compute; the flag says g was read
        if (wave == 0 && lane == 0 && g != GEN_POISON) store_agent(&p.sync->gflag[pr * (I / 64) + m], next_gen(g));
        if (publisher) {
            const float w = route_weights(p, lane, lg, es, k, mysel, myslot);
            if (lane < k && p.idx_out) {
                p.idx_out[t * k + lane] = mysel;
                p.w_out[t * k + lane] = w;
            }
        }
        return;
    }
    // x's terms and the publication before the tile loads (x arrived with the routing inputs;
    // done later they would hold registers across the tile)
    if (wave < VCH) chunk_terms(xr, wave, lane, vec, KP, table);
    if (publisher) {
        const float w = route_weights(p, lane, lg, es, k, mysel, myslot);
        if (lane < k && p.idx_out) {
            p.idx_out[t * k + lane] = mysel;
            p.w_out[t * k + lane] = w;
        }
    }
    const uint8_t* base = p.pool + slot * L.slot_bytes;
    const bool hbias = L.gate_bias_off >= 0;
    const int64_t brow = row0 + (lane & 15);
    const uint32_t bw = bias_word(base + (hbias ? L.gate_bias_off : 0), L.bias_dtype, hbias ? 2 * (int64_t)I : 0, brow);
    Tile<MM> tl;
    tile_load<MM>(tl, base + L.gate_off + (row0 / 16) * p.gu_tile, p.gu_tile,
                  base + L.gate_scales_off + (row0 / 16) * p.gu_stile, p.gu_stile, lane);
    tile_stash(tl, stash, lane);
    lds_zero(zero, 0, KP, tid, 64 * F_WAVES);
    __syncthreads();  // B1: x's terms and the stashes
    const float a = tile_dot<MM, 1>(tl, a_source(vec, zero, KP, lane), table, lane, stash);
    const float tot = a + bias_word_value(bw, L.bias_dtype, brow);  // lanes 0..15: row row0 + lane
    // rows alternate gate, up: lane 2r (r < 8) holds h value 8 (wave % 4) + r of block kb,
    // rounded to bf16 as the reference's bf16 expert computes it
    const float up = __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(tot), 0xB1, 0xF, 0xF, false));
    const float hv = bf16_bits_to_f32(f32_to_bf16_bits(swiglu_oai(L, tot, up)));
    // the maximum over lanes 0, 2, .., 14: quad_perm [2,3,0,1] (lane 4i then holds its quad's),
    // then row_ror 4 and 8 (each lane of the first row then holds all four quads')
    float mx = lane < 16 && (lane & 1) == 0 ? fabsf(hv) : 0.0f;
    mx = fmaxf(mx, __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(mx), 0x4E, 0xF, 0xF, false)));
    mx = fmaxf(mx, __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(mx), 0x124, 0xF, 0xF, false)));
    mx = fmaxf(mx, __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(mx), 0x128, 0xF, 0xF, false)));
    if (lane == 0) s_max[wave] = mx;
    __syncthreads();  // B2: the waves' maxima
    const int w0 = wave & ~3;
    const float bm = fmaxf(fmaxf(s_max[w0], s_max[w0 + 1]), fmaxf(s_max[w0 + 2], s_max[w0 + 3]));
    // the block's scale as chunk_terms takes it (exponent of the largest |h|, clamped)
    const uint32_t mb = f32_to_bf16_bits(bm) & 0x7FFFu;
    const int e = mb ? min(max((int)(mb >> 7) - 127, -120), 127) : 0;
    const float s = __uint_as_float((uint32_t)(134 - e) << 23);
    uint32_t hi2, lo2;
    fp8_terms(hv * s, 0.0f, hi2, lo2);
    // lanes 0, 2, .., 14 hold the wave's 8 values: gather 4 per dword, stored by lanes 0 and 8
    const uint32_t hb = (hi2 & 255u) | ((lo2 & 255u) << 8);
    const uint32_t b1 = (uint32_t)__shfl_down((int)hb, 2), b2 = (uint32_t)__shfl_down((int)hb, 4),
                   b3 = (uint32_t)__shfl_down((int)hb, 6);
    if (lane == 0 || lane == 8) {
        const uint32_t ph = (hb & 255u) | ((b1 & 255u) << 8) | ((b2 & 255u) << 16) | ((b3 & 255u) << 24);
        const uint32_t pl = (hb >> 8) | ((b1 >> 8) << 8) | ((b2 >> 8) << 16) | ((b3 >> 8) << 24);
        const int64_t o = (int64_t)kb * 32 + 8 * (wave & 3) + (lane >> 1);
        store_agent(reinterpret_cast<uint32_t*>(terms + o), ph);
        store_agent(reinterpret_cast<uint32_t*>(terms + I + o), pl);
    }
    // the block's A-scale byte at its place in the A-scale table (by the block's first wave);
    // the pair's first workgroup also gives the table's blocks past I a finite scale (1.0:
    // their terms read as zero)
    const int nb = I / 32;
    if ((wave & 3) == 0) {
        for (int b2i = lane; b2i < ASC_BYTES; b2i += 64) {
            if (b2i == kb || (m == 0 && wave == 0 && b2i >= nb)) {
                const int tb = 4 * (4 * (b2i / 16) + b2i % 4) + (b2i % 16) / 4;
                __hip_atomic_store(terms + 2 * I + tb, (uint8_t)(b2i == kb ? 120 + e : 127), __ATOMIC_RELAXED,
                                   __HIP_MEMORY_SCOPE_AGENT);
            }
        }
    }
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // the wave's stores are complete
    __syncthreads();  // B3
    if (tid == 0) store_agent(&p.sync->gflag[pr * (I / 64) + m], next_gen(g));
}

template <int MM>
__device__ __forceinline__ void fused_down(const MxtParams& p, int d) {
    extern __shared__ __align__(16) uint8_t smem[];
    constexpr int KP = 128 * MM;
    constexpr int KT = (KP + 1023) / 1024 * 1024;  // bytes per term in LDS (whole 1 KB transfers)
    const int tid = threadIdx.x, lane = tid & 63, wave = uniform(tid >> 6);
    const tsa_expert_layout& L = p.L;
    const int H = (int)L.hidden, I = (int)L.inter, k = p.k;
    const int RB = H / 16;
    const int t = d / RB;
    const int64_t n0 = (int64_t)(d % RB) * 16;
    int* s_slot = reinterpret_cast<int*>(smem);            // [16]
    float* s_w = reinterpret_cast<float*>(smem + 64);      // [16]
    int* s_fail = reinterpret_cast<int*>(smem + 128);      // a helper gave up, or the workspace is poisoned
    uint32_t* s_gen = reinterpret_cast<uint32_t*>(smem + 132);
    float* s_y = reinterpret_cast<float*>(smem + 256);     // [WAVES][16]
    uint8_t* tables = smem + 512;                          // [WAVES][128]: the pairs' A-scale tables
    uint8_t* hs = smem + F_MISC;                           // [WAVES][2][KT]: the pairs' terms
    uint8_t* zero = hs + WAVES * 2 * KT;                   // [KP]
    uint8_t* stash = zero + KP + (wave & 3) * (256 * Tile<MM>::MS);  // compute wave's B-scale words

    if (wave >= WAVES) {  // helpers
        const int j = wave - WAVES;
        if (j == 0) {  // gen, the routing and the workgroup's flag
            const uint32_t g = p.sync->gen;  // a plain load, as in the gate_up role
            if (p.logits) {
                float lg[4];
                int es[4], mysel, myslot;
#pragma unroll
                for (int jx = 0; jx < 4; ++jx) es[jx] = p.expert_slot[min(lane + 64 * jx, p.E - 1)];
                load4(p.logits, p.logits_dtype, (int64_t)t * p.E, p.E, lane, lg);
                const float w = route_weights(p, lane, lg, es, k, mysel, myslot);
                if (lane < k) {
                    s_slot[lane] = myslot;
                    s_w[lane] = w;
                }
            } else if (lane < k) {
                s_slot[lane] = p.sel_slot[t * k + lane];
                s_w[lane] = p.sel_w[t * k + lane];
            }
            if (lane == 0) {
                *s_gen = g;
                *s_fail = g == GEN_POISON;
                if (g != GEN_POISON) store_agent(&p.sync->dflag[d], next_gen(g));  // g has been read
            }
        }
        lds_zero(zero, 0, KP, tid - 64 * WAVES, 64 * WAVES);
        __syncthreads();  // B1: the selection
        if (j == 0) {  // helper 4: waits for the token's pairs, then copies their terms into LDS
            const uint32_t g = uniform((int)*s_gen);
            const uint32_t want = next_gen(g);
            bool ok = g != GEN_POISON;
            if (ok && d == p.T * RB - 1) {  // the last workgroup: once every workgroup has read g, advance gen
                ok = wait_flags(p.sync->dflag, p.T * RB, want, p.wait_limit, lane) &&
                     wait_flags(p.sync->gflag, p.T * k * (I / 64), want, p.wait_limit, lane);
                if (lane == 0) {
                    if (ok)
                        atomicCAS(&p.sync->gen, g, want);  // agent scope; fails only if a wait gave up meanwhile
                    else
                        poison(p.sync);
                }
            }
            if (ok && !wait_token(p, t, want, lane, d)) {
                ok = false;
                if (lane == 0) poison(p.sync);
            }
            for (int jp = 0; jp < k && ok; ++jp) {
                const int slot = uniform(s_slot[jp]);
                if (slot < 0 || slot >= p.n_slots) continue;
                const uint8_t* src = p.hterm + (t * k + jp) * pair_term_bytes(I);
                const uint32_t dst = (uint32_t)reinterpret_cast<uintptr_t>(hs + jp * 2 * KT);
#pragma unroll
                for (int r = 0; r < 2; ++r) {
                    const __amdgpu_buffer_rsrc_t rs =
                        __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t*>(src + r * I), (short)0, I, 0x00020000);
#pragma unroll
                    for (int i = 0; i < KT / 1024; ++i)
                        lds_dma16_agent(rs, (uint32_t)(1024 * i + 16 * lane), dst + (uint32_t)(r * KT + 1024 * i));
                }
                const __amdgpu_buffer_rsrc_t rt = __builtin_amdgcn_make_buffer_rsrc(
                    const_cast<uint8_t*>(src + 2 * I), (short)0, ASC_BYTES, 0x00020000);
                if (lane < 32)
                    lds_dma4_agent(rt, (uint32_t)(4 * lane), (uint32_t)reinterpret_cast<uintptr_t>(tables + 128 * jp));
            }
            if (!ok && lane == 0) *s_fail = 1;
            asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)" ::: "memory");  // the terms are in LDS
        }
        __syncthreads();  // B2
        __syncthreads();  // B3: the weighted rows
        return;
    }
    // compute wave j = wave: its expert's down tile while its helper fetches h
    __syncthreads();  // B1
    const int j = wave;
    const int64_t slot = j < k ? uniform(s_slot[j]) : -1;
    const float w = j < k ? s_w[j] : 0.0f;
    const bool live = slot >= 0 && slot < p.n_slots && !uniform(*s_fail);
    const bool hbias = L.down_bias_off >= 0;
    const int64_t brow = n0 + (lane & 15);
    Tile<MM> tl;
    uint32_t bw = 0;
    if (live) {
        const uint8_t* base = p.pool + slot * L.slot_bytes;
        bw = bias_word(base + (hbias ? L.down_bias_off : 0), L.bias_dtype, hbias ? (int64_t)H : 0, brow);
        tile_load<MM>(tl, base + L.down_off + (n0 / 16) * p.dn_tile, p.dn_tile,
                      base + L.down_scales_off + (n0 / 16) * p.dn_stile, p.dn_stile, lane);
        tile_stash(tl, stash, lane);
    }
    __syncthreads();  // B2
    float yv = 0.0f;
    if (uniform(*s_fail)) {
        yv = __builtin_nanf("");
    } else if (live) {
        const float a =
            tile_dot<MM, 1>(tl, a_source(hs + j * 2 * KT, zero, KT, lane), tables + 128 * j, lane, stash);
        yv = w * (a + bias_word_value(bw, L.bias_dtype, brow));
    }
    if (lane < 16) s_y[wave * 16 + lane] = yv;
    __syncthreads();  // B3
    if (wave == 0 && lane < 16) {
        float sum = 0.0f;
#pragma unroll
        for (int w2 = 0; w2 < WAVES; ++w2) sum += s_y[w2 * 16 + lane];
        store_out(p.y, p.y_dtype, (int64_t)t * H + n0 + lane, sum);
    }
}

// Both roles take MM = the larger piece count of hidden and inter (pieces past a row's end
// read zero).
template <int MM>
__global__ void __launch_bounds__(64 * F_WAVES) __attribute__((amdgpu_waves_per_eu(4, 4))) mxt_fused_kernel(MxtParams p) {
    const int b = (int)blockIdx.x;
    if (b < p.n_gu)
        fused_gate_up<MM>(p, b);
    else
        fused_down<MM>(p, b - p.n_gu);
}

const void* kernel_for_mm(int MM, int which) {
#define TSA_MXT_CASE(M)                                                                   \
    case M:                                                                               \
        return which == 1   ? reinterpret_cast<const void*>(&mxt_down_kernel<M, false>)   \
               : which == 2 ? reinterpret_cast<const void*>(&mxt_fused_kernel<M>)         \
               : which == 3 ? reinterpret_cast<const void*>(&mxt_gate_up_kernel<M, true>) \
               : which == 4 ? reinterpret_cast<const void*>(&mxt_down_kernel<M, true>)    \
                            : reinterpret_cast<const void*>(&mxt_gate_up_kernel<M, false>);
    switch (MM) {
        TSA_MXT_CASE(4)
        TSA_MXT_CASE(8)
        TSA_MXT_CASE(16)
        TSA_MXT_CASE(23)
        TSA_MXT_CASE(24)
        default: return nullptr;
    }
#undef TSA_MXT_CASE
}

int pick_mm(int64_t groups) {
    for (int mm : {4, 8, 16, 23, 24})
        if (groups <= mm) return mm;
    return 0;
}

int64_t al256(int64_t n) { return (n + 255) / 256 * 256; }

}  // namespace

// Workspace bytes of the tiled decode (after the sync area): h per (token, expert) pair, in
// bf16 (two launches) or as the down dot's terms (one launch), then the routed selection
// (int32 slots, float weights).
static int64_t h_bytes(const tsa_expert_layout& L, int64_t T, int k) { return al256(T * k * pair_term_bytes(L.inter)); }
int64_t mxt_ws_bytes(const tsa_expert_layout& L, int64_t T, int k) {
    return h_bytes(L, T, k) + 2 * al256(T * k * 4);
}

// Requirements of the MFMA decode beyond validate_layout, for tiled layouts and (the same
// kernels loading lane by lane) checkpoint-order ones: "" if met.
const char* mxt_unsupported(const tsa_expert_layout& L) {
    if (L.format != TSA_EXPERT_MXFP4 || L.act != TSA_ACT_SWIGLU_OAI) return "tiled layouts need MXFP4 experts with the SwiGLU-OAI activation";
    if (L.hidden % 32 || L.inter % 32) return "tiled layouts need hidden and inter to be multiples of 32";
    if (!pick_mm(mx_tile_groups(L.hidden)) || !pick_mm(mx_tile_groups(L.inter))) return "tiled layouts support hidden, inter <= 3072";
    if ((L.slot_bytes | L.gate_off | L.down_off | L.gate_scales_off | L.down_scales_off) & 15)
        return "tiled layouts need 16-byte aligned slots and matrix offsets";
    if (L.gate_bias_off >= 0 && (L.gate_bias_off | L.down_bias_off) & 15) return "tiled layouts need 16-byte aligned biases";
    return "";
}

// Enqueue the decode of T <= 4 tokens, k <= 16 (the caller checked the layout with
// mxt_unsupported and the pointers' alignment): one launch (mxt_form() 0, sync = the
// workspace's sync area) or two. Unrouted: slots / wts [T, k]; routed: logits [T, E] with
// E <= 256.
int mxt_decode(const tsa_expert_layout& L, const uint8_t* pool, int64_t n_slots, const int32_t* slots,
               const float* wts, const void* logits, int logits_dtype, int mode, const int32_t* expert_slot, int64_t E,
               int32_t* idx_out, float* w_out, int64_t T, int k, const void* x, void* y, int y_dtype, uint8_t* sync,
               uint8_t* ws, int64_t ws_bytes, hipStream_t st) {
    TSA_REQUIRE(T >= 1 && T <= MAXT && k >= 1 && k <= MAXK, TSA_ERR_SHAPE, "tiled decode launch: T %lld, k %d",
                (long long)T, k);
    TSA_REQUIRE(!logits || E <= 256, TSA_ERR_SHAPE, "fused routing supports E <= 256 (got %lld)", (long long)E);
    TSA_REQUIRE(ws_bytes >= mxt_ws_bytes(L, T, k), TSA_ERR_WORKSPACE, "workspace too small for the tiled decode");
    TSA_REQUIRE(L.hidden % 8 == 0 && (reinterpret_cast<uintptr_t>(x) & 15) == 0, TSA_ERR_INVALID_ARG,
                "tiled decode needs 16-byte aligned activations");
    const int ma = pick_mm(mx_tile_groups(L.hidden)), mb = pick_mm(mx_tile_groups(L.inter));
    const bool ck = !L.mx_tiled;  // checkpoint order: the same kernels with lane-wise tile loads
    const void* ka = kernel_for_mm(ma, ck ? 3 : 0);
    const void* kd = kernel_for_mm(mb, ck ? 4 : 1);
    TSA_REQUIRE(ka && kd && L.hidden <= 3072 && L.inter <= 3072, TSA_ERR_SHAPE, "tiled decode: unsupported sizes");

    MxtParams p{};
    p.L = L;
    p.pool = pool;
    p.n_slots = n_slots;
    uint8_t* h = ws;
    const int64_t hb = h_bytes(L, T, k);
    if (logits) {
        p.sel_slot = reinterpret_cast<int32_t*>(h + hb);
        p.sel_w = reinterpret_cast<float*>(h + hb + al256(T * k * 4));
    } else {
        p.sel_slot = const_cast<int32_t*>(slots);
        p.sel_w = const_cast<float*>(wts);
    }
    p.logits = logits;
    p.logits_dtype = logits_dtype;
    p.route_mode = mode;
    p.expert_slot = expert_slot;
    p.E = (int)E;
    p.idx_out = idx_out;
    p.w_out = w_out;
    p.T = (int)T;
    p.k = k;
    p.x = static_cast<const uint16_t*>(x);
    p.y = y;
    p.y_dtype = y_dtype;
    p.h = reinterpret_cast<uint16_t*>(h);
    p.gu_tile = 8 * L.hidden;
    p.gu_stile = mx_tile_scale_bytes(L.hidden);
    p.dn_tile = 8 * L.inter;
    p.dn_stile = mx_tile_scale_bytes(L.inter);

    void* args[] = {&p};
    const int64_t n_gu = T * k * (L.inter / 64), n_dn = T * (L.hidden / 16);
    if (!ck && sync && mxt_form() == 0 && k <= WAVES && L.inter % 64 == 0 && n_gu <= MXT_SYNC_GFLAGS &&
        n_dn <= MXT_SYNC_DFLAGS) {
        const int mm = ma > mb ? ma : mb;
        p.sync = reinterpret_cast<MxtSync*>(sync);
        p.hterm = h;
        p.wait_limit = mxt_wait_limit();
        p.n_gu = (int)n_gu;
        const size_t kp = 128 * (size_t)mm, kt = (kp + 1023) / 1024 * 1024, sb = 256 * (size_t)((mm + 3) / 4);
        const size_t la = F_MISC + 3 * kp + 128 + F_WAVES * sb, lb = F_MISC + 2 * WAVES * kt + kp + WAVES * sb;
        TSA_HIP_CHECK(hipLaunchKernel(kernel_for_mm(mm, 2), dim3((unsigned)(n_gu + n_dn)), dim3(64 * F_WAVES), args,
                                      la > lb ? la : lb, st));
        return TSA_OK;
    }
    const size_t ck_a = ck ? GU_WAVES * (CK_STAGE + 256 * (size_t)((ma + 3) / 4)) : 0;
    const size_t ck_b = ck ? WAVES * (CK_STAGE + 256 * (size_t)((mb + 3) / 4)) : 0;
    const size_t lds_a = 3 * 128 * (size_t)ma + ASC_BYTES + ck_a;
    const size_t lds_b = MISC_LDS + (2 * WAVES + 1) * 128 * (size_t)mb + ck_b;
    TSA_HIP_CHECK(hipLaunchKernel(ka, dim3((unsigned)(T * k * (L.inter / (8 * GU_WAVES)))), dim3(64 * GU_WAVES), args,
                                  lds_a, st));
    TSA_HIP_CHECK(hipLaunchKernel(kd, dim3((unsigned)(T * (L.hidden / 16))), dim3(256), args, lds_b, st));
    return TSA_OK;
}

}  // namespace tsa
