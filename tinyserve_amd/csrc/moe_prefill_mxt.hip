// Batched (prefill) MoE over MXFP4 experts in the 16-row MFMA tile order: the grouped
// expert GEMMs on the matrix cores.
//
// After the (token, expert) assignments are sorted expert-major (group_kernel), each
// expert's rows form one contiguous run of the sorted order, cut into tiles of up to 128
// rows (pf_table_kernel). Two persistent GEMM launches then cover every (row tile, weight
// tile) pair:
//   gate_up: h[i, :] = SwiGLU(x[token(i)] W_gu^T + b_gu), bf16, in sorted order;
//   down:    yk[a, :] = h[i] W_dn^T + b_dn, bf16, by assignment id a = perm[i]
// (bf16 like the reference's per-expert outputs), and a combine pass forms
// y[t] = sum_j w[t, j] yk[t k + j] over j in order, so every output has one writer and the
// result does not depend on scheduling.
//
// GEMM workgroup: 8 waves, a 256-weight-row x 128-token tile; wave (wn, wt) owns 64 rows
// x 64 tokens = 2 x 2 blocks of v_mfma_f32_32x32x16_bf16 (that form issues at the bf16
// peak with 4 independent chains per wave; 16x16x32 needs about 16). K advances in 128-wide
// pieces. Weights are the A operand: the MXFP4 16-row tile order delivers a 16-row piece
// as one contiguous 1 KB, which v_cvt_scalef32_pk_bf16_fp4 expands exactly (scale folded
// in). Activations are the B operand. Both reach LDS by direct buffer-to-LDS loads issued
// ahead of use (weights, which mostly come from HBM or the MALL, 4 pieces ahead in a 5-deep
// ring; activations, which mostly hit L2, 1 piece ahead), with one wait + barrier per piece.
// Workgroups are persistent, one per CU. XCD x (workgroup b runs on XCD b % 8) owns a
// group of row tiles, with all their weight tiles, in row-tile-major order, so the
// workgroups running together on an XCD share a row tile's activations in its L2. The
// table kernel forms the 8 groups to balance an estimated cost (a tile costs 96 + rows, in
// rows: partial row tiles are cheaper, not free), and each group ends on its cheapest row
// tiles. An XCD's workgroups take its tiles one at a time from a per-XCD counter (the next
// one is requested when a tile starts), so they finish together whatever the tiles cost.
//
// Semantics: tinyserve/expert_pipeline.py:166-239 (group by expert, batched forward,
// weighted scatter), tinyserve/_model_hooks.py:380-394 (MXFP4 expert with biases,
// clamped SwiGLU).

#include "fused_common.h"
#include "mfma_tile.h"
#include "fp6_terms.h"

namespace tsa {

int64_t mx_tile_scale_bytes(int64_t K);

namespace {

constexpr int PF_THREADS = 512;
constexpr int PF_BM = 128;                        // sorted rows (tokens) per workgroup tile
constexpr int PF_BN = 256;                        // weight rows per workgroup tile
constexpr int PF_XST = 2;                         // activation stages (mostly L2 hits)
constexpr int PF_WST = 5;                         // weight stages (from HBM / MALL: issued further ahead)
constexpr int PF_XAHEAD = PF_XST - 1;
constexpr int PF_WAHEAD = PF_WST - 1;
static_assert(PF_WAHEAD > PF_XAHEAD && PF_WAHEAD < 5, "weights of piece i must be issued before its activations");
constexpr int PF_XBYTES = PF_BM * 128 * 2;        // a piece of bf16 activations: 32 KB
constexpr int PF_WBYTES = (PF_BN / 16) * 1024;    // a piece of MXFP4 weights: 16 KB
constexpr int PF_SBYTES = (PF_BN / 16) * 256;     // one scale word per lane of every row tile: 4 KB
constexpr int PF_WOFF = PF_XST * PF_XBYTES;
constexpr int PF_SOFF = PF_WOFF + PF_WST * PF_WBYTES;
constexpr int PF_BIAS_OFF = PF_SOFF + 2 * PF_SBYTES;  // the tile's 256 bias values (up to 1 KB)
constexpr int PF_LDS = PF_BIAS_OFF + 1024;            // 153 KB
constexpr int PF_CTR_STRIDE = 32;                 // ints between per-XCD tile counters (one 128-byte line each)
constexpr int PF_CTR_INTS = 2 * 8 * PF_CTR_STRIDE;  // gate_up's 8 counters, then down's
constexpr int PF_HS_GU = 272;   // LDS row stride (bytes) of the staged gate_up outputs: 128 h + 16 B
constexpr int PF_HS_DN = 528;   // ... of the staged down outputs: 256 values + 16 B
static_assert(PF_BM * PF_HS_DN <= PF_LDS, "the staged outputs fit in the stages");
constexpr int PF_COST0 = 96;  // a tile's estimated cost is PF_COST0 + rows (measured: 16 rows ~0.5 x 128 rows)
// fp6 form of the activations (TSA_PREFILL_FP6): a row is a run of records, one per 128-wide
// piece of K: 4 blocks of 32 values, each 24 bytes of hi codes then 24 of lo codes
// (fp6_terms.h), then the 4 hi scale bytes, then 12 bytes of padding (208 = 13 x 16 bytes:
// whole DMA chunks, and a record stride of 52 dwords keeps the operand reads of 8
// consecutive tokens on distinct LDS banks).
constexpr int PF_QREC = 208;
constexpr int PF_QSCALE = 192;
constexpr int PF_QCHUNKS = PF_QREC / 16;
static_assert(PF_BM * PF_QREC <= PF_XBYTES, "a piece of fp6 records fits an activation stage");
constexpr int PF_HS_Q = 528;  // LDS row stride (bytes) of gate_up's fp32 outputs in the fp6 form: 128 h + 16 B
static_assert(PF_BM * PF_HS_Q <= PF_LDS, "the staged fp32 outputs fit in the stages");

struct PfEntry {
    int slot, row0, rows, expert;
};

struct PfGemm {
    tsa_expert_layout L;
    const uint8_t* pool;
    const int* n_entries;     // device: [0] all table entries, [1 + x] .. [2 + x] XCD x's group
    const PfEntry* table;
    const void* src;          // gate_up: x rows gathered through perm; down: h rows in sorted order
    int64_t src_rows;         // rows of src (bounds of its buffer resource)
    int64_t src_stride;       // bytes per src row (bf16: 2 K; fp6 records: 208 MP)
    const int32_t* perm;      // sorted position -> assignment id (token * k + j)
    int* ctr;                 // 8 per-XCD tile counters (stride PF_CTR_STRIDE), zero at launch
    int k;
    uint16_t* out;            // gate_up: h [n, N / 2] (bf16 form); down: yk [T k, N]
    uint8_t* qout;            // gate_up in the fp6 form: h as fp6 records, rows of out_stride bytes
    int64_t out_stride;
    int N, K, NT, MP;         // weight rows, reduction length, tiles along N, pieces along K
    int64_t w_off, s_off, b_off;        // slot offsets of the tiled blocks, tiled scales, bias (< 0: none)
    int64_t tile_bytes, stile_bytes;    // per 16-row tile
};

typedef int v4i __attribute__((ext_vector_type(4)));
typedef float v16f __attribute__((ext_vector_type(16)));

// Raw buffer descriptor (base, num_records bytes; loads past the end return zero), its
// words from the first lane: the copies' "s" operand must sit in scalar registers, which
// the compiler only guarantees for values it can prove wave-uniform.
__device__ __forceinline__ v4i buf_desc(const void* p, uint32_t bytes) {
    const uint64_t a = reinterpret_cast<uint64_t>(p);
    return v4i{__builtin_amdgcn_readfirstlane((int)(uint32_t)a), __builtin_amdgcn_readfirstlane((int)(uint32_t)(a >> 32)),
               __builtin_amdgcn_readfirstlane((int)bytes), 0x00020000};
}

// 16 (or 4) bytes per lane from buffer offset voff straight into LDS at lds + 16 lane (or
// 4 lane): one contiguous 1 KB (256 B) per wave. Issued as inline assembly so that the
// compiler does not place its conservative vmcnt(0) before every later LDS read: the K loop
// waits for exactly what it needs (pf_wait). Loads return in order, so the compiler's own
// waits for its loads can only get stricter, never too weak.
__device__ __forceinline__ void pf_dma(const v4i& r, uint32_t voff, uint32_t lds) {
    asm volatile("s_mov_b32 m0, %2\n\tbuffer_load_dwordx4 %0, %1, 0 offen lds" ::"v"(voff), "s"(r), "s"(lds)
                 : "memory", "m0");
}
__device__ __forceinline__ void pf_dma4(const v4i& r, uint32_t voff, uint32_t lds) {
    asm volatile("s_mov_b32 m0, %2\n\tbuffer_load_dword %0, %1, 0 offen lds" ::"v"(voff), "s"(r), "s"(lds)
                 : "memory", "m0");
}

// This wave's loads except the newest n are complete (and its LDS work), then the
// workgroup barrier: every wave's part of the piece is in LDS, and every wave is done
// reading the stages that are refilled next.
#define PF_WAIT_CASE(n) \
    case n: asm volatile("s_waitcnt vmcnt(" #n ") lgkmcnt(0)\n\ts_barrier" ::: "memory"); break;
__device__ __forceinline__ void pf_wait(int n) {
    switch (n) {  // n above 16 waits for 16 (stricter)
        PF_WAIT_CASE(0) PF_WAIT_CASE(1) PF_WAIT_CASE(2) PF_WAIT_CASE(3) PF_WAIT_CASE(4) PF_WAIT_CASE(5)
        PF_WAIT_CASE(6) PF_WAIT_CASE(7) PF_WAIT_CASE(8) PF_WAIT_CASE(9) PF_WAIT_CASE(10) PF_WAIT_CASE(11)
        PF_WAIT_CASE(12) PF_WAIT_CASE(13) PF_WAIT_CASE(14) PF_WAIT_CASE(15)
        default: asm volatile("s_waitcnt vmcnt(16) lgkmcnt(0)\n\ts_barrier" ::: "memory"); break;
    }
}
#undef PF_WAIT_CASE

// One 128-wide piece of a wave's 64-row x 64-token block on v_mfma_f32_32x32x16_bf16
// (2 x 2 blocks of 32 x 32). K order within the piece: step j (0..7) covers, for lanes
// 32g..32g+31, dword 2g + j%2 of MXFP4 block j/2, so a weight lane (row r, group g) reads
// the 8 contiguous bytes at 16 (16 (j/2) + r%16) + 8g of its 16-row tile, and the
// activation fragment (subtile, j) is one contiguous 1 KB, laid out so by the DMA. NB of
// the 2 token subtiles are live. Lanes whose block starts at or past K get a zero weight
// operand (past the end of a row the bytes belong to the next tile, and the activations
// there are stand-ins).
template <int NB>
__device__ __forceinline__ void pf_piece(v16f (&acc)[2][2], const uint8_t* xs, const uint8_t* ws, const uint8_t* ss,
                                         int mp, int K, int wn, int wt, int lane) {
    const int g = lane >> 5, rr = lane & 31;
    uint2 A[2][4];
    float s[2][4];
#pragma unroll
    for (int rb = 0; rb < 2; ++rb) {
        const int rt = 4 * wn + 2 * rb + (rr >> 4);  // row tile in the workgroup tile
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const int lt = 16 * q + (rr & 15);      // the 16-row tile's lane holding this row's block q
            A[rb][q] = *reinterpret_cast<const uint2*>(ws + rt * 1024 + 16 * lt + 8 * g);
            s[rb][q] = e8m0_to_f32(ss[rt * 256 + 4 * lt + (mp & 3)]);
        }
    }
    if (128 * (mp + 1) > K) {  // the row's last, partial piece
#pragma unroll
        for (int rb = 0; rb < 2; ++rb)
#pragma unroll
            for (int q = 0; q < 4; ++q)
                if (128 * mp + 32 * q >= K) A[rb][q] = make_uint2(0u, 0u);
    }
    // activations: token row (64 wt + 32 b + lane % 32) of the piece, chunk 4 (j / 2) + 2g + j % 2
    // stored at slot chunk ^ (token % 16)
    const uint8_t* xrow = xs + (64 * wt + rr) * 256;
    auto bfrag = [&](int b, int j) {
        const int ch = 4 * (j >> 1) + 2 * g + (j & 1);
        return *reinterpret_cast<const bf16x8*>(xrow + b * 32 * 256 + 16 * (ch ^ (rr & 15)));
    };
    bf16x8 B[2][NB];
#pragma unroll
    for (int b = 0; b < NB; ++b) B[0][b] = bfrag(b, 0);
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        if (j < 7) {
#pragma unroll
            for (int b = 0; b < NB; ++b) B[(j + 1) & 1][b] = bfrag(b, j + 1);
        }
        __builtin_amdgcn_sched_barrier(0);  // the next step's reads go out before this step's MFMAs
#pragma unroll
        for (int rb = 0; rb < 2; ++rb) {
            const uint32_t w = (j & 1) ? A[rb][j >> 1].y : A[rb][j >> 1].x;
            const bf16x8 Af = expand(w, s[rb][j >> 1]);
#pragma unroll
            for (int b = 0; b < NB; ++b)
                acc[rb][b] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(Af, B[j & 1][b], acc[rb][b], 0, 0, 0);
        }
        __builtin_amdgcn_sched_barrier(0);
    }
}

typedef int v8i __attribute__((ext_vector_type(8)));

// acc += A (fp4 weights, e8m0 scale sa) x B (fp6 e2m3 activations, scale byte OPB of sb).
template <int OPB>
__device__ __forceinline__ v16f mfma_f4f6(const v8i& a, const v8i& b, const v16f& c, int sa, int sb) {
    return __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(a, b, c, 4, 2, 0, sa, OPB, sb);
}

// One 128-wide piece of a wave's 64-row x 64-token block on the scaled MFMA
// v_mfma_scale_f32_32x32x64_f8f6f4 (fp4 weights as A, fp6 activation terms as B; 2 x 2
// blocks of 32 x 32, two K-steps of 64, each a hi and a lo product). Lane (q, r) = (lane /
// 32, lane % 32) supplies, for K-step ks, block 2 ks + q of weight row r: the 16 bytes of
// its 16-row tile's lane 16 (2 ks + q) + r % 16 and that lane's scale byte for the piece;
// and of token column r: the block's 24 bytes of hi (or lo) codes and its scale, which the
// instruction takes from byte 2 ks of the scale word shifted down by q bytes. Blocks at
// or past K get a zero weight operand with a unit scale (their activation records are
// zero, but the weight bytes and scales there belong to the next tile).
template <int NB>
__device__ __forceinline__ void pf_piece_q6(v16f (&acc)[2][2], const uint8_t* xs, const uint8_t* ws,
                                            const uint8_t* ss, int mp, int K, int wn, int wt, int lane) {
    const int q = lane >> 5, rr = lane & 31;
    v8i A[2][2];
    int sa[2][2];
#pragma unroll
    for (int rb = 0; rb < 2; ++rb) {
        const int rt = 4 * wn + 2 * rb + (rr >> 4);
#pragma unroll
        for (int ks = 0; ks < 2; ++ks) {
            const int lt = 16 * (2 * ks + q) + (rr & 15);
            const u32x4 w = *reinterpret_cast<const u32x4*>(ws + rt * 1024 + 16 * lt);
            A[rb][ks] = v8i{(int)w[0], (int)w[1], (int)w[2], (int)w[3], 0, 0, 0, 0};
            sa[rb][ks] = ss[rt * 256 + 4 * lt + (mp & 3)];
        }
    }
    if (128 * (mp + 1) > K) {  // the row's last, partial piece
#pragma unroll
        for (int rb = 0; rb < 2; ++rb)
#pragma unroll
            for (int ks = 0; ks < 2; ++ks)
                if (128 * mp + 32 * (2 * ks + q) >= K) {
                    A[rb][ks] = v8i{0, 0, 0, 0, 0, 0, 0, 0};
                    sa[rb][ks] = 127;
                }
    }
    v8i Bh[2][NB], Bl[2][NB];
    int sh[NB], sl[NB];
#pragma unroll
    for (int b = 0; b < NB; ++b) {
        const uint8_t* rec = xs + (64 * wt + 32 * b + rr) * PF_QREC;
        sh[b] = (int)(*reinterpret_cast<const uint32_t*>(rec + PF_QSCALE) >> (8 * q));
        sl[b] = sh[b] - 0x05050505;  // lo scale = hi scale - 5 (every scale byte is >= 5)
#pragma unroll
        for (int ks = 0; ks < 2; ++ks) {
            const uint8_t* blk = rec + 48 * (2 * ks + q);
            const u32x4 d0 = *reinterpret_cast<const u32x4*>(blk);
            const u32x4 d1 = *reinterpret_cast<const u32x4*>(blk + 16);
            const u32x4 d2 = *reinterpret_cast<const u32x4*>(blk + 32);
            Bh[ks][b] = v8i{(int)d0[0], (int)d0[1], (int)d0[2], (int)d0[3], (int)d1[0], (int)d1[1], 0, 0};
            Bl[ks][b] = v8i{(int)d1[2], (int)d1[3], (int)d2[0], (int)d2[1], (int)d2[2], (int)d2[3], 0, 0};
        }
    }
#pragma unroll
    for (int rb = 0; rb < 2; ++rb)
#pragma unroll
        for (int b = 0; b < NB; ++b) acc[rb][b] = mfma_f4f6<0>(A[rb][0], Bh[0][b], acc[rb][b], sa[rb][0], sh[b]);
#pragma unroll
    for (int rb = 0; rb < 2; ++rb)
#pragma unroll
        for (int b = 0; b < NB; ++b) acc[rb][b] = mfma_f4f6<0>(A[rb][0], Bl[0][b], acc[rb][b], sa[rb][0], sl[b]);
#pragma unroll
    for (int rb = 0; rb < 2; ++rb)
#pragma unroll
        for (int b = 0; b < NB; ++b) acc[rb][b] = mfma_f4f6<2>(A[rb][1], Bh[1][b], acc[rb][b], sa[rb][1], sh[b]);
#pragma unroll
    for (int rb = 0; rb < 2; ++rb)
#pragma unroll
        for (int b = 0; b < NB; ++b) acc[rb][b] = mfma_f4f6<2>(A[rb][1], Bl[1][b], acc[rb][b], sa[rb][1], sl[b]);
}

// The K loop of one tile, as a stream of steps s = -PF_WAHEAD .. MP - 1: step s waits for
// and multiplies piece s (s >= 0), then issues the activations of piece s + PF_XAHEAD and
// the weights of piece s + PF_WAHEAD, in that order. The weights of piece i therefore go
// out in an earlier step than its activations, so once this wave's loads up to X(s) are
// complete, W(s) and its scale word are too; the loads newer than X(s) are counted
// exactly (never fewer than issued: a wait for fewer outstanding is only stricter). NB = 0:
// the wave has no live block in this tile and only takes part in the loads and barriers.
template <int NB, bool Q6, class IX, class IW, class WL>
__device__ __forceinline__ void pf_kloop(v16f (&acc)[2][2], IX& issue_x, IW& issue_w, WL& w_loads, int MP, int K,
                                         int wn, int wt, int lane) {
    extern __shared__ __align__(16) uint8_t smem[];
    auto x_loads = [&](int i) { return i >= 0 && i < MP ? 4 : 0; };
    for (int st = -PF_WAHEAD; st < MP; ++st) {
        if (st >= 0) {
            int newer = w_loads(st - PF_XAHEAD + PF_WAHEAD);
#pragma unroll
            for (int u = st - PF_XAHEAD + 1; u < st; ++u) newer += x_loads(u + PF_XAHEAD) + w_loads(u + PF_WAHEAD);
            pf_wait(newer);
        }
        if (st + PF_XAHEAD >= 0 && st + PF_XAHEAD < MP) issue_x(st + PF_XAHEAD);
        if (st + PF_WAHEAD < MP) issue_w(st + PF_WAHEAD);
        if (NB > 0 && st >= 0) {
            const uint8_t* xs = smem + (st % PF_XST) * PF_XBYTES;
            const uint8_t* ws = smem + PF_WOFF + (st % PF_WST) * PF_WBYTES;
            const uint8_t* ss = smem + PF_SOFF + ((st >> 2) & 1) * PF_SBYTES;
            if constexpr (Q6) pf_piece_q6<NB ? NB : 1>(acc, xs, ws, ss, st, K, wn, wt, lane);
            else pf_piece<NB ? NB : 1>(acc, xs, ws, ss, st, K, wn, wt, lane);
        }
    }
}

template <bool GATE_UP, bool Q6>
__global__ void __launch_bounds__(PF_THREADS, 1) pf_gemm_kernel(PfGemm p) {
    extern __shared__ __align__(16) uint8_t smem[];
    const int tid = threadIdx.x, lane = tid & 63, wave = uniform(tid >> 6);
    const int wn = wave & 3, wt = wave >> 2;
    const int g = lane >> 5, rr = lane & 31;
    const int N = p.N, K = p.K, MP = p.MP;
    const int xcd = blockIdx.x & 7, R = gridDim.x >> 3;
    const int m0 = uniform(p.n_entries[1 + xcd]);
    const int total = (uniform(p.n_entries[2 + xcd]) - m0) * p.NT;  // this XCD's tiles
    int* const ctr = p.ctr + PF_CTR_STRIDE * xcd;
    __shared__ int s_next;
    const int W = (int)(p.stile_bytes >> 8);  // scale words per lane
    const uint32_t lds0 = (uint32_t)reinterpret_cast<uintptr_t>(smem);
    const v4i xr = buf_desc(p.src, (uint32_t)(p.src_rows * p.src_stride));

    // The first tile of workgroup b is b / 8; later ones come from the counter (offset by R,
    // so the first R are never handed out twice).
    for (int tl = (int)(blockIdx.x >> 3); tl < total;) {
        const int m = m0 + tl / p.NT, nt = tl % p.NT;
        int grabbed = 0;
        if (tid == 0) grabbed = R + __hip_atomic_fetch_add(ctr, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        const PfEntry e = p.table[m];
        const int slot = uniform(e.slot), row0 = uniform(e.row0), rows = uniform(e.rows);
        const uint8_t* base = p.pool + (int64_t)slot * p.L.slot_bytes;

        // Activation DMA: each instruction copies 4 whole token rows of the piece (4 x 256 B,
        // coalesced): lanes 16 i .. 16 i + 15 carry token 4 (4 w + c) + i (c = 0..3), lane slot
        // s = lane % 16 the row's 16-byte chunk s ^ (token % 16). The swizzle keeps the B
        // fragment reads (one chunk of 32 tokens per lane group) free of bank conflicts.
        // Tokens past the tile's rows re-read token 0's row (their columns are dropped).
        // fp6 form: the piece's 128 records are 13 x 128 chunks of 16 bytes, chunk i at LDS
        // offset 16 i; instruction c of wave w carries chunks 64 (4 w + c) + lane (those past
        // the tile's rows, and the 384 past 128 records, re-read token 0's and land in the
        // unused end of the stage).
        uint32_t xoff[4];
#pragma unroll
        for (int c = 0; c < 4; ++c) {
            int tok, ch = 0;
            if constexpr (Q6) {
                const int ci = 64 * (4 * wave + c) + lane;
                tok = ci / PF_QCHUNKS;
                ch = ci - PF_QCHUNKS * tok;
            } else {
                tok = 16 * wave + 4 * c + (lane >> 4);
            }
            if (tok >= rows) tok = 0;
            const int64_t srow = GATE_UP ? p.perm[row0 + tok] / p.k : row0 + tok;
            xoff[c] = (uint32_t)(srow * p.src_stride + 16 * ch);
        }
        // Weight DMA: wave w fills row tiles 2w, 2w+1 of the workgroup's 16; one resource
        // spans the workgroup's live tiles (tiles past N read zero).
        const int rtw = nt * (PF_BN / 16);
        int nrw = N / 16 - rtw;
        nrw = nrw > PF_BN / 16 ? PF_BN / 16 : nrw;
        const v4i wr = buf_desc(base + p.w_off + (int64_t)rtw * p.tile_bytes, (uint32_t)(nrw * p.tile_bytes));
        const uint32_t tb = (uint32_t)p.tile_bytes;
        // Scale DMA: with the weights of the first piece of every group of 4, word mp / 4 of
        // the same row tiles (chunked lane-major: word w of a lane at 1024 (w / 4) + 4 width
        // lane + 4 (w % 4), width = min(4, W - 4 (w / 4))) into ring slot (mp / 4) % 2.
        const v4i sr = buf_desc(base + p.s_off + (int64_t)rtw * p.stile_bytes, (uint32_t)(nrw * p.stile_bytes));
        const uint32_t sb = (uint32_t)p.stile_bytes;
        auto issue_x = [&](int mp) {
            const uint32_t st = lds0 + (uint32_t)((mp % PF_XST) * PF_XBYTES) + 16 * wave * 256;
            if constexpr (Q6) {
#pragma unroll
                for (int c = 0; c < 4; ++c) pf_dma(xr, xoff[c] + PF_QREC * mp, st + c * 1024);
                return;
            }
#pragma unroll
            for (int c = 0; c < 4; ++c) {
                const int tok = 16 * wave + 4 * c + (lane >> 4);
                int kk = 128 * mp + 8 * ((lane & 15) ^ (tok & 15));
                if (kk >= K) kk = 0;  // stand-in inside the row; its weight operand is zeroed
                pf_dma(xr, xoff[c] + 2 * kk, st + c * 1024);
            }
        };
        auto issue_w = [&](int mp) {  // 2 loads, + 2 scale loads when mp % 4 == 0
            const uint32_t st = lds0 + PF_WOFF + (uint32_t)((mp % PF_WST) * PF_WBYTES);
#pragma unroll
            for (int jj = 0; jj < 2; ++jj)
                pf_dma(wr, (2 * wave + jj) * tb + 1024 * mp + 16 * lane, st + (2 * wave + jj) * 1024);
            if ((mp & 3) == 0) {
                const int w = mp >> 2;
                const int wc = W - 4 * (w >> 2) < 4 ? W - 4 * (w >> 2) : 4;
#pragma unroll
                for (int jj = 0; jj < 2; ++jj)
                    pf_dma4(sr, (2 * wave + jj) * sb + 1024 * (w >> 2) + 4 * wc * lane + 4 * (w & 3),
                            lds0 + PF_SOFF + (w & 1) * PF_SBYTES + (2 * wave + jj) * 256);
            }
        };
        auto w_loads = [&](int mp) { return mp >= 0 && mp < MP ? 2 + ((mp & 3) == 0 ? 2 : 0) : 0; };

        // This wave's block: row tiles rtw + 4wn .. +3 (two 32-row blocks), tokens 64 wt .. +63.
        const int rt0 = rtw + 4 * wn;
        const bool rows_live = rt0 < N / 16;
        int nsub = (rows - 64 * wt + 31) >> 5;
        nsub = nsub < 0 ? 0 : (nsub > 2 ? 2 : nsub);
        const bool active = rows_live && nsub > 0;

        // The tile's bias, copied into LDS now (wave 0, before the K loop's loads, so that every
        // later wait covers it) and read by the epilogue; rows past N read zero (the buffer
        // range check).
        const int bes = p.L.bias_dtype == TSA_F32 ? 4 : 2;
        if (wave == 0 && p.b_off >= 0) {
            const int64_t brows = N - 16 * rtw;
            const v4i br = buf_desc(base + p.b_off + (int64_t)16 * rtw * bes, (uint32_t)(brows > 0 ? brows * bes : 0));
            for (int i = 0; i < bes; ++i) pf_dma4(br, 256 * i + 4 * lane, lds0 + PF_BIAS_OFF + 256 * i);
        }

        v16f acc[2][2];
#pragma unroll
        for (int a = 0; a < 2; ++a)
#pragma unroll
            for (int b = 0; b < 2; ++b)
#pragma unroll
                for (int v = 0; v < 16; ++v) acc[a][b][v] = 0.0f;
        // One K loop per live-subtile count, so the accumulators keep one register home
        // (a per-piece branch made the compiler copy them after every piece).
        if (!active) pf_kloop<0, Q6>(acc, issue_x, issue_w, w_loads, MP, K, wn, wt, lane);
        else if (nsub == 2) pf_kloop<2, Q6>(acc, issue_x, issue_w, w_loads, MP, K, wn, wt, lane);
        else pf_kloop<1, Q6>(acc, issue_x, issue_w, w_loads, MP, K, wn, wt, lane);
        if (tid == 0) s_next = grabbed;
        __syncthreads();  // every wave is done with the last stages before the next tile refills them
        tl = uniform(s_next);  // rewritten only after the next tile's K loop, which has a barrier per piece

        // Epilogue, 1: the outputs (bias added; SwiGLU for gate_up) as bf16 into LDS, one row
        // per token (the stages are free: every wave is past the K loop's last LDS read).
        // acc[rb][b][4u + r] is row 32 rb + 8u + 4g + r of the wave's 64 (r = 0..3), token
        // column 64 wt + 32 b + (lane % 32).
        constexpr int HS = GATE_UP ? (Q6 ? PF_HS_Q : PF_HS_GU) : PF_HS_DN;
        if (active) {
#pragma unroll
            for (int rb = 0; rb < 2; ++rb) {
#pragma unroll
                for (int u = 0; u < 4; ++u) {
                    const int c = 64 * wn + 32 * rb + 8 * u + 4 * g;  // weight row within the workgroup tile
                    if (16 * rtw + c >= N) continue;  // N % 32 == 16: the block's second row tile is past N
                    const v4f bias = p.b_off >= 0 ? bias_value(*reinterpret_cast<const u32x4*>(smem + PF_BIAS_OFF + c * bes),
                                                               p.L.bias_dtype)
                                                  : v4f{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
                    for (int b = 0; b < 2; ++b) {
                        const int tk = 64 * wt + 32 * b + rr;
                        if (b >= nsub || tk >= rows) continue;
                        const v4f v = v4f{acc[rb][b][4 * u], acc[rb][b][4 * u + 1], acc[rb][b][4 * u + 2], acc[rb][b][4 * u + 3]} + bias;
                        if (GATE_UP && Q6)
                            *reinterpret_cast<float2*>(smem + tk * HS + 2 * c) =
                                make_float2(swiglu_oai_fast(p.L, v[0], v[1]), swiglu_oai_fast(p.L, v[2], v[3]));
                        else if (GATE_UP)
                            *reinterpret_cast<uint32_t*>(smem + tk * HS + c) =
                                pack_bf16x2(swiglu_oai_fast(p.L, v[0], v[1]), swiglu_oai_fast(p.L, v[2], v[3]));
                        else
                            *reinterpret_cast<uint2*>(smem + tk * HS + 2 * c) = make_uint2(pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3]));
                    }
                }
            }
        }
        __syncthreads();
        // 2, fp6 form of gate_up: thread (token tk, block bq) turns h[row0 + tk, 128 nt + 32 bq ..]
        // into its fp6 terms, written to record nt of the row (blocks past the row's end as
        // zero codes with a unit scale: the down GEMM multiplies them by zero weights).
        if constexpr (GATE_UP && Q6) {
            const int tk = tid & (PF_BM - 1), bq = tid >> 7;
            if (tk < rows) {
                uint32_t hi[6], lo[6], sc = 127u;
                const int c0 = 128 * nt + 32 * bq;
                if (c0 < N / 2) {
                    float v[32];
#pragma unroll
                    for (int i = 0; i < 8; ++i) {
                        const v4f f = *reinterpret_cast<const v4f*>(smem + tk * HS + 128 * bq + 16 * i);
                        v[4 * i] = f[0];
                        v[4 * i + 1] = f[1];
                        v[4 * i + 2] = f[2];
                        v[4 * i + 3] = f[3];
                    }
                    sc = fp6_terms(v, hi, lo);
                } else {
#pragma unroll
                    for (int d = 0; d < 6; ++d) hi[d] = lo[d] = 0u;
                }
                uint8_t* rec = p.qout + (int64_t)(row0 + tk) * p.out_stride + (int64_t)nt * PF_QREC;
                *reinterpret_cast<uint4*>(rec + 48 * bq) = make_uint4(hi[0], hi[1], hi[2], hi[3]);
                *reinterpret_cast<uint4*>(rec + 48 * bq + 16) = make_uint4(hi[4], hi[5], lo[0], lo[1]);
                *reinterpret_cast<uint4*>(rec + 48 * bq + 32) = make_uint4(lo[2], lo[3], lo[4], lo[5]);
                rec[PF_QSCALE + bq] = (uint8_t)sc;
            }
        } else {
            // 2: whole rows out, 16 bytes (8 values) per lane, consecutive lanes along a row:
            // gate_up h[row0 + tk, 128 nt ..] (256 B a row), down yk[perm[row0 + tk], 256 nt ..] (512 B).
            constexpr int CPR = GATE_UP ? 16 : 32;  // 16-byte chunks per row
            const int ncol = GATE_UP ? N / 2 - 128 * nt : N - 256 * nt;  // live values in the row (multiple of 8)
#pragma unroll
            for (int j = 0; j < PF_BM * CPR / PF_THREADS; ++j) {
                const int i = tid + PF_THREADS * j, tk = i / CPR, ch = i % CPR;
                if (tk >= rows || 8 * ch >= ncol) continue;
                const uint4 v = *reinterpret_cast<const uint4*>(smem + tk * HS + 16 * ch);
                if (GATE_UP) {
                    *reinterpret_cast<uint4*>(p.out + (int64_t)(row0 + tk) * (N / 2) + 128 * nt + 8 * ch) = v;
                } else {
                    const int64_t asg = p.perm[row0 + tk];
                    *reinterpret_cast<uint4*>(p.out + asg * N + 256 * nt + 8 * ch) = v;
                }
            }
        }
        __syncthreads();  // the staged rows are read before the next tile's loads refill the stages
    }
}

// Tile table: expert e with a resident slot and c_e sorted rows gets ceil(c_e / 128)
// entries (slot, first sorted row, rows, e), in 8 contiguous groups, one per XCD of the
// GEMM launches: n_entries[1 + x] .. n_entries[2 + x] for XCD x, n_entries[0] = all. The
// full 128-row entries (experts in order) are cut into 8 contiguous runs, so an expert's
// row tiles stay on few XCDs and share its weights in L2; then the partial ones, largest
// first, each go to the group with the least estimated cost so far (PF_COST0 + rows per
// entry). Within a group the full entries come first, then the partial ones largest first. Equal-row partial entries are ranked in any order: the results do not
// depend on the order. Also zeroes the GEMMs' tile counters. E <= 1024.
__global__ void __launch_bounds__(1024) pf_table_kernel(const int32_t* __restrict__ counts,
                                                        const int32_t* __restrict__ offsets,
                                                        const int32_t* __restrict__ expert_slot, int E,
                                                        int64_t n_slots, int* __restrict__ n_entries,
                                                        PfEntry* __restrict__ table, int* __restrict__ ctr) {
    __shared__ int wsum[16];
    __shared__ int hist[PF_BM];    // partial entries with r rows
    __shared__ int pos[PF_BM];     // rank (offset by the full entries) of the next partial entry with r rows
    __shared__ int prow[1024];     // partial entries by rank: rows
    __shared__ int pgrp[1024], pidx[1024];  // ... group and place among the group's partial entries
    __shared__ int gstart[8], gfull[8];
    const int e = threadIdx.x;
    if (e < PF_CTR_INTS) ctr[e] = 0;
    if (e < PF_BM) hist[e] = 0;
    int slot = -1, c = 0, nt = 0, r = 0, o = 0;
    if (e < E) {  // the three loads go out together
        slot = expert_slot[e];
        c = counts[e];
        o = offsets[e];
        if (slot >= 0 && slot < n_slots) {
            nt = c / PF_BM;
            r = c % PF_BM;
        }
    }
    __syncthreads();  // hist cleared
    if (r > 0) atomicAdd(&hist[r], 1);
    int F;
    const int pre = block_incl_sum(nt, wsum, F);  // inclusive scan of the full entries (its barriers order hist)
    // pos[b] = F + partial entries with more than b rows: F + all of hist - its inclusive
    // prefix sum to b, by wave 0 (lane l: b = 2l, 2l + 1)
    static_assert(PF_BM == 128, "two hist entries per lane of one wave");
    if (e < 64) {
        const int h0 = hist[2 * e], h1 = hist[2 * e + 1];
        int s = h0 + h1;
        for (int d = 1; d < 64; d <<= 1) {
            const int t = __shfl_up(s, d, 64);
            if (e >= d) s += t;
        }
        const int all = __shfl(s, 63, 64);
        pos[2 * e] = F + all - (s - h1);
        pos[2 * e + 1] = F + all - s;
    }
    __syncthreads();
    const int P = pos[0] - F;
    __syncthreads();  // pos[0] is read before the partial entries take ranks (r > 0 never touches it)
    int q = -1;
    if (r > 0) {
        q = atomicAdd(&pos[r], 1) - F;
        prow[q] = r;
    }
    __syncthreads();
    if (e < 64) {  // the groups, by wave 0: lane x < 8 holds group x; P <= E steps of an argmin
        const int x = e;
        const int nf = x < 8 ? F * (x + 1) / 8 - F * x / 8 : 0;
        int cost = x < 8 ? nf * (PF_COST0 + PF_BM) : 0x7FFFFFFF, np = 0;
        int rn = P > 0 ? prow[0] : 0;
        for (int i = 0; i < P; ++i) {
            const int r_i = rn;
            if (i + 1 < P) rn = prow[i + 1];  // read ahead, off the cost dependency
            int key = x < 8 ? (cost << 3) | x : 0x7FFFFFFF;  // the least cost, ties to the lower group
            key = min(key, dpp_i<0xB1, 0xF, 0xF>(key, key));   // quad_perm [1,0,3,2]
            key = min(key, dpp_i<0x4E, 0xF, 0xF>(key, key));   // quad_perm [2,3,0,1]
            key = min(key, dpp_i<0x141, 0xF, 0xF>(key, key));  // row_half_mirror: the other quad of the 8
            if (x == (key & 7)) {
                pgrp[i] = x;
                pidx[i] = np++;
                cost += PF_COST0 + r_i;
            }
        }
        int s = x < 8 ? nf + np : 0;  // exclusive scan over the 8 groups
        for (int d = 1; d < 8; d <<= 1) {
            const int v = __shfl_up(s, d);
            if (x >= d) s += v;
        }
        if (x < 8) {
            gfull[x] = nf;
            gstart[x] = s - nf - np;
            n_entries[1 + x] = s - nf - np;
            if (x == 7) {
                n_entries[9] = s;
                n_entries[0] = s;
            }
        }
    }
    __syncthreads();
    for (int j = 0; j < nt; ++j) {
        const int f = pre - nt + j;  // full entry f: run x with F x / 8 <= f < F (x + 1) / 8
        int x = 0;
#pragma unroll
        for (int y = 1; y < 8; ++y) x += F * y / 8 <= f ? 1 : 0;
        table[gstart[x] + f - F * x / 8] = PfEntry{slot, o + PF_BM * j, PF_BM, e};
    }
    if (q >= 0) {
        const int x = pgrp[q];
        table[gstart[x] + gfull[x] + pidx[q]] = PfEntry{slot, o + PF_BM * nt, r, e};
    }
}

// x [rows, K] bf16 -> fp6 records (rows of MP records; blocks at or past K as zero codes with a
// unit scale). One thread per (row, 32-value block).
__global__ void __launch_bounds__(256) pf_quant_kernel(const uint16_t* __restrict__ x, int64_t rows, int K, int MP,
                                                       uint8_t* __restrict__ out) {
    const int64_t g = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    const int nb = 4 * MP;
    if (g >= rows * nb) return;
    const int64_t r = g / nb;
    const int b = (int)(g - r * nb);
    uint32_t hi[6], lo[6], sc = 127u;
    if (32 * b < K) {
        // a bounded buffer resource over x: no alignment assumption beyond the element's
        const __amdgpu_buffer_rsrc_t xr = __builtin_amdgcn_make_buffer_rsrc(
            const_cast<uint16_t*>(x), (short)0, (int)(rows * K * 2), 0x00020000);
        float v[32];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const u32x4 w = __builtin_bit_cast(
                u32x4, __builtin_amdgcn_raw_buffer_load_b128(xr, (int)((r * K + 32 * b + 8 * i) * 2), 0, 0));
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                v[8 * i + 2 * j] = bf16_bits_to_f32(w[j] & 0xFFFFu);
                v[8 * i + 2 * j + 1] = bf16_bits_to_f32(w[j] >> 16);
            }
        }
        sc = fp6_terms(v, hi, lo);
    } else {
#pragma unroll
        for (int d = 0; d < 6; ++d) hi[d] = lo[d] = 0u;
    }
    uint8_t* rec = out + r * (int64_t)MP * PF_QREC + (int64_t)(b >> 2) * PF_QREC;
    const int bq = b & 3;
    *reinterpret_cast<uint4*>(rec + 48 * bq) = make_uint4(hi[0], hi[1], hi[2], hi[3]);
    *reinterpret_cast<uint4*>(rec + 48 * bq + 16) = make_uint4(hi[4], hi[5], lo[0], lo[1]);
    *reinterpret_cast<uint4*>(rec + 48 * bq + 32) = make_uint4(lo[2], lo[3], lo[4], lo[5]);
    rec[PF_QSCALE + bq] = (uint8_t)sc;
}

// y[t] = sum_j w[t, j] yk[t k + j] over the live assignments, j in order; 8 columns per thread.
__global__ void __launch_bounds__(256) pf_combine_kernel(const uint16_t* __restrict__ yk,
                                                         const int32_t* __restrict__ idx,
                                                         const float* __restrict__ w,
                                                         const int32_t* __restrict__ expert_slot, int64_t E,
                                                         int64_t n_slots, int64_t T, int k, int H, void* y,
                                                         int y_dtype) {
    const int64_t g = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    const int cpr = H / 8;
    if (g >= T * cpr) return;
    const int64_t t = g / cpr;
    const int c = (int)(g % cpr);
    float acc[8] = {0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f};
    // Four assignments at a time: their ids, weights and output rows are loaded together
    // (a dropped assignment's row is read but not used), then the slots, then the sums in
    // j order.
    constexpr int JB = 4;
    for (int j0 = 0; j0 < k; j0 += JB) {
        int e[JB];
        float wj[JB];
        u32x4 v[JB];
#pragma unroll
        for (int jj = 0; jj < JB; ++jj) {
            const int j = j0 + jj;
            e[jj] = j < k ? idx[t * k + j] : -1;
            wj[jj] = j < k ? w[t * k + j] : 0.0f;
            v[jj] = j < k ? *reinterpret_cast<const u32x4*>(yk + (t * k + j) * H + 8 * c) : u32x4{0u, 0u, 0u, 0u};
        }
        bool live[JB];
#pragma unroll
        for (int jj = 0; jj < JB; ++jj) {
            live[jj] = e[jj] >= 0 && e[jj] < E;
            if (live[jj]) {
                const int s = expert_slot[e[jj]];
                live[jj] = s >= 0 && s < n_slots;
            }
        }
#pragma unroll
        for (int jj = 0; jj < JB; ++jj) {
            if (!live[jj]) continue;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                acc[2 * i] += wj[jj] * bf16_bits_to_f32(v[jj][i] & 0xFFFFu);
                acc[2 * i + 1] += wj[jj] * bf16_bits_to_f32(v[jj][i] >> 16);
            }
        }
    }
    if (y_dtype == TSA_BF16) {  // one 16-byte store (H % 8 == 0 keeps it aligned)
        *reinterpret_cast<uint4*>(static_cast<uint16_t*>(y) + t * H + 8 * c) =
            make_uint4(pack_bf16x2(acc[0], acc[1]), pack_bf16x2(acc[2], acc[3]), pack_bf16x2(acc[4], acc[5]),
                       pack_bf16x2(acc[6], acc[7]));
        return;
    }
#pragma unroll
    for (int i = 0; i < 8; ++i) store_out(y, y_dtype, t * H + 8 * c + i, acc[i]);
}

}  // namespace

// ---------------------------------------------------------------- host side

// Whether the tiled MXFP4 grouped-GEMM path covers this call (else the caller uses the
// fused decode kernel token chunk by token chunk).
static int64_t q6_row_bytes(int64_t K) { return (K + 127) / 128 * PF_QREC; }

bool pf_mxt_supported(const tsa_expert_layout& L, int x_dtype, int64_t T, int k) {
    const int64_t n = T * k, lim = (int64_t)1 << 32;
    const bool bf16_ok = T * L.hidden * 2 < lim && n * L.inter * 2 < lim;
    const bool q6_ok = L.prefill_mfma != TSA_PREFILL_FP6 || (T * q6_row_bytes(L.hidden) < lim &&
                                                            n * q6_row_bytes(L.inter) < lim);
    return L.format == TSA_EXPERT_MXFP4 && L.mx_tiled && x_dtype == TSA_BF16 && L.hidden % 16 == 0 &&
           L.inter % 16 == 0 && bf16_ok && q6_ok;
}

static int64_t al256(int64_t v) { return (v + 255) / 256 * 256; }

struct PfWs {
    int64_t counts, offsets, perm, nent, ctr, table, h, xq, yk, total;
};

static PfWs pf_ws_layout(const tsa_expert_layout& L, int64_t T, int k, int64_t E) {
    const int64_t n = T * k;
    PfWs w;
    int64_t o = 0;
    w.counts = o; o += al256(4 * E);
    w.offsets = o; o += al256(4 * (E + 1));
    w.perm = o; o += al256(4 * n);
    w.nent = o; o += 256;
    w.ctr = o; o += al256(4 * PF_CTR_INTS);
    w.table = o; o += al256((int64_t)sizeof(PfEntry) * (n / PF_BM + E + 1));
    const bool q6 = L.prefill_mfma == TSA_PREFILL_FP6;
    w.h = o; o += al256(q6 ? n * q6_row_bytes(L.inter) : 2 * n * L.inter);  // h: fp6 records or bf16
    w.xq = o; o += q6 ? al256(T * q6_row_bytes(L.hidden)) : 0;              // x as fp6 records
    w.yk = o; o += al256(2 * n * L.hidden);
    w.total = o;
    return w;
}

int64_t pf_mxt_workspace_bytes(const tsa_expert_layout& L, int64_t T, int k, int64_t E) {
    return pf_ws_layout(L, T, k, E).total;
}

int launch_group_kernel(const int32_t* idx, int64_t n, int E, int32_t* counts, int32_t* offsets, int32_t* perm,
                        hipStream_t stream, const int32_t* expert_slot = nullptr, int64_t n_slots = 0,
                        int tile_rows = 0, int* n_entries = nullptr, void* table = nullptr);

// y[t] = sum_j w[t, j] yk[t k + j] over the live assignments, j in order (H % 8 == 0).
int pf_combine(const uint16_t* yk, const int32_t* idx, const float* w, const int32_t* expert_slot, int64_t E,
               int64_t n_slots, int64_t T, int k, int H, void* y, int y_dtype, hipStream_t stream) {
    const int64_t threads = T * (H / 8);
    hipLaunchKernelGGL(pf_combine_kernel, dim3((unsigned)((threads + 255) / 256)), dim3(256), 0, stream, yk, idx, w,
                       expert_slot, E, n_slots, T, k, H, y, y_dtype);
    TSA_LAUNCH_CHECK();
    return TSA_OK;
}

int pf_mxt_prefill(const tsa_expert_layout& L, const uint8_t* pool, int64_t n_slots, const int32_t* expert_slot,
                   int64_t E, const int32_t* idx, const float* weights, int64_t T, int k, const uint16_t* x, void* y,
                   int y_dtype, uint8_t* ws, hipStream_t stream) {
    const PfWs w = pf_ws_layout(L, T, k, E);
    int32_t* counts = reinterpret_cast<int32_t*>(ws + w.counts);
    int32_t* offsets = reinterpret_cast<int32_t*>(ws + w.offsets);
    int32_t* perm = reinterpret_cast<int32_t*>(ws + w.perm);
    int* nent = reinterpret_cast<int*>(ws + w.nent);
    int* ctr = reinterpret_cast<int*>(ws + w.ctr);
    PfEntry* table = reinterpret_cast<PfEntry*>(ws + w.table);
    uint16_t* h = reinterpret_cast<uint16_t*>(ws + w.h);
    uint16_t* yk = reinterpret_cast<uint16_t*>(ws + w.yk);
    const int H = (int)L.hidden, I = (int)L.inter;

    int rc = launch_group_kernel(idx, T * k, (int)E, counts, offsets, perm, stream);
    if (rc) return rc;
    hipLaunchKernelGGL(pf_table_kernel, dim3(1), dim3(1024), 0, stream, counts, offsets, expert_slot, (int)E, n_slots,
                       nent, table, ctr);
    TSA_LAUNCH_CHECK();

    for (const void* f : {reinterpret_cast<const void*>(pf_gemm_kernel<true, false>),
                          reinterpret_cast<const void*>(pf_gemm_kernel<false, false>),
                          reinterpret_cast<const void*>(pf_gemm_kernel<true, true>),
                          reinterpret_cast<const void*>(pf_gemm_kernel<false, true>)}) {
        const hipError_t e = ensure_dynamic_lds(f, PF_LDS);
        TSA_REQUIRE(e == hipSuccess, TSA_ERR_HIP, "hipFuncSetAttribute(LDS %d): %s", PF_LDS, hipGetErrorString(e));
    }
    const int grid = (num_cus() / 8) * 8;
    PfGemm g{};
    g.L = L;
    g.pool = pool;
    g.n_entries = nent;
    g.table = table;
    g.perm = perm;
    g.ctr = ctr;
    g.k = k;
    const bool q6 = L.prefill_mfma == TSA_PREFILL_FP6;
    uint8_t* xq = ws + w.xq;
    if (q6) {  // x as fp6 records
        const int64_t threads = T * 4 * ((H + 127) / 128);
        hipLaunchKernelGGL(pf_quant_kernel, dim3((unsigned)((threads + 255) / 256)), dim3(256), 0, stream, x, T, H,
                           (H + 127) / 128, xq);
        TSA_LAUNCH_CHECK();
    }
    // gate_up: [2I, H] -> h
    g.src = q6 ? static_cast<const void*>(xq) : static_cast<const void*>(x);
    g.src_rows = T;
    g.src_stride = q6 ? q6_row_bytes(H) : 2 * (int64_t)H;
    g.out = h;
    g.qout = ws + w.h;
    g.out_stride = q6_row_bytes(I);
    g.N = 2 * I;
    g.K = H;
    g.NT = (2 * I + PF_BN - 1) / PF_BN;
    g.MP = (H + 127) / 128;
    g.w_off = L.gate_off;
    g.s_off = L.gate_scales_off;
    g.b_off = L.gate_bias_off;
    g.tile_bytes = 16 * (int64_t)H / 2;
    g.stile_bytes = mx_tile_scale_bytes(H);
    if (q6) hipLaunchKernelGGL((pf_gemm_kernel<true, true>), dim3(grid), dim3(PF_THREADS), PF_LDS, stream, g);
    else hipLaunchKernelGGL((pf_gemm_kernel<true, false>), dim3(grid), dim3(PF_THREADS), PF_LDS, stream, g);
    TSA_LAUNCH_CHECK();
    // down: [H, I] -> yk
    g.src = ws + w.h;
    g.src_rows = T * k;
    g.src_stride = q6 ? q6_row_bytes(I) : 2 * (int64_t)I;
    g.ctr = ctr + 8 * PF_CTR_STRIDE;
    g.out = yk;
    g.N = H;
    g.K = I;
    g.NT = (H + PF_BN - 1) / PF_BN;
    g.MP = (I + 127) / 128;
    g.w_off = L.down_off;
    g.s_off = L.down_scales_off;
    g.b_off = L.down_bias_off;
    g.tile_bytes = 16 * (int64_t)I / 2;
    g.stile_bytes = mx_tile_scale_bytes(I);
    if (q6) hipLaunchKernelGGL((pf_gemm_kernel<false, true>), dim3(grid), dim3(PF_THREADS), PF_LDS, stream, g);
    else hipLaunchKernelGGL((pf_gemm_kernel<false, false>), dim3(grid), dim3(PF_THREADS), PF_LDS, stream, g);
    TSA_LAUNCH_CHECK();

    return pf_combine(yk, idx, weights, expert_slot, E, n_slots, T, k, H, y, y_dtype, stream);
}

}  // namespace tsa
