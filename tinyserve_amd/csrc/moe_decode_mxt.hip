// MoE decode over MXFP4 experts stored in the 16-row tile order (mx_tile.hip): routing,
// gate_up, clamped SwiGLU, down and the weighted top-k sum in two launches, each a pure
// weight stream. Every weight byte is read by contiguous 1 KB wave loads and fed to the
// matrix cores as it arrives, still in fp4.
//
// Arithmetic. One 1 KB piece m of a 16-row tile is the B operand of one
// v_mfma_f32_16x16x128_f8f6f4 (fp4 e2m1, no conversion): lane 16q+i holds block 4m+q of
// row i, which is exactly that instruction's fp4 operand layout (column i, K = 32q..32q+31).
// The A operand carries the activation vector v (x for gate_up, h for down) in fp8 e4m3,
// block-diagonally: A row 4r+b holds term r of v restricted to block b of the piece (zero
// elsewhere), so D[4r+b][i] = sum over block b of e2m1(i, k) * term_r(k), one partial dot per
// (row, block) with the block scale not yet applied. The lane holding D[4r+b][i] multiplies
// it by the e8m0 scale of (row i, block 4m+b) and accumulates. The activation is split into
// two e4m3 terms, v*s = hi + lo, with hi = e4m3(v*s) and lo = e4m3(v*s - hi): for a bf16 v
// the pair is exact (hi keeps 4 significant bits, lo the remaining 4) unless v is more than
// 2^10 below the scaled maximum, so the products are those of the reference's bf16
// arithmetic. The scale s is a power of two: per token for x (from max |x|), fixed for h
// (|h| <= (limit + 1) * limit after the clamped SwiGLU).
//
// Launch 1 (gate_up): workgroup (kb, pair) multiplies 64 gate_up rows of the pair's expert
//   (one 16-row tile per wave) by x of the pair's token; bias, clamped SwiGLU, h rounded to
//   bf16 (the reference runs its experts in bf16) and written to the workspace as its two
//   fp8 terms. A routed launch selects the experts in every workgroup (one wave, from the
//   token's logits); the first workgroup of each token also writes the selection.
// Launch 2 (down): workgroup (token, 16 output rows): wave j multiplies expert j's 16-row
//   down tile by h(token, j); the waves' weighted rows are summed in a fixed order in LDS
//   (one writer per output, deterministic).
// No workgroup waits for another: stream order between the launches is the only
// synchronisation, so the grid needs no co-residency and the workspace carries no state
// from one call to the next.
//
// Semantics: tinyserve/_model_hooks.py:380-394 (MXFP4 expert with biases, clamped
// SwiGLU), :456-473 (routing), tinyserve/csrc/expert_loop.cpp:83-121 (weighted sum).
#include "fused_common.h"
#include "mfma_tile.h"

namespace tsa {

int64_t mx_tile_groups(int64_t K);
int64_t mx_tile_scale_bytes(int64_t K);

namespace {

constexpr int MAXT = FUSED_MAXT;
constexpr int MAXK = FUSED_MAXK;
constexpr int WAVES = 4;
constexpr int MISC_LDS = 1024;  // slot/weight tables, per-wave maxima and rows

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
    uint8_t* h;  // [T k][2][I] fp8 terms of h * h_scale (hi, then lo)
    int64_t gu_tile, gu_stile, dn_tile, dn_stile;  // bytes per 16-row tile: blocks, scale words
    float h_scale, h_inv;
};

// A wave's 16-row tile: MM pieces of 1 KB and the scale words (byte m%4 of word m/4).
// Buffer resources span exactly the tile, so pieces past a short row (K < 128 MM) read
// zero without touching memory.
template <int MM>
struct Tile {
    static constexpr int MS = (MM + 3) / 4;
    static constexpr int CHUNKS = (MS + 3) / 4;  // scale loads
    u32x4 q[MM];
    uint32_t sc[MS];
};

// The scale words (W per lane, W = stile_bytes / 256 <= MS) come in lane-major chunks of
// up to 4 words: one 16-byte load per chunk, bounded to the tile's scale area. A load
// wider than a lane's part of a chunk picks up the next lane's words; words >= W are
// zeroed, so they can only meet the zero blocks of groups past the row end. Issues exactly
// CHUNKS + MM buffer loads, in that order.
template <int MM>
__device__ __forceinline__ void tile_load(Tile<MM>& tl, const uint8_t* blocks, int64_t tile_bytes,
                                          const uint8_t* scales, int64_t stile_bytes, int lane) {
    const __amdgpu_buffer_rsrc_t rb =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t*>(blocks), (short)0, (int)tile_bytes, 0x00020000);
    const __amdgpu_buffer_rsrc_t rs =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t*>(scales), (short)0, (int)stile_bytes, 0x00020000);
    const int W = (int)(stile_bytes >> 8);
#pragma unroll
    for (int c = 0; c < Tile<MM>::CHUNKS; ++c) {
        const int wc = W - 4 * c < 4 ? (W - 4 * c > 0 ? W - 4 * c : 0) : 4;  // this chunk's words per lane
        const u32x4 v = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rs, 4 * wc * lane, 1024 * c, 0));
#pragma unroll
        for (int d = 0; d < 4 && 4 * c + d < Tile<MM>::MS; ++d) tl.sc[4 * c + d] = 4 * c + d < W ? v[d] : 0u;
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

// s[b] = word v of lane 16 b + (lane & 15): the scales of blocks 4m + b of the lane's
// column, gathered from the four lane groups (v_permlane32_swap swaps the upper half of
// its first operand with the lower half of its second, v_permlane16_swap likewise within
// each 32-lane half).
__device__ __forceinline__ void gather_groups(uint32_t v, uint32_t s[4]) {
    const auto h = __builtin_amdgcn_permlane32_swap(v, v, false, false);        // groups g&1, (g&1)+2
    const auto a = __builtin_amdgcn_permlane16_swap(h[0], h[0], false, false);  // groups 0, 1
    const auto b = __builtin_amdgcn_permlane16_swap(h[1], h[1], false, false);  // groups 2, 3
    s[0] = a[0];
    s[1] = a[1];
    s[2] = b[0];
    s[3] = b[1];
}

// One piece's scale bytes: byte e of word s[b] -> 2^(e - 127) as a float (e = 0 reads as 0).
__device__ __forceinline__ void scale_fma(float (&acc)[4], const v4f& d, const uint32_t (&s)[4], int pp) {
#pragma unroll
    for (int b = 0; b < 4; ++b) acc[b] = fmaf(d[b], __uint_as_float(((s[b] >> (8 * pp)) & 255u) << 23), acc[b]);
}

// sum over the tile's K of W[i][k] * term_g(k) in lane 16 g + i (g = 0, 1; lanes 32..63 hold
// zero rows), W the lane's 16-row tile and term_g the g-th fp8 term of a vector in LDS. a_lo
// and a_hi are the lane's A-operand sources (a_sources); four accumulators (one per block
// position) keep the FMAs independent.
template <int MM>
__device__ __forceinline__ float tile_dot(const Tile<MM>& tl, const uint8_t* a_lo, const uint8_t* a_hi) {
    float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    u32x4 lo = *reinterpret_cast<const u32x4*>(a_lo), hi = *reinterpret_cast<const u32x4*>(a_hi);
    uint32_t s[4];
    gather_groups(tl.sc[0], s);
    v4f dp = v4f{0.0f, 0.0f, 0.0f, 0.0f};
    // Software pipeline: piece m's MFMA is issued, piece m+1's A operand is read into the
    // registers it has just consumed, and piece m-1's result is scaled and accumulated while
    // the MFMA runs. The empty asm statement pins the accumulators at the end of each piece:
    // without it the compiler sinks every piece's scaling to the end of the loop and keeps
    // all MM results live (and spills).
#pragma unroll
    for (int m = 0; m < MM; ++m) {
        const v8i A = {(int)lo[0], (int)lo[1], (int)lo[2], (int)lo[3], (int)hi[0], (int)hi[1], (int)hi[2], (int)hi[3]};
        const v8i B = {(int)tl.q[m][0], (int)tl.q[m][1], (int)tl.q[m][2], (int)tl.q[m][3], 0, 0, 0, 0};
        // fp8 e4m3 A (cbsz 0) x fp4 e2m1 B (blgp 4); zero scale operands select the unscaled
        // instruction
        const v4f d = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(A, B, v4f{0.0f, 0.0f, 0.0f, 0.0f}, 0, 4, 0, 0,
                                                                      0, 0);
        if (m + 1 < MM) {
            lo = *reinterpret_cast<const u32x4*>(a_lo + 128 * (m + 1));
            hi = *reinterpret_cast<const u32x4*>(a_hi + 128 * (m + 1));
        }
        if (m > 0) {
            scale_fma(acc, dp, s, (m - 1) % 4);
            if (m % 4 == 0) gather_groups(tl.sc[m / 4], s);  // piece m's word, after piece m-1 used the last
        }
        asm volatile("" : "+v"(acc[0]), "+v"(acc[1]), "+v"(acc[2]), "+v"(acc[3]));
        dp = d;
        __builtin_amdgcn_sched_barrier(0);
    }
    scale_fma(acc, dp, s, (MM - 1) % 4);
    return (acc[0] + acc[1]) + (acc[2] + acc[3]);
}

// The lane's A-operand sources for a vector whose two terms start at `terms` (term r at
// terms + r * kp, zero past the vector's end): row 4r+b of A, K slice kq = lane / 16. Bytes
// 0..15 of the operand are K = 16 kq .. 16 kq + 15 (block kq / 2), bytes 16..31 are
// K = 64 + 16 kq .. (block 2 + kq / 2); a lane whose row and slice do not meet reads a zero
// area instead (rows 8..15 are all zero).
__device__ __forceinline__ void a_sources(const uint8_t* terms, const uint8_t* zero, int kp, int lane,
                                          const uint8_t*& lo, const uint8_t*& hi) {
    const int row = lane & 15, r = row >> 2, b = row & 3, kq = lane >> 4;
    const uint8_t* src = terms + r * kp + 32 * b + 16 * (kq & 1);
    const bool live = r < 2;
    lo = live && b < 2 && (kq >> 1) == b ? src : zero;
    hi = live && b >= 2 && (kq >> 1) == b - 2 ? src : zero;
}

// 16 bytes per lane from buffer offset voff straight into LDS at lds + 16 lane (one 1 KB
// wave transfer). Issued from inline assembly: the compiler does not count these loads, so
// the caller waits for them with its own s_waitcnt before reading the LDS area.
__device__ __forceinline__ void lds_dma16(const __amdgpu_buffer_rsrc_t& r, uint32_t voff, uint32_t lds) {
    asm volatile("s_mov_b32 m0, %2\n\tbuffer_load_dwordx4 %0, %1, 0 offen lds" ::"v"(voff), "s"(r), "s"(lds)
                 : "memory", "m0");
}

// Two e4m3 terms of v * s: hi = RNE(v s), lo = RNE(v s - hi) (OCP e4m3; |v s| < 448).
__device__ __forceinline__ void fp8_terms(float v0, float v1, uint32_t& hi2, uint32_t& lo2) {
    const int h = __builtin_amdgcn_cvt_pk_fp8_f32(v0, v1, 0, false);
    const float r0 = v0 - __builtin_amdgcn_cvt_f32_fp8(h, 0), r1 = v1 - __builtin_amdgcn_cvt_f32_fp8(h, 1);
    hi2 = (uint32_t)h & 0xFFFFu;
    lo2 = (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(r0, r1, 0, false) & 0xFFFFu;
}

// Zero bytes [from, to) of an LDS area (16-byte multiples), spread over nthr threads.
__device__ __forceinline__ void lds_zero(uint8_t* a, int from, int to, int me, int nthr) {
    for (int o = from + 16 * me; o < to; o += 16 * nthr) *reinterpret_cast<u32x4*>(a + o) = u32x4{0u, 0u, 0u, 0u};
}

constexpr int XCH = 3072 / 8 / (64 * (WAVES - 1));  // x chunks (8 values) per loading thread, H <= 3072

// ---- launch 1: gate_up tiles of one (token, expert) pair, SwiGLU, h terms to the workspace.
// Workgroup b: pair b % (T k), 64-row block b / (T k) (pair-major, so neighbouring
// workgroups stream different experts).
template <int MM>
__global__ void __launch_bounds__(256, 2) mxt_gate_up_kernel(MxtParams p) {
    extern __shared__ __align__(16) uint8_t smem[];
    constexpr int KP = 128 * MM;  // padded vector length
    const int tid = threadIdx.x, lane = tid & 63, wave = uniform(tid >> 6);
    const tsa_expert_layout& L = p.L;
    const int H = (int)L.hidden, I = (int)L.inter, k = p.k;
    const int pairs = p.T * k;
    const int kb = (int)blockIdx.x / pairs, pr = (int)blockIdx.x % pairs, t = pr / k;
    int* s_slot = reinterpret_cast<int*>(smem);                     // [MAXT*MAXK]
    float* s_w = reinterpret_cast<float*>(smem + 4 * MAXT * MAXK);  // [MAXT*MAXK]
    float* s_xmax = reinterpret_cast<float*>(smem + 8 * MAXT * MAXK);  // [WAVES]
    uint8_t* vec = smem + MISC_LDS;  // x terms [2][KP], then a zero area [KP]
    uint8_t* zero = vec + 2 * KP;

    // ---- prologue: waves 1..3 load x of token t into registers (every load issued before
    // the first is used) and take its max |x|; wave 0 selects the token's experts and clears
    // the terms' padding and the zero area.
    u32x4 xr[XCH];
    if (wave > 0) {
        const int me = tid - 64;
        const uint16_t* xt = p.x + (int64_t)t * H;
#pragma unroll
        for (int i = 0; i < XCH; ++i) {
            const int c = me + 64 * (WAVES - 1) * i;
            xr[i] = c < H / 8 ? *reinterpret_cast<const u32x4*>(xt + 8 * c) : u32x4{0u, 0u, 0u, 0u};
        }
        float mx = 0.0f;
#pragma unroll
        for (int i = 0; i < XCH; ++i)
#pragma unroll
            for (int d = 0; d < 4; ++d)
                mx = fmaxf(mx, fmaxf(fabsf(bf16_bits_to_f32(xr[i][d] & 0xFFFFu)), fabsf(bf16_bits_to_f32(xr[i][d] >> 16))));
        mx = wave_max_u(mx);
        if (lane == 0) s_xmax[wave] = mx;
    } else {
        if (p.logits) {
            int es[4];
#pragma unroll
            for (int j = 0; j < 4; ++j) es[j] = p.expert_slot[min(lane + 64 * j, p.E - 1)];
            const int sel = route_token(p, t, lane, es, s_slot, s_w);
            if (kb == 0 && pr % k == 0 && lane < k) {  // the token's first workgroup publishes the selection
                p.sel_slot[t * k + lane] = s_slot[t * k + lane];
                p.sel_w[t * k + lane] = s_w[t * k + lane];
                if (p.idx_out) {
                    p.idx_out[t * k + lane] = sel;
                    p.w_out[t * k + lane] = s_w[t * k + lane];
                }
            }
        } else if (lane == 0) {
            s_slot[pr] = p.sel_slot[pr];
        }
        lds_zero(vec, H, KP, lane, 64);
        lds_zero(vec + KP, H, KP, lane, 64);
        lds_zero(zero, 0, KP, lane, 64);
    }
    __syncthreads();

    // ---- the wave's gate_up tile: rows row0 .. row0 + 15 of the pair's expert
    const int64_t slot = uniform(s_slot[pr]);
    const bool live = slot >= 0 && slot < p.n_slots;
    const int64_t row0 = (int64_t)kb * 64 + 16 * wave;
    const uint8_t* base = p.pool + (live ? slot : 0) * L.slot_bytes;
    const bool hbias = L.gate_bias_off >= 0;
    Tile<MM> tl;
    u32x4 braw = u32x4{0u, 0u, 0u, 0u};
    if (live) {
        if (hbias) braw = bias_raw(base + L.gate_bias_off, L.bias_dtype, 2 * (int64_t)I, row0 + (lane & 15));
        const int64_t tile = row0 / 16;
        tile_load<MM>(tl, base + L.gate_off + tile * p.gu_tile, p.gu_tile, base + L.gate_scales_off + tile * p.gu_stile,
                      p.gu_stile, lane);
    }
    // x terms: scale 2^(7 - e), e = exponent of max |x| (scaled maximum in [128, 256))
    const float mx = fmaxf(fmaxf(s_xmax[1], s_xmax[2]), s_xmax[3]);
    int e = (int)((__float_as_uint(mx) >> 23) & 255u) - 127;
    e = mx > 0.0f ? min(max(e, -100), 100) : 0;
    if (wave > 0) {
        const float sc = __uint_as_float((uint32_t)(127 + 7 - e) << 23);
#pragma unroll
        for (int i = 0; i < XCH; ++i) {
            const int c = tid - 64 + 64 * (WAVES - 1) * i;
            if (c < H / 8) {
                uint32_t hw[4], lw[4];
#pragma unroll
                for (int d = 0; d < 4; ++d) {
                    uint32_t h2, l2;
                    fp8_terms(bf16_bits_to_f32(xr[i][d] & 0xFFFFu) * sc, bf16_bits_to_f32(xr[i][d] >> 16) * sc, h2, l2);
                    hw[d] = h2;
                    lw[d] = l2;
                }
                *reinterpret_cast<uint2*>(vec + 8 * c) = uint2{hw[0] | (hw[1] << 16), hw[2] | (hw[3] << 16)};
                *reinterpret_cast<uint2*>(vec + KP + 8 * c) = uint2{lw[0] | (lw[1] << 16), lw[2] | (lw[3] << 16)};
            }
        }
    }
    __syncthreads();
    if (!live) return;  // a dead pair's h is never read

    const uint8_t *a_lo, *a_hi;
    a_sources(vec, zero, KP, lane, a_lo, a_hi);
    const float a = tile_dot<MM>(tl, a_lo, a_hi);
    const auto sw = __builtin_amdgcn_permlane16_swap(__float_as_uint(a), __float_as_uint(a), false, false);
    const float x_inv = __uint_as_float((uint32_t)(127 - 7 + e) << 23);
    const float bias = hbias ? bias_value(braw, L.bias_dtype)[0] : 0.0f;
    const float tot = (a + __uint_as_float(sw[1])) * x_inv + bias;  // lanes 0..15: row row0 + lane
    // rows alternate gate, up: lane 2r holds h[row0 / 2 + r]
    const float up = __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(tot), 0xB1, 0xF, 0xF, false));
    const float hv = bf16_bits_to_f32(f32_to_bf16_bits(swiglu_oai(L, tot, up))) * p.h_scale;
    uint32_t hi, lo;
    fp8_terms(hv, 0.0f, hi, lo);
    // lanes 0 and 8 gather four values each and store 4 bytes per term
    const uint32_t hb = (hi & 255u) | ((lo & 255u) << 8);
    const uint32_t b1 = (uint32_t)__shfl_down((int)hb, 2), b2 = (uint32_t)__shfl_down((int)hb, 4),
                   b3 = (uint32_t)__shfl_down((int)hb, 6);
    if (lane == 0 || lane == 8) {
        const uint32_t ph = (hb & 255u) | ((b1 & 255u) << 8) | ((b2 & 255u) << 16) | ((b3 & 255u) << 24);
        const uint32_t pl = (hb >> 8) | ((b1 >> 8) << 8) | ((b2 >> 8) << 16) | ((b3 >> 8) << 24);
        uint8_t* dst = p.h + (int64_t)pr * 2 * I + row0 / 2 + (lane >> 1);
        *reinterpret_cast<uint32_t*>(dst) = ph;
        *reinterpret_cast<uint32_t*>(dst + I) = pl;
    }
}

// ---- launch 2: down tiles of every selected expert of one token, weighted sum in a fixed
// order. Workgroup b: token b / (H / 16), output rows 16 (b % (H / 16)) .. + 15.
template <int MM>
__global__ void __launch_bounds__(256, 2) mxt_down_kernel(MxtParams p) {
    extern __shared__ __align__(16) uint8_t smem[];
    constexpr int KP = 128 * MM;                   // padded vector length
    constexpr int TPB = (KP + 1023) / 1024 * 1024;  // bytes per h term in LDS (whole 1 KB transfers)
    const int tid = threadIdx.x, lane = tid & 63, wave = uniform(tid >> 6);
    const tsa_expert_layout& L = p.L;
    const int H = (int)L.hidden, I = (int)L.inter, k = p.k;
    const int RB = H / 16;
    const int t = (int)blockIdx.x / RB;
    const int64_t n0 = (int64_t)((int)blockIdx.x % RB) * 16;
    float* s_y = reinterpret_cast<float*>(smem);  // [WAVES][16]
    uint8_t* hs = smem + MISC_LDS + wave * 2 * TPB;  // this wave's h terms
    uint8_t* zero = smem + MISC_LDS + WAVES * 2 * TPB;
    const uint32_t hs_lds = (uint32_t)reinterpret_cast<uintptr_t>(hs);
    const bool hbias = L.down_bias_off >= 0;
    const int rounds = (k + WAVES - 1) / WAVES;

    float yv = 0.0f;  // lanes 0..15: row n0 + lane, this wave's weighted experts
    for (int rd = 0; rd < rounds; ++rd) {
        const int j = rd * WAVES + wave;
        const int64_t slot = j < k ? uniform(p.sel_slot[t * k + j]) : -1;
        const float w = j < k ? p.sel_w[t * k + j] : 0.0f;
        const bool live = slot >= 0 && slot < p.n_slots;
        const uint8_t* base = p.pool + (live ? slot : 0) * L.slot_bytes;
        Tile<MM> tl;
        u32x4 braw = u32x4{0u, 0u, 0u, 0u};
        if (live) {
            // h(t, j) first, straight into LDS (each term zero-filled to TPB by the buffer
            // bound), then the bias and the tile: CHUNKS + MM + 1 loads younger than the DMA
            const uint8_t* src = p.h + (int64_t)(t * k + j) * 2 * I;
#pragma unroll
            for (int r = 0; r < 2; ++r) {
                const __amdgpu_buffer_rsrc_t rh =
                    __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t*>(src + r * I), (short)0, I, 0x00020000);
#pragma unroll
                for (int i = 0; i < TPB / 1024; ++i)
                    lds_dma16(rh, (uint32_t)(1024 * i + 16 * lane), hs_lds + (uint32_t)(r * TPB + 1024 * i));
            }
            braw = bias_raw(base + (hbias ? L.down_bias_off : 0), L.bias_dtype, hbias ? (int64_t)H : 0,
                            n0 + (lane & 15));
            tile_load<MM>(tl, base + L.down_off + (n0 / 16) * p.dn_tile, p.dn_tile,
                          base + L.down_scales_off + (n0 / 16) * p.dn_stile, p.dn_stile, lane);
        }
        if (rd == 0) {
            lds_zero(zero, 0, KP, tid, 256);
            __syncthreads();
        }
        if (live) {
            asm volatile("s_waitcnt vmcnt(%0)" ::"n"(Tile<MM>::CHUNKS + MM + 1) : "memory");
            const uint8_t *a_lo, *a_hi;
            a_sources(hs, zero, TPB, lane, a_lo, a_hi);
            const float a = tile_dot<MM>(tl, a_lo, a_hi);
            const auto sw = __builtin_amdgcn_permlane16_swap(__float_as_uint(a), __float_as_uint(a), false, false);
            // used unconditionally (zero without a bias: the load's bound is 0), so the load
            // stays and the count above holds
            const float bias = bias_value(braw, L.bias_dtype)[0];
            yv += w * ((a + __uint_as_float(sw[1])) * p.h_inv + bias);
        }
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

const void* kernel_for_mm(int MM, bool down) {
#define TSA_MXT_CASE(M)                                                                  \
    case M:                                                                              \
        return down ? reinterpret_cast<const void*>(&mxt_down_kernel<M>)                 \
                    : reinterpret_cast<const void*>(&mxt_gate_up_kernel<M>);
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

// Workspace bytes of the tiled decode (after the header): h terms, 2 inter bytes per
// (token, expert) pair, then the routed selection (int32 slots, float weights).
int64_t mxt_ws_bytes(const tsa_expert_layout& L, int64_t T, int k) {
    return al256(T * k * 2 * L.inter) + 2 * al256(T * k * 4);
}

// Requirements of the tiled path beyond validate_layout: "" if met.
const char* mxt_unsupported(const tsa_expert_layout& L) {
    if (L.format != TSA_EXPERT_MXFP4 || L.act != TSA_ACT_SWIGLU_OAI) return "tiled layouts need MXFP4 experts with the SwiGLU-OAI activation";
    if (L.hidden % 32 || L.inter % 32) return "tiled layouts need hidden and inter to be multiples of 32";
    if (!pick_mm(mx_tile_groups(L.hidden)) || !pick_mm(mx_tile_groups(L.inter))) return "tiled layouts support hidden, inter <= 3072";
    if ((L.slot_bytes | L.gate_off | L.down_off | L.gate_scales_off | L.down_scales_off) & 15)
        return "tiled layouts need 16-byte aligned slots and matrix offsets";
    if (L.gate_bias_off >= 0 && (L.gate_bias_off | L.down_bias_off) & 15) return "tiled layouts need 16-byte aligned biases";
    return "";
}

// Enqueue the two launches for T <= 4 tokens, k <= 16 (the caller checked the layout with
// mxt_unsupported and the pointers' alignment). Unrouted: slots / wts [T, k]; routed:
// logits [T, E] with E <= 256.
int mxt_decode(const tsa_expert_layout& L, const uint8_t* pool, int64_t n_slots, const int32_t* slots,
               const float* wts, const void* logits, int logits_dtype, int mode, const int32_t* expert_slot, int64_t E,
               int32_t* idx_out, float* w_out, int64_t T, int k, const void* x, void* y, int y_dtype, uint8_t* ws,
               int64_t ws_bytes, hipStream_t st) {
    TSA_REQUIRE(T >= 1 && T <= MAXT && k >= 1 && k <= MAXK, TSA_ERR_SHAPE, "tiled decode launch: T %lld, k %d",
                (long long)T, k);
    TSA_REQUIRE(!logits || E <= 256, TSA_ERR_SHAPE, "fused routing supports E <= 256 (got %lld)", (long long)E);
    TSA_REQUIRE(ws_bytes >= mxt_ws_bytes(L, T, k), TSA_ERR_WORKSPACE, "workspace too small for the tiled decode");
    TSA_REQUIRE(L.hidden % 8 == 0 && (reinterpret_cast<uintptr_t>(x) & 15) == 0, TSA_ERR_INVALID_ARG,
                "tiled decode needs 16-byte aligned activations");
    const int ma = pick_mm(mx_tile_groups(L.hidden)), mb = pick_mm(mx_tile_groups(L.inter));
    const void* ka = kernel_for_mm(ma, false);
    const void* kd = kernel_for_mm(mb, true);
    TSA_REQUIRE(ka && kd && L.hidden <= 3072, TSA_ERR_SHAPE, "tiled decode: unsupported sizes");

    MxtParams p{};
    p.L = L;
    p.pool = pool;
    p.n_slots = n_slots;
    uint8_t* h = ws;
    const int64_t hb = al256(T * k * 2 * L.inter);
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
    p.h = h;
    p.gu_tile = 8 * L.hidden;
    p.gu_stile = mx_tile_scale_bytes(L.hidden);
    p.dn_tile = 8 * L.inter;
    p.dn_stile = mx_tile_scale_bytes(L.inter);
    // h terms: |h| <= (limit + 1) * limit after the clamps; scale it into [64, 128) at most
    const float hmax = (L.swiglu_limit + 1.0f) * L.swiglu_limit;
    int e = 0;
    if (hmax > 0.0f && hmax < 1e30f) frexpf(hmax, &e);  // hmax < 2^e
    e = e < -100 ? -100 : (e > 100 ? 100 : e);
    p.h_scale = ldexpf(1.0f, 7 - e);
    p.h_inv = ldexpf(1.0f, e - 7);

    const size_t lds_a = MISC_LDS + 3 * 128 * (size_t)ma;
    const size_t tpb = (128 * (size_t)mb + 1023) / 1024 * 1024;
    const size_t lds_b = MISC_LDS + WAVES * 2 * tpb + 128 * (size_t)mb;
    void* args[] = {&p};
    TSA_HIP_CHECK(hipLaunchKernel(ka, dim3((unsigned)(T * k * (L.inter / 32))), dim3(256), args, lds_a, st));
    TSA_HIP_CHECK(hipLaunchKernel(kd, dim3((unsigned)(T * (L.hidden / 16))), dim3(256), args, lds_b, st));
    return TSA_OK;
}

}  // namespace tsa
