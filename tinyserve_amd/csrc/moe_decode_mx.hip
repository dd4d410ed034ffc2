// MXFP4 MoE decode over the checkpoint-order layout (gfx950): routing + gate_up + clamped
// SwiGLU + down + weighted top-k sum in two launches.
//
// Launch 1 (gate_up), workgroup = (token t, expert j, 64 gate_up rows): each of the 4
//   waves owns 16 consecutive rows (16 x 1440 B contiguous for K = 2880) and streams them
//   with fully contiguous 16-byte-per-lane buffer loads: lane l of load s holds 16-byte
//   group chunk c = 64 s + l of the tile, i.e. row c / G, group c % G. Each chunk (32 e2m1
//   values) is expanded to bf16 pairs with v_cvt_scalef32_pk_bf16_fp4 (exact) and dotted
//   with the activation's bf16 pairs from LDS by v_dot2c_f32_bf16 (fp32 accumulate), then
//   scaled by its e8m0 group scale and accumulated into the lane's partial of that row.
//   DPP wave reductions give the 16 row sums; row pairs (gate, up) go through the clamped
//   SwiGLU and the 8 h values go to the workspace.
// Launch 2 (down), workgroup = (token t, 16 output rows): wave j computes expert j's 16
//   down rows the same way, with h (rounded to bf16, like the reference's bf16
//   activations) staged in LDS; the waves' weighted rows are summed in a fixed order in
//   LDS, so each output has one writer and the result is deterministic.
// No workgroup waits for another (stream order is the only synchronisation), so the
// workspace holds no counters and nothing needs resetting between calls.
//
// Routing (optional) runs in every workgroup's prologue of both launches on wave 0 with
// DPP reductions (descending logit, ties to the lower expert id) while the other waves
// stage x; both launches select the same experts from the same logits.
//
// Semantics: tinyserve/_model_hooks.py:380-394 (MXFP4 expert with biases, clamped
// SwiGLU), :456-473 (routing), tinyserve/csrc/expert_loop.cpp:83-121 (weighted sum).
#include "fused_common.h"

namespace tsa {
namespace {

typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

constexpr int MAXT = FUSED_MAXT;
constexpr int MAXK = FUSED_MAXK;
constexpr int WAVES = 4;
constexpr int ROWS = 16;  // rows per wave tile
constexpr int MISC_LDS = 2048;  // slot/weight/selection tables, per-wave row sums

struct MxParams {
    tsa_expert_layout L;
    const uint8_t* pool;
    int64_t n_slots;
    const int32_t* slots;        // [T, k] (unrouted) or null
    const float* wts;            // [T, k] (unrouted) or null
    const void* logits;          // [T, E] (routed) or null
    const int32_t* expert_slot;  // [E] (routed)
    int32_t* idx_out;            // [T, k] (routed, optional)
    float* w_out;                // [T, k] (routed, optional)
    int logits_dtype, route_mode, E;
    int T, k;
    const uint16_t* x;  // bf16 [T, H]
    void* y;
    int y_dtype;
    float* h;  // [T, k, I] intermediate (workspace)
};


// Byte offset in LDS of 16-byte chunk q (0..3) of 32-value group g of a bf16 vector:
// chunks rotate by g/2 so that 16 lanes reading consecutive groups hit 8 distinct bank
// quads (two 128-byte cycles, the minimum for 256 bytes).
__device__ __forceinline__ int xchunk(int g, int q) { return 64 * g + 16 * ((q + (g >> 1)) & 3); }


typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));

struct XFrag {
    bf16x8 v[4];
};

// The 32 bf16 activations of group g (LDS, swizzled).
__device__ __forceinline__ XFrag load_x(const uint8_t* xs, int g) {
    XFrag f;
#pragma unroll
    for (int d = 0; d < 4; ++d) f.v[d] = *reinterpret_cast<const bf16x8*>(xs + xchunk(g, d));
    return f;
}

// Dot of one 16-byte MXFP4 chunk (32 e2m1 values) with 32 bf16 activations, unscaled.
// The activation pairs are taken as bf16 shuffles of the 8-wide LDS read: going through
// 32-bit dwords (bitcast of an element of a <4 x i32>) miscompiles with this toolchain -
// all four v_dot2c operands of a read collapse onto one register (found with an
// on-device probe; this form keeps them distinct and is exact).
__device__ __forceinline__ float chunk_dot(const u32x4& q, const XFrag& x) {
    float acc = 0.0f;
#pragma unroll
    for (int d = 0; d < 4; ++d) {
        const uint32_t w = q[d];
        const bf16x8 xv = x.v[d];
        acc = __builtin_amdgcn_fdot2_f32_bf16(__builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(w, 1.0f, 0),
                                              __builtin_shufflevector(xv, xv, 0, 1), acc, false);
        acc = __builtin_amdgcn_fdot2_f32_bf16(__builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(w, 1.0f, 1),
                                              __builtin_shufflevector(xv, xv, 2, 3), acc, false);
        acc = __builtin_amdgcn_fdot2_f32_bf16(__builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(w, 1.0f, 2),
                                              __builtin_shufflevector(xv, xv, 4, 5), acc, false);
        acc = __builtin_amdgcn_fdot2_f32_bf16(__builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(w, 1.0f, 3),
                                              __builtin_shufflevector(xv, xv, 6, 7), acc, false);
    }
    return acc;
}

// A wave's 16-row tile: S contiguous loads of 64 x 16 B; its 16*G scale bytes (also
// contiguous) go through LDS, loaded first so that waiting for them does not wait for
// the tile.
template <int G>
struct Tile {
    static constexpr int S = (ROWS * G + 63) / 64;
    u32x4 q[S];
};

// Buffer resources start at the tile, so chunks past the matrix end read zero (no fault).
template <int G>
__device__ __forceinline__ void tile_load(Tile<G>& tl, uint8_t* rs, const uint8_t* blocks, const uint8_t* scales,
                                          int64_t nrows, int64_t row0, int lane) {
    static_assert(ROWS * G <= 128 * 16, "two 16-byte scale loads per lane");
    const __amdgpu_buffer_rsrc_t rb = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<uint8_t*>(blocks + row0 * G * 16), (short)0, (int)((nrows - row0) * G * 16), 0x00020000);
    const __amdgpu_buffer_rsrc_t rsc = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<uint8_t*>(scales + row0 * G), (short)0, (int)((nrows - row0) * G), 0x00020000);
    const u32x4 s0 = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rsc, 16 * lane, 0, 0));
    const u32x4 s1 = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rsc, 16 * (64 + lane), 0, 0));
#pragma unroll
    for (int s = 0; s < Tile<G>::S; ++s)
        tl.q[s] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rb, 16 * (64 * s + lane), 0, 2));
    if (16 * lane < ROWS * G) *reinterpret_cast<u32x4*>(rs + 16 * lane) = s0;
    if (16 * (64 + lane) < ROWS * G) *reinterpret_cast<u32x4*>(rs + 16 * (64 + lane)) = s1;
}

// Row sums of the tile against the bf16 vector xs: lane r < 16 returns row r's sum.
// A row is wave-reduced right after the step holding its last chunk, so only the rows
// still in progress keep partial registers. Chunks past row 15 are dropped.
template <int G>
__device__ __forceinline__ float tile_rows(const Tile<G>& tl, const uint8_t* rs, const uint8_t* xs, int lane) {
    float acc[ROWS];
#pragma unroll
    for (int r = 0; r < ROWS; ++r) acc[r] = 0.0f;
    float mine = 0.0f;
#pragma unroll
    for (int s = 0; s < Tile<G>::S; ++s) {
        const int c = 64 * s + lane;
        const int r = c / G;
        const XFrag x = load_x(xs, c - r * G);
        const uint32_t sc = rs[c < ROWS * G ? c : 0];
        const float v = chunk_dot(tl.q[s], x) * e8m0_to_f32(sc);
        const int rlo = (64 * s) / G, rhi = (64 * s + 63) / G;
#pragma unroll
        for (int rr = rlo; rr <= rhi; ++rr) {
            if (rr >= ROWS) break;
            acc[rr] += (r == rr) ? v : 0.0f;
            if (G * (rr + 1) - 1 <= 64 * s + 63) {  // last chunk of row rr is in this step
                const float sr = wave_sum_u(acc[rr]);
                mine = lane == rr ? sr : mine;
            }
        }
    }
    return mine;
}

// A copy of v the compiler cannot see through: lane-derived addressing is then recomputed
// where it is used instead of being hoisted and kept live (which would cost ~4 VGPRs per
// load step).
__device__ __forceinline__ int opaque(int v) {
    asm volatile("" : "+v"(v));
    return v;
}


// Stage n bf16 values (n % 32 == 0, 16-aligned source) into LDS with the chunk swizzle.
__device__ __forceinline__ void stage_bf16(uint8_t* xs, const uint16_t* src, int n, int tid, int nthreads) {
    const __amdgpu_buffer_rsrc_t r =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t*>(src), (short)0, n * 2, 0x00020000);
    for (int c0 = 0; c0 < n / 8; c0 += 2 * nthreads) {  // two 16-byte loads in flight per thread
        const int ca = c0 + tid, cb = c0 + nthreads + tid;
        const u32x4 a = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(r, 16 * ca, 0, 0));
        const u32x4 b = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(r, 16 * cb, 0, 0));
        if (ca < n / 8) *reinterpret_cast<u32x4*>(xs + xchunk(ca >> 2, ca & 3)) = a;
        if (cb < n / 8) *reinterpret_cast<u32x4*>(xs + xchunk(cb >> 2, cb & 3)) = b;
    }
}

// I floats (published h) -> bf16 into LDS with the chunk swizzle. Piece p holds floats
// 4p..4p+3 = group p/8, chunk (p%8)/2, bytes 8*(p%2) of that chunk.
__device__ __forceinline__ void stage_h(uint8_t* hs, const float* src, int I, int lane) {
    const __amdgpu_buffer_rsrc_t r =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(src), (short)0, I * 4, 0x00020000);
    constexpr int B = 6;  // pieces per lane per batch, loads in flight together
    const int pieces = I / 4;
    for (int base = 0; base < pieces; base += 64 * B) {
        u32x4 v[B];
#pragma unroll
        for (int b = 0; b < B; ++b)
            v[b] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(r, 16 * (base + 64 * b + lane), 0, 0));
#pragma unroll
        for (int b = 0; b < B; ++b) {
            const int pc = base + 64 * b + lane;
            if (pc < pieces) {
                const uint32_t lo = (uint32_t)f32_to_bf16_bits(__uint_as_float(v[b][0])) |
                                    ((uint32_t)f32_to_bf16_bits(__uint_as_float(v[b][1])) << 16);
                const uint32_t hi = (uint32_t)f32_to_bf16_bits(__uint_as_float(v[b][2])) |
                                    ((uint32_t)f32_to_bf16_bits(__uint_as_float(v[b][3])) << 16);
                const int g = pc >> 3, q = (pc & 7) >> 1;
                *reinterpret_cast<uint2*>(hs + xchunk(g, q) + 8 * (pc & 1)) = make_uint2(lo, hi);
            }
        }
    }
}

// PHASE 0: launch 1 (workgroup b = gate_up task b); PHASE 1: launch 2 (workgroup b = down task b).
template <int G, int PHASE>
__global__ void __launch_bounds__(256, 2) mx_decode_kernel(MxParams p) {
    extern __shared__ __align__(16) uint8_t smem[];
    const int tid = threadIdx.x, lane = tid & 63, wave = uniform(tid >> 6);
    const tsa_expert_layout& L = p.L;
    const int H = (int)L.hidden, I = (int)L.inter;  // H == I == 32 G
    const int T = p.T, k = p.k;
    int* s_slot = reinterpret_cast<int*>(smem);                      // [MAXT*MAXK]
    float* s_w = reinterpret_cast<float*>(smem + 4 * MAXT * MAXK);   // [MAXT*MAXK]
    float* s_y = reinterpret_cast<float*>(smem + 12 * MAXT * MAXK);  // [WAVES][16]
    uint8_t* rsc = smem + MISC_LDS + wave * ROWS * G;  // this wave's tile scales
    uint8_t* vec = smem + MISC_LDS + WAVES * ROWS * G;  // launch 1: x [T][H] bf16; launch 2: h [WAVES][I] bf16

    // ---- prologue: routing / slot table on wave 0 while the other waves stage the
    // activations into LDS (launch 1 only)
    constexpr bool stage = PHASE == 0;
    if (p.logits) {
        if (wave == 0) {
            int es[4];
#pragma unroll
            for (int j = 0; j < 4; ++j) es[j] = p.expert_slot[min(lane + 64 * j, p.E - 1)];
            for (int t = 0; t < T; ++t) {
                const int sel = route_token(p, t, lane, es, s_slot, s_w);
                if (PHASE == 0 && blockIdx.x == 0 && p.idx_out && lane < k) {
                    p.idx_out[t * k + lane] = sel;
                    p.w_out[t * k + lane] = s_w[t * k + lane];
                }
            }
        } else if (stage) {
            for (int t = 0; t < T; ++t) stage_bf16(vec + t * H * 2, p.x + (int64_t)t * H, H, tid - 64, blockDim.x - 64);
        }
    } else {
        for (int i = tid; i < T * k; i += blockDim.x) {
            s_slot[i] = p.slots[i];
            s_w[i] = p.wts[i];
        }
        if (stage)
            for (int t = 0; t < T; ++t) stage_bf16(vec + t * H * 2, p.x + (int64_t)t * H, H, tid, blockDim.x);
    }
    __syncthreads();

    if (PHASE == 0) {
        // ---- gate_up rows -> SwiGLU -> h
        const int task = blockIdx.x;
        const int tiles = I / 32;  // 64-row tiles per expert, 32 h values each
        const int t = task / (k * tiles), j = (task / tiles) % k, kb = task % tiles;
        const int64_t slot = uniform(s_slot[t * k + j]);
        if (slot < 0 || slot >= p.n_slots) return;  // a dead pair's h is never read
        const int64_t row0 = (int64_t)kb * 64 + ROWS * wave;
        const uint8_t* base = p.pool + slot * L.slot_bytes;
        float bias = 0.0f;
        if (L.gate_bias_off >= 0) bias = load_bias(base + L.gate_bias_off, L.bias_dtype, row0 + (lane & (ROWS - 1)));
        Tile<G> tl;
        tile_load<G>(tl, rsc, base + L.gate_off, base + L.gate_scales_off, 2 * (int64_t)I, row0, lane);
        const float rs = tile_rows<G>(tl, rsc, vec + t * H * 2, opaque(lane)) + bias;  // lane r < 16: row r
        const float up = __shfl_down(rs, 1, 64);                                       // lane 2i: (gate, up) of h row0/2 + i
        const float hv = swiglu_oai(L, rs, up);
        if (lane < ROWS && (lane & 1) == 0) p.h[(int64_t)(t * k + j) * I + row0 / 2 + lane / 2] = hv;
        return;
    }

    // ---- down rows of every selected expert, weighted sum in a fixed order
    const int RB = H / ROWS;
    const int rounds = (k + WAVES - 1) / WAVES;
    uint8_t* hs = vec + wave * I * 2;
    const int b = blockIdx.x;
    const int t = b / RB;
    const int64_t n0 = (int64_t)(b % RB) * ROWS;
    float yv = 0.0f;  // lane r < 16: this wave's weighted row n0 + r
    for (int rd = 0; rd < rounds; ++rd) {
        const int j = rd * WAVES + wave;
        const int64_t slot = j < k ? uniform(s_slot[t * k + j]) : -1;
        if (slot < 0 || slot >= p.n_slots) continue;
        const uint8_t* base = p.pool + slot * L.slot_bytes;
        float bias = 0.0f;
        if (L.down_bias_off >= 0) bias = load_bias(base + L.down_bias_off, L.bias_dtype, n0 + (lane & (ROWS - 1)));
        Tile<G> tl;
        tile_load<G>(tl, rsc, base + L.down_off, base + L.down_scales_off, (int64_t)H, n0, lane);
        // h of (t, j) -> bf16 in this wave's LDS area, all loads issued before the first use
        stage_h(hs, p.h + (int64_t)(t * k + j) * I, I, lane);
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
        const float rs = tile_rows<G>(tl, rsc, hs, opaque(lane)) + bias;
        yv += s_w[t * k + j] * rs;
    }
    if (lane < ROWS) s_y[wave * ROWS + lane] = yv;
    __syncthreads();
    if (wave == 0 && lane < ROWS) {
        float sum = 0.0f;
#pragma unroll
        for (int w = 0; w < WAVES; ++w) sum += s_y[w * ROWS + lane];
        store_out(p.y, p.y_dtype, (int64_t)t * H + n0 + lane, sum);
    }
}

template <int G>
const void* kernel_ptr(int phase) {
    return phase ? reinterpret_cast<const void*>(&mx_decode_kernel<G, 1>)
                 : reinterpret_cast<const void*>(&mx_decode_kernel<G, 0>);
}

const void* kernel_for_g(int G, int phase) {
    switch (G) {
        case 16: return kernel_ptr<16>(phase);
        case 32: return kernel_ptr<32>(phase);
        case 64: return kernel_ptr<64>(phase);
        case 90: return kernel_ptr<90>(phase);
        default: return nullptr;
    }
}

}  // namespace

int64_t mx_fused_ws_bytes(const tsa_expert_layout& L, int64_t T, int k) {
    return (T * k * L.inter * 4 + 255) / 256 * 256;
}

// Enqueue the two launches: TSA_OK, 1 if the shape/layout/dtype is outside what they
// handle (the caller then uses the row kernels), or an error status.
int mx_fused_decode(const tsa_expert_layout& L, const uint8_t* pool, int64_t n_slots, const int32_t* slots,
                    const float* wts, const void* logits, int logits_dtype, int mode, const int32_t* expert_slot,
                    int64_t E, int32_t* idx_out, float* w_out, int64_t T, int k, const void* x, int x_dtype, void* y,
                    int y_dtype, uint8_t* ws, int64_t ws_bytes, hipStream_t st) {
    if (L.format != TSA_EXPERT_MXFP4 || L.act != TSA_ACT_SWIGLU_OAI || x_dtype != TSA_BF16) return 1;
    if (T < 1 || T > MAXT || k < 1 || k > MAXK || L.hidden != L.inter) return 1;
    const int G = (int)(L.hidden / 32);
    const void* ka = kernel_for_g(G, 0);
    const void* kb = kernel_for_g(G, 1);
    if (!ka || !kb) return 1;
    if (logits && E > 256) return 1;
    const uintptr_t al = reinterpret_cast<uintptr_t>(pool) | reinterpret_cast<uintptr_t>(x) | (uintptr_t)L.slot_bytes |
                         (uintptr_t)L.gate_off | (uintptr_t)L.down_off;
    if (al & 15) return 1;
    TSA_REQUIRE(ws_bytes >= mx_fused_ws_bytes(L, T, k), TSA_ERR_WORKSPACE,
                "workspace too small for the fused decode");
    const size_t lds_a = MISC_LDS + (size_t)WAVES * ROWS * G + (size_t)(T * L.hidden * 2);
    const size_t lds_b = MISC_LDS + (size_t)WAVES * ROWS * G + (size_t)(WAVES * L.inter * 2);

    MxParams p{};
    p.L = L;
    p.pool = pool;
    p.n_slots = n_slots;
    p.slots = slots;
    p.wts = wts;
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
    p.h = reinterpret_cast<float*>(ws);
    void* args[] = {&p};
    TSA_HIP_CHECK(hipLaunchKernel(ka, dim3((unsigned)(T * k * (L.inter / 32))), dim3(256), args, lds_a, st));
    TSA_HIP_CHECK(hipLaunchKernel(kb, dim3((unsigned)(T * (L.hidden / ROWS))), dim3(256), args, lds_b, st));
    return TSA_OK;
}

}  // namespace tsa
