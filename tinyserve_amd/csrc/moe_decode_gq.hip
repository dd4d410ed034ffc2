// Top-k MoE decode over GGUF experts (gate, up and down as native Q8_0 / Q4_K / Q5_K / Q6_K
// block streams): two launches, both routing in-kernel when router logits are given.
//
//   gq_phase_a: workgroup = one (token, expert) pair and 4 waves x rw rows (rw <= GQ_RW) of
//     the intermediate dimension. Each wave streams the super-blocks of its rw gate rows and
//     rw up rows (gguf_dot.h: one unit per lane, 16-byte loads, dot2 over bf16 codes),
//     reduces them across the wave and writes h = act(gate, up) as bf16 (the reference
//     runs its experts in bf16) into the workspace.
//   gq_phase_b: workgroup = one token and 8 waves. Wave w takes expert w % kk (kk =
//     min(k, 8); further experts in rounds) and slice w / kk of rb output rows (rb <=
//     GQ_RB; the workgroup covers 8 / kk slices), stages that
//     expert's h in its LDS area, streams the down rows the same way and keeps the
//     router-weighted partial per row; the workgroup sums the partials over experts in a
//     fixed order, so every output has one writer and the result is deterministic.
//
// Semantics: tinyserve/ggml_forward.py:88-115 (GGUF expert: silu(W_g x) * (W_u x), then
// W_d), tinyserve/csrc/expert_loop.cpp:83-121 (weighted top-k sum), :85 (slot < 0
// contributes nothing), tinyserve/_model_hooks.py:456-473 (routing).
#include "fused_common.h"
#include "mfma_tile.h"
#include "gguf_dot.h"

namespace tsa {
namespace {

constexpr int GQ_RW = 4;         // phase A: intermediate rows per wave, at most
constexpr int GQ_RB = 8;         // phase B: output rows per wave, at most
constexpr int GQ_B_WAVES = 8;
constexpr int GQ_MISC = 2048;    // slot / weight tables, per-(expert, row) partials
constexpr int GQ_XC = 4;         // phase A: 8-value chunks of x per thread (hidden <= 8192)

struct GqParams {
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
    const void* x;
    int x_dtype;
    void* y;
    int y_dtype;
    uint16_t* h;  // bf16 [T k, I]
    int64_t h_bytes;              // bytes of h (the records of its buffer resource)
    int32_t* tab_slot;            // routed: the slots and weights phase A chose, [T, k]
    float* tab_w;
    int rw, rb;                   // rows per wave of phase A and of phase B (host-chosen)
    int raw_off_a, raw_stride_a;  // phase A: LDS offset and per-wave stride of the raw super-block areas
    int vec_stride_b;             // phase B: per-wave stride of the staged h vectors (16-byte multiple)
    int raw_off_b, raw_stride_b;  // phase B: raw areas
};

__device__ __forceinline__ float gq_act(const tsa_expert_layout& L, float gate, float up) {
    if (L.act == TSA_ACT_SWIGLU_OAI) return swiglu_oai(L, gate, up);
    return gate * sigmoidf_(gate) * up;
}

// Phase A units of one wave: lane i takes units i, i + 64, ... of gate (i < nu) then up.
template <int TG, bool WRAP, bool SPLIT>
__device__ __forceinline__ void gq_a_units(const uint8_t* rbuf, uint32_t raw, const uint32_t shift[2], uint32_t s0,
                                           uint32_t u0, uint32_t nu, int n0, int H, uint32_t lo, uint32_t hi,
                                           const GqVec& xv, int lane, float (&acc)[2][GQ_RW]) {
    using U = GqUnit<TG>;
    constexpr uint32_t VS = TG == 8 ? 32 : 256, SB = U::SB;
    for (uint32_t i = lane; i < 2 * nu; i += 64) {
        const bool up = i >= nu;
        const uint32_t u = u0 + (up ? i - nu : i);
        const uint32_t g0 = u * U::V, row = g0 / (uint32_t)H, kk0 = g0 - row * (uint32_t)H;
        const uint8_t* sb = rbuf + (up ? raw : 0) + shift[up] + (g0 / VS - s0) * SB;
        float pa = 0.0f, pb = 0.0f;
        gq_unit<TG, WRAP, SPLIT>(sb, u, kk0, H, lo, hi, xv, pa, pb);
        const int r = (int)row - n0;
        if (up) {
            acc_add(acc[1], r, pa);
            if (WRAP) acc_add(acc[1], r + 1, pb);
        } else {
            acc_add(acc[0], r, pa);
            if (WRAP) acc_add(acc[0], r + 1, pb);
        }
    }
}

// Phase B units of one wave (one expert's rows [n0, n1) of down), weighted by wj.
template <int TD, bool WRAP>
__device__ __forceinline__ void gq_b_units(const uint8_t* rbuf, uint32_t shift, uint32_t s0, uint32_t u0, uint32_t nu,
                                           int n0, int I, uint32_t lo, uint32_t hi, const GqVec& hv, float wj,
                                           int lane, float (&acc)[GQ_RB]) {
    using U = GqUnit<TD>;
    constexpr uint32_t VS = TD == 8 ? 32 : 256, SB = U::SB;
    for (uint32_t i = lane; i < nu; i += 64) {
        const uint32_t u = u0 + i;
        const uint32_t g0 = u * U::V, row = g0 / (uint32_t)I, kk0 = g0 - row * (uint32_t)I;
        const uint8_t* sb = rbuf + shift + (g0 / VS - s0) * SB;
        float pa = 0.0f, pb = 0.0f;
        gq_unit<TD, WRAP>(sb, u, kk0, I, lo, hi, hv, pa, pb);
        const int r = (int)row - n0;
        acc_add(acc, r, wj * pa);
        if (WRAP) acc_add(acc, r + 1, wj * pb);
    }
}

// SPLIT: x is fp32 / fp16, staged as a bf16 hi / lo pair (its own instantiation: the pair's
// registers would otherwise set the bf16 kernel's register budget, and so its occupancy).
template <int TG, bool SPLIT>
__global__ void __launch_bounds__(256) gq_phase_a(GqParams p) {
    extern __shared__ __align__(16) uint8_t smem[];
    const int tid = threadIdx.x, lane = tid & 63, wave = uniform(tid >> 6);
    const tsa_expert_layout& L = p.L;
    const int H = (int)L.hidden, I = (int)L.inter, k = p.k;
    const int a = blockIdx.y, t = a / k, jj = a % k;
    int* s_slot = reinterpret_cast<int*>(smem);
    float* s_w = reinterpret_cast<float*>(smem + 4 * FUSED_MAXT * FUSED_MAXK);
    constexpr bool split = SPLIT;  // p.x_dtype != TSA_BF16
    const GqVec xv = gq_vec(smem + GQ_MISC, H, split);

    // ---- loads, all issued before any is used: this thread's chunks of x (thread order,
    // zero past the vector), then the routing inputs (or the pair's slot as a scalar load)
    const int xes = p.x_dtype == TSA_F32 ? 4 : 2, cpv = H / 8;
    const __amdgpu_buffer_rsrc_t rx = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<uint8_t*>(static_cast<const uint8_t*>(p.x) + (int64_t)t * H * xes), (short)0, H * xes, 0x00020000);
    GqRaw xr[GQ_XC];
#pragma unroll
    for (int c = 0; c < GQ_XC; ++c) xr[c] = gq_chunk_load_buf(rx, xes, tid + 256 * c);
    const bool routed = p.logits != nullptr;
    float lg[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    int es[4] = {0, 0, 0, 0};
    int64_t slot = -1;
    if (routed) {
#pragma unroll
        for (int j = 0; j < 4; ++j) es[j] = p.expert_slot[min(lane + 64 * j, p.E - 1)];
        load4(p.logits, p.logits_dtype, (int64_t)t * p.E, p.E, lane, lg);
    } else {
        slot = uniform(p.slots[(int64_t)t * k + jj]);
    }
    // ---- every wave selects the pair's expert itself (round jj of the top-k); wave 0 of the
    // token's first workgroup makes all k selections and writes the table for phase B
    if (routed) {
        if (blockIdx.x == 0 && jj == 0 && wave == 0) {
            const int sel = route_token_v(p, t, lane, lg, es, s_slot, s_w);
            if (lane < k) {
                if (p.idx_out) {
                    p.idx_out[t * k + lane] = sel;
                    p.w_out[t * k + lane] = s_w[t * k + lane];
                }
                p.tab_slot[t * k + lane] = s_slot[t * k + lane];  // written by this lane
                p.tab_w[t * k + lane] = s_w[t * k + lane];
            }
            slot = uniform(s_slot[t * k]);  // lane 0's own write
        } else {
            uint32_t myk;
            int mysel, myslot;
            select_topk(p, lane, lg, es, jj + 1, myk, mysel, myslot);
            slot = __builtin_amdgcn_readlane(myslot, jj);
        }
    }
    // every wave of the workgroup made the same selection: all return here or none
    if (slot < 0 || slot >= p.n_slots) return;  // a dead pair's h is never read
    // ---- x into LDS (every wave its chunks), then the super-block copies
#pragma unroll
    for (int c = 0; c < GQ_XC; ++c) {
        if (256 * c >= cpv) break;
        const int i = tid + 256 * c;
        gq_chunk_store(xr[c], i < cpv, smem + GQ_MISC, 0, p.x_dtype, H, cpv, i);
    }
    const int n0 = ((int)blockIdx.x * 4 + wave) * p.rw;
    const bool has_rows = n0 < I;
    const int n1 = n0 + p.rw < I ? n0 + p.rw : I;
    const uint8_t* base = p.pool + slot * L.slot_bytes;
    using U = GqUnit<TG>;
    constexpr uint32_t VS = TG == 8 ? 32 : 256, SB = U::SB;
    const uint32_t lo = (uint32_t)n0 * H, hi = (uint32_t)(has_rows ? n1 : n0) * H;
    const uint32_t u0 = lo / U::V, nu = (hi + U::V - 1) / U::V - u0;
    // the super-blocks of rows [n0, n1) of gate and up into this wave's LDS area
    const uint32_t s0 = lo / VS, nsb = gq_sb_count<TG>(lo, hi);
    const uint32_t raw = gq_raw_bytes(nsb, SB);
    uint8_t* rbuf = smem + p.raw_off_a + wave * p.raw_stride_a;
    const uint32_t lds_r = (uint32_t)reinterpret_cast<uintptr_t>(rbuf);
    // copies read 16-byte-aligned memory: the buffer starts at the boundary at or below the slot
    const uint32_t mis = (uint32_t)reinterpret_cast<uintptr_t>(base) & 15u;
    uint32_t shift[2];
#pragma unroll
    for (int m = 0; m < 2; ++m) {
        const uint32_t first = mis + (uint32_t)(m ? L.up_off : L.gate_off) + s0 * SB;  // byte in the buffer
        shift[m] = first & 15u;
        if (has_rows)
            gq_stage_raw(base - mis, gq_records((uint64_t)L.slot_bytes, mis), first - shift[m], raw, lds_r + m * raw,
                         lane);
    }
    gq_wait_dma();
    __syncthreads();  // x complete (every wave's chunks)
    if (!has_rows) return;
    float acc[2][GQ_RW];
#pragma unroll
    for (int m = 0; m < 2; ++m)
#pragma unroll
        for (int r = 0; r < GQ_RW; ++r) acc[m][r] = 0.0f;
    const bool wrap = H % U::V != 0;
    if (!wrap && !split)
        gq_a_units<TG, false, false>(rbuf, raw, shift, s0, u0, nu, n0, H, lo, hi, xv, lane, acc);
    else if (!wrap)
        gq_a_units<TG, false, true>(rbuf, raw, shift, s0, u0, nu, n0, H, lo, hi, xv, lane, acc);
    else if (!split)
        gq_a_units<TG, true, false>(rbuf, raw, shift, s0, u0, nu, n0, H, lo, hi, xv, lane, acc);
    else
        gq_a_units<TG, true, true>(rbuf, raw, shift, s0, u0, nu, n0, H, lo, hi, xv, lane, acc);
    static_assert(GQ_RW == 4, "gate and up rows fill the 8 rows of one wave_sum_rows");
    const float rows8[8] = {acc[0][0], acc[0][1], acc[0][2], acc[0][3], acc[1][0], acc[1][1], acc[1][2], acc[1][3]};
    const float tot = wave_sum_rows<8>(rows8, lane);     // lane 8 i: gate row i (i < 4) / up row i - 4
    // up row r (lane 32 + 8 r) lands beside gate row r: the swap's second half, lower lanes
    const float up = __uint_as_float(__builtin_amdgcn_permlane32_swap(__float_as_uint(tot), __float_as_uint(tot), false, false)[1]);
    const int r = lane >> 3;
    if ((lane & 7) == 0 && r < GQ_RW && n0 + r < n1)
        p.h[(int64_t)a * I + n0 + r] = f32_to_bf16_bits(gq_act(L, tot, up));
}

template <int TD>
__global__ void __launch_bounds__(64 * GQ_B_WAVES) gq_phase_b(GqParams p) {
    extern __shared__ __align__(16) uint8_t smem[];
    const int tid = threadIdx.x, lane = tid & 63, wave = uniform(tid >> 6);
    const tsa_expert_layout& L = p.L;
    const int H = (int)L.hidden, I = (int)L.inter, k = p.k;
    const int t = blockIdx.y;
    float* s_part = reinterpret_cast<float*>(smem + 8 * FUSED_MAXT * FUSED_MAXK);  // [8 waves][GQ_RB]
    uint8_t* hbuf = smem + GQ_MISC + (wave % (k < GQ_B_WAVES ? k : GQ_B_WAVES)) * p.vec_stride_b;  // this wave's expert
    for (int i = tid; i < GQ_B_WAVES * GQ_RB; i += blockDim.x) s_part[i] = 0.0f;  // ordered by the rounds' barriers

    const int kk = k < GQ_B_WAVES ? k : GQ_B_WAVES;          // experts per round
    const int S = GQ_B_WAVES / kk;                            // row slices
    const int slice = wave / kk, jw = wave % kk;
    const int rows_per = p.rb;
    const int nb0 = (int)blockIdx.x * S * rows_per;
    const int n0 = nb0 + slice * rows_per;
    const int n1 = n0 + rows_per < H ? n0 + rows_per : H;
    using U = GqUnit<TD>;
    constexpr uint32_t VS = TD == 8 ? 32 : 256, SB = U::SB;
    float acc[GQ_RB];
#pragma unroll
    for (int r = 0; r < GQ_RB; ++r) acc[r] = 0.0f;
    const bool mine = slice < S && n0 < n1;
    const uint32_t lo = (uint32_t)n0 * I, hi = (uint32_t)(mine ? n1 : n0) * I;
    const uint32_t u0 = lo / U::V, nu = (hi + U::V - 1) / U::V - u0;
    const uint32_t s0 = lo / VS, raw = gq_raw_bytes(gq_sb_count<TD>(lo, hi), SB);
    uint8_t* rbuf = smem + p.raw_off_b + wave * p.raw_stride_b;
    const uint32_t lds_r = (uint32_t)reinterpret_cast<uintptr_t>(rbuf);
    for (int j0 = 0; j0 < k; j0 += kk) {  // rounds of kk experts (workgroup-uniform)
        const int j = j0 + jw, nj = k - j0 < kk ? k - j0 : kk;
        // the wave's expert as scalar loads of the [T, k] table (phase A's routed one or the
        // caller's), ahead of every vector load
        const int64_t slot = j < k ? uniform(p.slots[(int64_t)t * k + j]) : -1;
        const float wj = j < k ? __int_as_float(uniform(__float_as_int(p.wts[(int64_t)t * k + j]))) : 0.0f;
        const bool live = mine && j < k && slot >= 0 && slot < p.n_slots;
        const uint8_t* sbase = p.pool + (live ? slot : 0) * L.slot_bytes;
        const uint32_t mis = (uint32_t)reinterpret_cast<uintptr_t>(sbase) & 15u;  // as in phase A
        const uint32_t first = mis + (uint32_t)L.down_off + s0 * SB, shift = first & 15u;
        if (live) gq_stage_raw(sbase - mis, gq_records((uint64_t)L.slot_bytes, mis), first - shift, raw, lds_r, lane);
        // the round's h vectors (bf16 from phase A) into LDS once for the workgroup: vector jj
        // at smem + GQ_MISC + jj * vec_stride_b, staged by all threads together
        gq_stage_vecs(smem + GQ_MISC, p.vec_stride_b, p.h, TSA_BF16, (int64_t)(t * k + j0) * I, I, I, nj, tid,
                      blockDim.x);
        gq_wait_dma();
        __syncthreads();
        if (live) {
            const GqVec hv = gq_vec(hbuf, I);
            if (I % U::V == 0)
                gq_b_units<TD, false>(rbuf, shift, s0, u0, nu, n0, I, lo, hi, hv, wj, lane, acc);
            else
                gq_b_units<TD, true>(rbuf, shift, s0, u0, nu, n0, I, lo, hi, hv, wj, lane, acc);
        }
        __syncthreads();  // the round's h and raw areas are free again
    }
    static_assert(GQ_RB == 8, "one wave_sum_rows over the rows");
    const float tot = wave_sum_rows<GQ_RB>(acc, lane);  // lane 8 r: row r
    if ((lane & 7) == 0 && (lane >> 3) < rows_per) s_part[wave * GQ_RB + (lane >> 3)] = tot;
    __syncthreads();
    if (tid < S * rows_per) {  // row nb0 + tid = slice tid / rows_per, row tid % rows_per of that slice
        const int sl = tid / rows_per, r = tid % rows_per;
        float sum = 0.0f;
        for (int j = 0; j < kk; ++j) sum += s_part[(sl * kk + j) * GQ_RB + r];
        if (nb0 + tid < H) store_out(p.y, p.y_dtype, (int64_t)t * H + nb0 + tid, sum);
    }
}

template <int TG>
const void* phase_a_fn(bool split) {
    return split ? reinterpret_cast<const void*>(&gq_phase_a<TG, true>) : reinterpret_cast<const void*>(&gq_phase_a<TG, false>);
}
template <int TD>
const void* phase_b_fn() { return reinterpret_cast<const void*>(&gq_phase_b<TD>); }

const void* pick_a(int t, bool split = false) {
    switch (t) {
        case 8: return phase_a_fn<8>(split);
        case 12: return phase_a_fn<12>(split);
        case 13: return phase_a_fn<13>(split);
        case 14: return phase_a_fn<14>(split);
    }
    return nullptr;
}
const void* pick_b(int t) {
    switch (t) {
        case 8: return phase_b_fn<8>();
        case 12: return phase_b_fn<12>();
        case 13: return phase_b_fn<13>();
        case 14: return phase_b_fn<14>();
    }
    return nullptr;
}

}  // namespace

// Requirements beyond validate_layout: "" if met.
const char* gq_unsupported(const tsa_expert_layout& L) {
    if (L.format != TSA_EXPERT_GGUF) return "not a GGUF layout";
    if (L.gate_type != L.up_type) return "gate and up must share one ggml type";
    if (!pick_a(L.gate_type) || !pick_b(L.down_type)) return "unsupported ggml type";
    if (L.gate_bias_off >= 0 || L.down_bias_off >= 0) return "GGUF experts carry no biases";
    if (L.hidden % 32 || L.inter % 32) return "hidden and inter must be multiples of 32";
    if (2 * L.inter * L.hidden >= ((int64_t)1 << 31)) return "matrices of 2^31 values or more are not supported";
    if (L.hidden > 8192 || L.inter > 4096) return "hidden above 8192 or inter above 4096 is not supported";
    return "";
}

int gs_decode(const tsa_expert_layout& L, const uint8_t* pool, int64_t n_slots, const int32_t* slots, const float* wts,
              const void* logits, int logits_dtype, int mode, const int32_t* expert_slot, int64_t E, int32_t* idx_out,
              float* w_out, int64_t T, int k, const void* x, int x_dtype, void* y, int y_dtype, uint8_t* ws,
              int64_t ws_bytes, hipStream_t st);

int gq_decode(const tsa_expert_layout& L, const uint8_t* pool, int64_t n_slots, const int32_t* slots, const float* wts,
              const void* logits, int logits_dtype, int mode, const int32_t* expert_slot, int64_t E, int32_t* idx_out,
              float* w_out, int64_t T, int k, const void* x, int x_dtype, void* y, int y_dtype, uint8_t* ws,
              int64_t ws_bytes, hipStream_t st) {
    const char* why = gq_unsupported(L);
    TSA_REQUIRE(!*why, TSA_ERR_SHAPE, "GGUF decode: %s", why);
    TSA_REQUIRE(T >= 1 && T <= 65535 && k >= 1 && k <= FUSED_MAXK && T * k <= 65535, TSA_ERR_SHAPE,
                "GGUF decode: T %lld, k %d", (long long)T, k);
    TSA_REQUIRE(!logits || (E <= 256 && T <= FUSED_MAXT), TSA_ERR_SHAPE, "GGUF decode routing: E %lld, T %lld",
                (long long)E, (long long)T);
    // h (bf16) then, for routed calls, the slot / weight table phase A writes for phase B
    const int64_t h_bytes = T * k * L.inter * 2, tab_off = (h_bytes + 255) / 256 * 256;
    TSA_REQUIRE(ws_bytes >= tab_off + T * k * 8, TSA_ERR_WORKSPACE, "workspace too small for the GGUF decode");
    // the sub-block stream kernels where they cover the call
    const int rs = gs_decode(L, pool, n_slots, slots, wts, logits, logits_dtype, mode, expert_slot, E, idx_out, w_out,
                             T, k, x, x_dtype, y, y_dtype, ws, ws_bytes, st);
    if (rs <= 0) return rs;
    GqParams p{};
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
    p.x = x;
    p.x_dtype = x_dtype;
    p.y = y;
    p.y_dtype = y_dtype;
    p.h = reinterpret_cast<uint16_t*>(ws);
    p.h_bytes = h_bytes;
    p.tab_slot = reinterpret_cast<int32_t*>(ws + tab_off);
    p.tab_w = reinterpret_cast<float*>(ws + tab_off + T * k * 4);
    // rows per wave (gq_cost) and the raw staging per wave: phase A rw rows of gate and of
    // up (K = hidden); phase B rb rows of one expert's down (K = inter); the largest over
    // row alignments
    const int ta = L.gate_type, tb = L.down_type;
    auto sb_bytes = [](int t) { return t == 8 ? 34u : t == 12 ? 144u : t == 13 ? 176u : 210u; };
    auto vs = [](int t) { return t == 8 ? 32u : 256u; };
    auto uv = [](int t) { return gq_unit_values(t); };
    const int cus = num_cus();
    const size_t vecA = ((size_t)gq_vec_bytes((int)L.hidden, x_dtype != TSA_BF16) + 15) / 16 * 16;
    const size_t vecB = ((size_t)gq_vec_bytes((int)L.inter) + 15) / 16 * 16;
    auto raw_a = [&](int rw) { return gq_raw_bytes((rw * (uint32_t)L.hidden + vs(ta) - 1) / vs(ta) + 1, sb_bytes(ta)); };
    auto raw_b = [&](int rb) { return gq_raw_bytes((rb * (uint32_t)L.inter + vs(tb) - 1) / vs(tb) + 1, sb_bytes(tb)); };
    const int kk = k < GQ_B_WAVES ? k : GQ_B_WAVES;
    const int S = GQ_B_WAVES / kk;
    double best_a = 0.0, best_b = 0.0;
    for (int rw = 1; rw <= GQ_RW; ++rw) {
        if (GQ_MISC + vecA + 8 * (size_t)raw_a(rw) > 160 * 1024) break;
        const double c = gq_cost(2 * gq_units(rw, L.hidden, uv(ta)), (double)((L.inter + rw - 1) / rw) * T * k, cus);
        if (p.rw == 0 || c <= best_a) { best_a = c; p.rw = rw; }
    }
    for (int rb = 1; rb <= GQ_RB; ++rb) {
        if (GQ_MISC + GQ_B_WAVES * (vecB + raw_b(rb)) > 160 * 1024) break;
        const double c = gq_cost(gq_units(rb, L.inter, uv(tb)) * ((k + kk - 1) / kk),
                                 (double)((L.hidden + S * rb - 1) / (S * rb)) * GQ_B_WAVES * T, cus);
        if (p.rb == 0 || c <= best_b) { best_b = c; p.rb = rb; }
    }
    TSA_REQUIRE(p.rw > 0 && p.rb > 0, TSA_ERR_SHAPE, "GGUF decode: rows of %lld / %lld values exceed LDS",
                (long long)L.hidden, (long long)L.inter);
    const uint32_t rawA = raw_a(p.rw), rawB = raw_b(p.rb);
    const size_t lds_a = GQ_MISC + vecA + 4 * 2 * (size_t)rawA;
    p.raw_off_a = (int)(GQ_MISC + vecA);
    p.raw_stride_a = (int)(2 * rawA);
    p.vec_stride_b = (int)vecB;
    p.raw_off_b = (int)(GQ_MISC + GQ_B_WAVES * vecB);
    p.raw_stride_b = (int)rawB;
    const size_t lds_b = GQ_MISC + GQ_B_WAVES * (vecB + rawB);
    TSA_REQUIRE(lds_a <= 160 * 1024 && lds_b <= 160 * 1024, TSA_ERR_SHAPE, "GGUF decode: LDS %zu / %zu bytes", lds_a,
                lds_b);
    const void* fa = pick_a(L.gate_type, x_dtype != TSA_BF16);
    const void* fb = pick_b(L.down_type);
    TSA_HIP_CHECK(ensure_dynamic_lds(fb, (int)lds_b));
    TSA_HIP_CHECK(ensure_dynamic_lds(fa, (int)lds_a));
    void* args[] = {&p};
    const dim3 ga((unsigned)((L.inter + 4 * p.rw - 1) / (4 * p.rw)), (unsigned)(T * k));
    TSA_HIP_CHECK(hipLaunchKernel(fa, ga, dim3(256), args, lds_a, st));
    GqParams pb = p;  // phase B takes the routed table as its slot / weight input
    if (logits) {
        pb.logits = nullptr;
        pb.slots = p.tab_slot;
        pb.wts = p.tab_w;
    }
    void* args_b[] = {&pb};
    const dim3 gb((unsigned)((L.hidden + S * pb.rb - 1) / (S * pb.rb)), (unsigned)T);
    TSA_HIP_CHECK(hipLaunchKernel(fb, gb, dim3(64 * GQ_B_WAVES), args_b, lds_b, st));
    return TSA_OK;
}

}  // namespace tsa
