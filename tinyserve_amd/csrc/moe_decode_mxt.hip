// Fused single-launch MoE decode over MXFP4 experts stored in the 16-row MFMA tile order
// (mx_tile.hip): routing + gate_up + clamped SwiGLU + down + weighted top-k sum in one
// persistent launch, with every weight byte streamed by contiguous 1 KB wave loads and
// multiplied on the matrix cores.
//
// Work is a task list, phase A first:
//   phase A task = (token t, expert j, 64 gate_up rows): each of the 4 waves owns one
//     16-row tile. Piece m of the tile (1 KB) arrives as one 16-byte-per-lane buffer
//     load; lane 16q+i holds MXFP4 block 4m+q of row i, which v_cvt_scalef32_pk_bf16_fp4
//     expands (block scale folded in, exact) into the bf16 A operands of four
//     v_mfma_f32_16x16x32_bf16 (K-slices u = 0..3). The B operand is the activation:
//     every lane of row q reads the same 8 bf16 values from LDS (a broadcast), so all 16
//     result columns carry the same dot products and any lane of row q holds rows 4q..4q+3
//     of the tile. Row pairs (gate, up) go through the clamped SwiGLU; the 8 h values are
//     rounded to bf16 (the reference runs its experts in bf16) and published with
//     agent-coherent stores; when all 4 waves' stores are complete the workgroup adds 1
//     to the completion counter of its (token, expert) pair.
//   phase B task = (token t, 16 output rows): wave j multiplies expert j's 16-row down
//     tile the same way against h(t, j), staged from the workspace into its LDS area; the
//     waves' weighted rows are summed in a fixed order in LDS, so each output has one
//     writer and the result is deterministic.
//
// Schedule: one workgroup per phase A task; a workgroup takes its phase B task (if any)
// after its phase A task, so its down-tile loads queue behind its gate_up loads and the
// gate_up bytes that every phase B task waits for arrive first.
//
// Synchronisation: per-(token, expert) completion counters as in moe_decode_mx.hip, but
// only wave 0 of a phase B workgroup polls (the token's k counters, spaced by s_sleep),
// after every wave has issued its down-tile loads, and the others wait at a barrier:
// hundreds of waves polling the same few lines with agent-scope loads measurably slowed
// the weight stream. The grid never exceeds the co-resident workgroup count and phase A
// work precedes every poll, so every wait ends; the spin limit is a backstop that raises
// the workspace error flag. The last phase B workgroup out resets the counters.
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
constexpr int MISC_LDS = 1024;  // slot/weight tables, per-wave row sums, flag

struct MxtParams {
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
    uint16_t* h;    // bf16 [T, k, I] published intermediate
    unsigned* bar;  // workspace header: [1] phase B workgroups finished, [2] error flag
    unsigned* flags;  // [T k][WS_FLAG_WORDS]: gate_up task kb of pair (t, j) is published
    int nA, nB, grid;
    int64_t gu_tile, gu_stile, dn_tile, dn_stile;  // bytes per 16-row tile: blocks, scale words
    int b_off;  // phase B task 0 goes to workgroup b_off (then b_off + 1, ... modulo grid)
};

// A wave's 16-row tile: MM pieces of 1 KB and the scale words (byte m%4 of word m/4).
// Buffer resources span exactly the tile, so pieces past a short row (K < 128 MM) read
// zero without touching memory.
template <int MM>
struct Tile {
    static constexpr int MS = (MM + 3) / 4;
    u32x4 q[MM];
    uint32_t sc[MS];
};

// The scale words (W per lane, W = stile_bytes / 256 <= MS) come in lane-major chunks of
// up to 4 words: one 16-byte load per chunk, bounded to the tile's scale area. A load
// wider than a lane's part of a chunk picks up the next lane's words; words >= W are
// zeroed, so they can only meet the zero blocks of groups past the row end.
template <int MM>
__device__ __forceinline__ void tile_load(Tile<MM>& tl, const uint8_t* blocks, int64_t tile_bytes,
                                          const uint8_t* scales, int64_t stile_bytes, int lane) {
    const __amdgpu_buffer_rsrc_t rb =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t*>(blocks), (short)0, (int)tile_bytes, 0x00020000);
    const __amdgpu_buffer_rsrc_t rs =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t*>(scales), (short)0, (int)stile_bytes, 0x00020000);
    const int W = (int)(stile_bytes >> 8);
#pragma unroll
    for (int c = 0; c < (Tile<MM>::MS + 3) / 4; ++c) {
        const int wc = W - 4 * c < 4 ? (W - 4 * c > 0 ? W - 4 * c : 0) : 4;  // this chunk's words per lane
        const u32x4 v = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rs, 1024 * c + 4 * wc * lane, 0, 0));
#pragma unroll
        for (int d = 0; d < 4 && 4 * c + d < Tile<MM>::MS; ++d) tl.sc[4 * c + d] = 4 * c + d < W ? v[d] : 0u;
    }
    __builtin_amdgcn_sched_barrier(0);
    // Every piece is issued, in order, before any is used: left alone the scheduler sinks
    // loads into the MFMA loop to save registers (a third of the tile in flight) or
    // reorders them so that the first MFMA waits for nearly the whole tile.
#pragma unroll
    for (int m = 0; m < MM; ++m) {  // nt: streamed once, keep it out of the caches' way
        tl.q[m] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rb, 1024 * m + 16 * lane, 0, 2));
        __builtin_amdgcn_sched_barrier(0);
    }
}

// Rows 4q..4q+3 of W_tile * v (lanes 16q+i; the result is in lane 16q), v a zero-padded
// bf16 vector [128 MM] in LDS. Only B column 0 is needed, so only lanes 0, 16, 32, 48 read
// their 8 activations (exec-masked): the other lanes keep stale values, which only reach
// result columns 1..15. (A full-wave broadcast read returns 1 KB into VGPRs per 16-byte
// useful read and slowed the concurrent weight stream.) Two accumulators alternate so
// that consecutive MFMAs are independent.
template <int MM>
__device__ __forceinline__ v4f tile_mfma(const Tile<MM>& tl, const uint8_t* vec, int lane) {
    v4f acc[2];
    acc[0] = acc[1] = v4f{0.0f, 0.0f, 0.0f, 0.0f};
    const uint8_t* vb = vec + 64 * (lane >> 4);  // K-slice q of piece m: values 128 m + 32 q ..
    const bool col0 = (lane & 15) == 0;
    bf16x8 b[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) b[u] = bf16x8{};
#pragma unroll
    for (int m = 0; m < MM; ++m) {
        const float s = e8m0_to_f32((tl.sc[m >> 2] >> (8 * (m & 3))) & 255u);
        if (col0) {
#pragma unroll
            for (int u = 0; u < 4; ++u) b[u] = *reinterpret_cast<const bf16x8*>(vb + 256 * m + 16 * u);
        }
#pragma unroll
        for (int u = 0; u < 4; ++u)
            acc[u & 1] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(expand(tl.q[m][u], s), b[u], acc[u & 1], 0, 0, 0);
    }
    return acc[0] + acc[1];
}

// n bf16 values (n % 8 == 0, 16-aligned source) into LDS, zero-filled up to npad.
// sc1 selects the agent-coherent load policy (for data other XCDs published).
template <int AUX>
__device__ __forceinline__ void stage_vec(uint8_t* dst, const uint16_t* src, int n, int npad, int tid, int nthreads) {
    const __amdgpu_buffer_rsrc_t r =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t*>(src), (short)0, n * 2, 0x00020000);
    constexpr int B = 4;  // 16-byte loads in flight per thread
    for (int c0 = 0; c0 < npad / 8; c0 += B * nthreads) {
        u32x4 v[B];
#pragma unroll
        for (int b = 0; b < B; ++b)  // chunks past n read zero
            v[b] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(r, 16 * (c0 + b * nthreads + tid), 0, AUX));
#pragma unroll
        for (int b = 0; b < B; ++b) {
            const int c = c0 + b * nthreads + tid;
            if (c < npad / 8) *reinterpret_cast<u32x4*>(dst + 16 * c) = v[b];
        }
    }
}

template <int MM>
__global__ void __launch_bounds__(256, 3) mxt_decode_kernel(MxtParams p) {
    extern __shared__ __align__(16) uint8_t smem[];
    const int tid = threadIdx.x, lane = tid & 63, wave = uniform(tid >> 6);
    const int q = lane >> 4;
    const tsa_expert_layout& L = p.L;
    const int H = (int)L.hidden, I = (int)L.inter;
    const int T = p.T, k = p.k;
    constexpr int KP = 128 * MM;  // padded vector length in LDS
    int* s_slot = reinterpret_cast<int*>(smem);                      // [MAXT*MAXK]
    float* s_w = reinterpret_cast<float*>(smem + 4 * MAXT * MAXK);   // [MAXT*MAXK]
    float* s_y = reinterpret_cast<float*>(smem + 8 * MAXT * MAXK);   // [WAVES][16]
    int* s_flag = reinterpret_cast<int*>(smem + 8 * MAXT * MAXK + 4 * WAVES * 16);
    uint8_t* vec = smem + MISC_LDS;  // phase A: x [T][KP] bf16; phase B: h [WAVES][KP] bf16

    // ---- prologue: routing / slot table on wave 0 while the other waves stage x
    const bool stage = (int)blockIdx.x < p.nA;
    if (p.logits) {
        if (wave == 0) {
            int es[4];
#pragma unroll
            for (int j = 0; j < 4; ++j) es[j] = p.expert_slot[min(lane + 64 * j, p.E - 1)];
            for (int t = 0; t < T; ++t) {
                const int sel = route_token(p, t, lane, es, s_slot, s_w);
                if (blockIdx.x == 0 && p.idx_out && lane < k) {
                    p.idx_out[t * k + lane] = sel;
                    p.w_out[t * k + lane] = s_w[t * k + lane];
                }
            }
        } else if (stage) {
            for (int t = 0; t < T; ++t) stage_vec<0>(vec + t * KP * 2, p.x + (int64_t)t * H, H, KP, tid - 64, 192);
        }
    } else {
        for (int i = tid; i < T * k; i += blockDim.x) {
            s_slot[i] = p.slots[i];
            s_w[i] = p.wts[i];
        }
        if (stage)
            for (int t = 0; t < T; ++t) stage_vec<0>(vec + t * KP * 2, p.x + (int64_t)t * H, H, KP, tid, 256);
    }
    if (tid == 0) s_flag[0] = 0;
    __syncthreads();

    // ---- phase A: gate_up tiles -> SwiGLU -> publish h (bf16)
    int task = blockIdx.x;
    const int tiles = I / 32;  // 64-row workgroup tasks per expert, 32 h values each
    for (; task < p.nA; task += p.grid) {
        const int t = task / (k * tiles), j = (task / tiles) % k, kb = task % tiles;
        const int64_t slot = uniform(s_slot[t * k + j]);
        const bool live = slot >= 0 && slot < p.n_slots;
        const int64_t row0 = (int64_t)kb * 64 + 16 * wave;
        uint32_t packed = 0;  // bf16 h rows row0/2 + 2q, +1
        if (live) {
            const uint8_t* base = p.pool + slot * L.slot_bytes;
            const int64_t tile = row0 / 16;
            const bool hb = L.gate_bias_off >= 0;
            u32x4 braw = u32x4{0u, 0u, 0u, 0u};
            if (hb) braw = bias_raw(base + L.gate_bias_off, L.bias_dtype, 2 * (int64_t)I, row0 + 4 * q);
            Tile<MM> tl;
            tile_load<MM>(tl, base + L.gate_off + tile * p.gu_tile, p.gu_tile, base + L.gate_scales_off + tile * p.gu_stile,
                          p.gu_stile, lane);
            v4f r = tile_mfma<MM>(tl, vec + t * KP * 2, lane);
            if (hb) r += bias_value(braw, L.bias_dtype);
            const float h0 = swiglu_oai(L, r[0], r[1]), h1 = swiglu_oai(L, r[2], r[3]);
            packed = (uint32_t)f32_to_bf16_bits(h0) | ((uint32_t)f32_to_bf16_bits(h1) << 16);
        }
        if ((lane & 15) == 0)
            __hip_atomic_store(reinterpret_cast<uint32_t*>(p.h + (int64_t)(t * k + j) * I + row0 / 2 + 2 * q), packed,
                               __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __builtin_amdgcn_s_waitcnt(0);  // this wave's h stores are complete ...
        __syncthreads();                // ... and so are the other waves' before the flag is set
        if (tid == 0)
            __hip_atomic_store(&p.flags[(t * k + j) * WS_FLAG_WORDS + kb], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }

    // ---- phase B: down tiles of every selected expert, weighted sum in a fixed order
    bool did_b = false;
    unsigned tok_ready = 0;  // tokens whose k pairs this workgroup has seen complete (workgroup-uniform)
    const int RB = H / 16;
    const int rounds = (k + WAVES - 1) / WAVES;
    uint8_t* hs = vec + wave * KP * 2;
    {
        int bt = (int)blockIdx.x - p.b_off;
        if (bt < 0) bt += p.grid;
        task = p.nA + bt;
    }
    for (; task < p.nA + p.nB; task += p.grid) {
        did_b = true;
        const int b = task - p.nA;
        const int t = b / RB;
        const int64_t n0 = (int64_t)(b % RB) * 16;
        v4f yv = v4f{0.0f, 0.0f, 0.0f, 0.0f};  // rows n0 + 4q .. +3, weighted sum over this wave's experts
        for (int rd = 0; rd < rounds; ++rd) {
            const int j = rd * WAVES + wave;
            const int64_t slot = j < k ? uniform(s_slot[t * k + j]) : -1;
            const bool live = slot >= 0 && slot < p.n_slots;
            const bool hb = L.down_bias_off >= 0;
            const uint8_t* base = p.pool + (live ? slot : 0) * L.slot_bytes;
            const int64_t tile = n0 / 16;
            u32x4 braw = u32x4{0u, 0u, 0u, 0u};
            Tile<MM> tl;
            if (live) {
                if (hb) braw = bias_raw(base + L.down_bias_off, L.bias_dtype, (int64_t)H, n0 + 4 * q);
                tile_load<MM>(tl, base + L.down_off + tile * p.dn_tile, p.dn_tile,
                              base + L.down_scales_off + tile * p.dn_stile, p.dn_stile, lane);
            }
            if (rd == 0 && !((tok_ready >> t) & 1)) {
                // The round's weights are in flight; wave 0 alone waits for the token's k pairs
                // (one poller per workgroup: polls of hot counter lines compete with the
                // weight stream, so they are few and spaced), the others wait at the barrier.
                if (wave == 0) {
                    for (int jj = 0; jj < k; ++jj) {
                        const int sj = uniform(s_slot[t * k + jj]);
                        if (sj < 0 || sj >= p.n_slots) continue;  // a dead pair's h is never read
                        unsigned* f = p.flags + (t * k + jj) * WS_FLAG_WORDS;
                        int spins = 0;
                        for (;;) {
                            bool done = true;
                            for (int i = lane; i < tiles; i += 64) done &= ld_relaxed(f + i) != 0u;
                            if (__all(done)) break;
                            __builtin_amdgcn_s_sleep(8);
                            if (++spins > SPIN_LIMIT) {
                                __hip_atomic_store(&p.bar[2], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                                s_flag[0] = 1;
                                break;
                            }
                        }
                    }
                }
                __syncthreads();
                tok_ready |= 1u << t;
            }
            if (live) {
                const int pair = t * k + j;
                // h of (t, j) -> this wave's LDS area (sc1: coherent with other XCDs' stores)
                stage_vec<16>(hs, p.h + (int64_t)pair * I, I, KP, lane, 64);
                __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
                __builtin_amdgcn_wave_barrier();
                __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
                v4f r = tile_mfma<MM>(tl, hs, lane);
                if (hb) r += bias_value(braw, L.bias_dtype);
                yv += s_w[pair] * r;
            }
        }
        if ((lane & 15) == 0)
            *reinterpret_cast<v4f*>(s_y + wave * 16 + 4 * q) = yv;
        __syncthreads();
        if (wave == 0 && lane < 16) {
            float sum = 0.0f;
#pragma unroll
            for (int w = 0; w < WAVES; ++w) sum += s_y[w * 16 + lane];
            store_out(p.y, p.y_dtype, (int64_t)t * H + n0 + lane, sum);
        }
        const bool aborted = s_flag[0] != 0;  // written before the barrier above
        __syncthreads();
        if (aborted) break;
    }
    // ---- leave: the last phase B workgroup out clears the flags for the next launch
    if (did_b) {
        if (tid == 0) {
            const unsigned nbw = (unsigned)(p.nB < p.grid ? p.nB : p.grid);
            const unsigned done = __hip_atomic_fetch_add(&p.bar[1], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            s_flag[1] = done == nbw - 1;
        }
        __syncthreads();
        if (s_flag[1]) {
            for (int i = tid; i < T * k * WS_FLAG_WORDS; i += blockDim.x)
                __hip_atomic_store(&p.flags[i], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            if (tid == 0) __hip_atomic_store(&p.bar[1], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
    }
}

const void* kernel_for_mm(int MM) {
    switch (MM) {
        case 4: return reinterpret_cast<const void*>(&mxt_decode_kernel<4>);
        case 8: return reinterpret_cast<const void*>(&mxt_decode_kernel<8>);
        case 16: return reinterpret_cast<const void*>(&mxt_decode_kernel<16>);
        case 24: return reinterpret_cast<const void*>(&mxt_decode_kernel<24>);
        default: return nullptr;
    }
}

int pick_mm(int64_t groups) {
    for (int mm : {4, 8, 16, 24})
        if (groups <= mm) return mm;
    return 0;
}

}  // namespace

// Bytes of bf16 h the tiled decode publishes in the workspace (after the header).
int64_t mxt_ws_bytes(const tsa_expert_layout& L, int64_t T, int k) { return (T * k * L.inter * 2 + 255) / 256 * 256; }

// Requirements of the tiled fused path beyond validate_layout: "" if met.
const char* mxt_unsupported(const tsa_expert_layout& L) {
    if (L.format != TSA_EXPERT_MXFP4 || L.act != TSA_ACT_SWIGLU_OAI) return "tiled layouts need MXFP4 experts with the SwiGLU-OAI activation";
    if (L.hidden % 32 || L.inter % 32) return "tiled layouts need hidden and inter to be multiples of 32";
    if (!pick_mm(mx_tile_groups(L.hidden)) || !pick_mm(mx_tile_groups(L.inter))) return "tiled layouts support hidden, inter <= 3072";
    if ((L.slot_bytes | L.gate_off | L.down_off | L.gate_scales_off | L.down_scales_off) & 15)
        return "tiled layouts need 16-byte aligned slots and matrix offsets";
    if (L.gate_bias_off >= 0 && (L.gate_bias_off | L.down_bias_off) & 15) return "tiled layouts need 16-byte aligned biases";
    return "";
}

// Enqueue the tiled fused kernel for T <= 4 tokens, k <= 16 (the caller checked the
// layout with mxt_unsupported and the pointers' alignment).
int mxt_fused_decode(const tsa_expert_layout& L, const uint8_t* pool, int64_t n_slots, const int32_t* slots,
                     const float* wts, const void* logits, int logits_dtype, int mode, const int32_t* expert_slot,
                     int64_t E, int32_t* idx_out, float* w_out, int64_t T, int k, const void* x, void* y, int y_dtype,
                     uint8_t* ws, int64_t ws_bytes, hipStream_t st) {
    TSA_REQUIRE(T >= 1 && T <= MAXT && k >= 1 && k <= MAXK, TSA_ERR_SHAPE, "tiled decode launch: T %lld, k %d",
                (long long)T, k);
    TSA_REQUIRE(!logits || E <= 256, TSA_ERR_SHAPE, "fused routing supports E <= 256 (got %lld)", (long long)E);
    TSA_REQUIRE(ws_bytes >= WS_HDR + mxt_ws_bytes(L, T, k), TSA_ERR_WORKSPACE, "workspace too small for the tiled decode");
    const int64_t ma = mx_tile_groups(L.hidden), mb = mx_tile_groups(L.inter);
    const int MM = pick_mm(ma > mb ? ma : mb);
    const void* kfn = kernel_for_mm(MM);
    TSA_REQUIRE(kfn, TSA_ERR_SHAPE, "tiled decode: unsupported sizes");
    const int64_t vec_bytes = 256 * (int64_t)MM * (T > WAVES ? T : WAVES);
    const size_t lds = MISC_LDS + (size_t)vec_bytes;

    MxtParams p{};
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
    p.bar = reinterpret_cast<unsigned*>(ws);
    p.flags = reinterpret_cast<unsigned*>(ws + WS_FLAG_OFF);
    p.h = reinterpret_cast<uint16_t*>(ws + WS_HDR);
    p.nA = (int)(T * k * (L.inter / 32));
    p.nB = (int)(T * (L.hidden / 16));
    p.gu_tile = 8 * L.hidden;
    p.gu_stile = mx_tile_scale_bytes(L.hidden);
    p.dn_tile = 8 * L.inter;
    p.dn_stile = mx_tile_scale_bytes(L.inter);

    int per_cu = 0;
    TSA_HIP_CHECK(hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kfn, 256, lds));
    const int cus = num_cus();
    TSA_REQUIRE(per_cu > 0 && cus > 0, TSA_ERR_HIP, "tiled decode kernel cannot be resident (lds %zu)", lds);
    const int resident = per_cu * cus;
    // One workgroup per gate_up task (when they fit): each runs its phase B task after its
    // phase A task, so down-tile loads are issued behind that workgroup's gate_up loads and
    // the gate_up stream, which every phase B task waits for, is served first. Phase B task
    // 0 goes to workgroup grid % cus: workgroups b and b + cus share a CU, so the first
    // grid % cus CUs already hold two phase A tasks and the phase B tasks go to the others
    // first (measured at 19.6 us per layer-token against 21.6 with one task per workgroup).
    const int need = p.nA > p.nB ? p.nA : p.nB;
    p.grid = need < resident ? need : resident;
    p.b_off = p.grid % cus;
    void* args[] = {&p};
    TSA_HIP_CHECK(hipLaunchKernel(kfn, dim3(p.grid), dim3(256), args, lds, st));
    return TSA_OK;
}

}  // namespace tsa
