// Fused top-k MoE decode over resident packed expert slots.
//
// Phase A (one launch for every (token, j) assignment and every block of the
// intermediate dimension): gate/up rows of the selected expert -> activation
// (GPT-OSS clamped SwiGLU or SiLU-gated) -> h[t, j, :] (float32, workspace).
// Phase B (one launch over tokens x output rows): each workgroup owns a block of
// output rows for one token and sums w[t, j] * (W_down[slot_j] h[t, j] + b_down)
// over j in registers, so every output element has exactly one writer (no atomics,
// deterministic order). Slots < 0 (or >= n_slots) contribute nothing.
//
// Semantics: tinyserve/_model_hooks.py:380-394 (MXFP4 expert with biases),
// tinyserve/ggml_forward.py:88-115 (GGUF expert), tinyserve/csrc/expert_loop.cpp:83-121
// (weighted top-k accumulation).
#include "rowdot.h"

#include <atomic>
#include <mutex>

namespace tsa {
namespace {

constexpr int H_PER_WG = 8;     // phase A: intermediate outputs per workgroup (2 per wave)
constexpr int ROWS_B_PER_WG = 8;  // phase B: output rows per workgroup (2 per wave)

__device__ __forceinline__ float activate(const tsa_expert_layout& L, float gate, float up) {
    if (L.act == TSA_ACT_SWIGLU_OAI) {
        const float g = fminf(gate, L.swiglu_limit);
        const float u = fminf(fmaxf(up, -L.swiglu_limit), L.swiglu_limit);
        return (u + 1.0f) * g * sigmoidf_(L.swiglu_alpha * g);
    }
    return gate * sigmoidf_(gate) * up;
}

__device__ __forceinline__ const uint8_t* slot_ptr(const uint8_t* pool, const tsa_expert_layout& L, int64_t slot) {
    return pool + slot * L.slot_bytes;
}

__device__ __forceinline__ void stage(float* xs, const void* x, int dt, int64_t off, int64_t n) {
    for (int64_t i = threadIdx.x; i < n; i += blockDim.x) xs[i] = load_act(x, dt, off + i);
}

// ---------------------------------------------------------------- MXFP4
template <int A>
__global__ void __launch_bounds__(256) mx_phase_a(tsa_expert_layout L, const uint8_t* __restrict__ pool,
                                                  int64_t n_slots, const int32_t* __restrict__ slots, int k,
                                                  const void* __restrict__ x, int x_dtype, float* __restrict__ h) {
    extern __shared__ float xs[];
    const int64_t a = blockIdx.y;  // assignment t*k + j
    const int64_t slot = slots[a];
    if (slot < 0 || slot >= n_slots) return;
    const int64_t H = L.hidden, I = L.inter, t = a / k;
    stage(xs, x, x_dtype, t * H, H);
    __syncthreads();
    const uint8_t* base = slot_ptr(pool, L, slot);
    const uint8_t* bl = base + L.gate_off;
    const uint8_t* sc = base + L.gate_scales_off;
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int64_t G = H / 32;
    for (int r = wave; r < H_PER_WG; r += 4) {
        const int64_t i = (int64_t)blockIdx.x * H_PER_WG + r;
        if (i >= I) break;
        float pg = mx_row_partial<A>(bl, sc, 2 * i, G, xs, lane);
        float pu = mx_row_partial<A>(bl, sc, 2 * i + 1, G, xs, lane);
        pg = wave_sum(pg);
        pu = wave_sum(pu);
        if (lane == 0) {
            if (L.gate_bias_off >= 0) {
                pg += load_act(base + L.gate_bias_off, L.bias_dtype, 2 * i);
                pu += load_act(base + L.gate_bias_off, L.bias_dtype, 2 * i + 1);
            }
            h[a * I + i] = activate(L, pg, pu);
        }
    }
}

template <int A>
__global__ void __launch_bounds__(256) mx_phase_b(tsa_expert_layout L, const uint8_t* __restrict__ pool,
                                                  int64_t n_slots, const int32_t* __restrict__ slots,
                                                  const float* __restrict__ wts, int k, const float* __restrict__ h,
                                                  void* __restrict__ y, int y_dtype) {
    extern __shared__ float hs[];
    const int64_t t = blockIdx.y, H = L.hidden, I = L.inter, G = I / 32;
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    float acc[ROWS_B_PER_WG / 4] = {};
    for (int j = 0; j < k; ++j) {
        const int64_t a = t * k + j, slot = slots[a];
        if (slot < 0 || slot >= n_slots) continue;  // uniform across the workgroup
        const float wj = wts[a];
        __syncthreads();
        stage(hs, h, TSA_F32, a * I, I);
        __syncthreads();
        const uint8_t* base = slot_ptr(pool, L, slot);
#pragma unroll
        for (int rr = 0; rr < ROWS_B_PER_WG / 4; ++rr) {
            const int64_t n = (int64_t)blockIdx.x * ROWS_B_PER_WG + wave + 4 * rr;
            if (n >= H) break;
            float p = wave_sum(mx_row_partial<A>(base + L.down_off, base + L.down_scales_off, n, G, hs, lane));
            if (L.down_bias_off >= 0) p += load_act(base + L.down_bias_off, L.bias_dtype, n);
            acc[rr] += wj * p;
        }
    }
#pragma unroll
    for (int rr = 0; rr < ROWS_B_PER_WG / 4; ++rr) {
        const int64_t n = (int64_t)blockIdx.x * ROWS_B_PER_WG + wave + 4 * rr;
        if (n < H && lane == 0) store_out(y, y_dtype, t * H + n, acc[rr]);
    }
}

// ---------------------------------------------------------------- GGUF
template <int TG, int AG>
__global__ void __launch_bounds__(256) gguf_phase_a(tsa_expert_layout L, const uint8_t* __restrict__ pool,
                                                    int64_t n_slots, const int32_t* __restrict__ slots, int k,
                                                    const void* __restrict__ x, int x_dtype, float* __restrict__ h) {
    extern __shared__ float xs[];
    const int64_t a = blockIdx.y;
    const int64_t slot = slots[a];
    if (slot < 0 || slot >= n_slots) return;
    const int64_t H = L.hidden, I = L.inter, t = a / k;
    stage(xs, x, x_dtype, t * H, H);
    __syncthreads();
    const uint8_t* base = slot_ptr(pool, L, slot);
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    for (int r = wave; r < H_PER_WG; r += 4) {
        const int64_t i = (int64_t)blockIdx.x * H_PER_WG + r;
        if (i >= I) break;
        const float pg = wave_sum(gguf_row_partial<TG, AG>(base + L.gate_off, i, H, xs, lane));
        const float pu = wave_sum(gguf_row_partial<TG, AG>(base + L.up_off, i, H, xs, lane));
        if (lane == 0) h[a * I + i] = activate(L, pg, pu);
    }
}

template <int TD, int AD>
__global__ void __launch_bounds__(256) gguf_phase_b(tsa_expert_layout L, const uint8_t* __restrict__ pool,
                                                    int64_t n_slots, const int32_t* __restrict__ slots,
                                                    const float* __restrict__ wts, int k, const float* __restrict__ h,
                                                    void* __restrict__ y, int y_dtype) {
    extern __shared__ float hs[];
    const int64_t t = blockIdx.y, H = L.hidden, I = L.inter;
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    float acc[ROWS_B_PER_WG / 4] = {};
    for (int j = 0; j < k; ++j) {
        const int64_t a = t * k + j, slot = slots[a];
        if (slot < 0 || slot >= n_slots) continue;
        const float wj = wts[a];
        __syncthreads();
        stage(hs, h, TSA_F32, a * I, I);
        __syncthreads();
        const uint8_t* base = slot_ptr(pool, L, slot);
#pragma unroll
        for (int rr = 0; rr < ROWS_B_PER_WG / 4; ++rr) {
            const int64_t n = (int64_t)blockIdx.x * ROWS_B_PER_WG + wave + 4 * rr;
            if (n >= H) break;
            acc[rr] += wj * wave_sum(gguf_row_partial<TD, AD>(base + L.down_off, n, I, hs, lane));
        }
    }
#pragma unroll
    for (int rr = 0; rr < ROWS_B_PER_WG / 4; ++rr) {
        const int64_t n = (int64_t)blockIdx.x * ROWS_B_PER_WG + wave + 4 * rr;
        if (n < H && lane == 0) store_out(y, y_dtype, t * H + n, acc[rr]);
    }
}

// ---------------------------------------------------------------- host side
struct Launch {
    dim3 ga, gb;
    size_t lds_a, lds_b;
};

Launch shapes(const tsa_expert_layout& L, int64_t T, int k) {
    Launch s;
    s.ga = dim3((unsigned)((L.inter + H_PER_WG - 1) / H_PER_WG), (unsigned)(T * k));
    s.gb = dim3((unsigned)((L.hidden + ROWS_B_PER_WG - 1) / ROWS_B_PER_WG), (unsigned)T);
    s.lds_a = (size_t)L.hidden * 4;
    s.lds_b = (size_t)L.inter * 4;
    return s;
}

template <int TG, int AG>
hipError_t launch_gguf_a(const Launch& s, const tsa_expert_layout& L, const uint8_t* pool, int64_t n_slots,
                         const int32_t* slots, int k, const void* x, int xdt, float* h, hipStream_t st) {
    hipLaunchKernelGGL((gguf_phase_a<TG, AG>), s.ga, dim3(256), s.lds_a, st, L, pool, n_slots, slots, k, x, xdt, h);
    return hipGetLastError();
}

template <int TD, int AD>
hipError_t launch_gguf_b(const Launch& s, const tsa_expert_layout& L, const uint8_t* pool, int64_t n_slots,
                         const int32_t* slots, const float* w, int k, const float* h, void* y, int ydt, hipStream_t st) {
    hipLaunchKernelGGL((gguf_phase_b<TD, AD>), s.gb, dim3(256), s.lds_b, st, L, pool, n_slots, slots, w, k, h, y, ydt);
    return hipGetLastError();
}

}  // namespace

int64_t mx_fused_ws_bytes(const tsa_expert_layout& L, int64_t T, int k);
int64_t mxt_ws_bytes(const tsa_expert_layout& L, int64_t T, int k);
const char* gq_unsupported(const tsa_expert_layout& L);
int gq_decode(const tsa_expert_layout& L, const uint8_t* pool, int64_t n_slots, const int32_t* slots, const float* wts,
              const void* logits, int logits_dtype, int mode, const int32_t* expert_slot, int64_t E, int32_t* idx_out,
              float* w_out, int64_t T, int k, const void* x, int x_dtype, void* y, int y_dtype, uint8_t* ws,
              int64_t ws_bytes, hipStream_t st);

// GGUF experts with 2-byte aligned tensors, one gate/up type and k <= 16 run on the
// super-block streaming kernels of moe_decode_gq.hip; the row kernels below cover the rest.
// The super-block GGUF decode covers 2-byte aligned slots, k <= 16 and T k <= 65535 (one
// grid row per assignment); other calls take the per-row kernels.
static bool use_gq(const tsa_expert_layout& L, const uint8_t* pl, int64_t T, int k) {
    const bool a2 = ((reinterpret_cast<uintptr_t>(pl) | L.slot_bytes | L.gate_off | L.up_off | L.down_off) & 1) == 0;
    return L.format == TSA_EXPERT_GGUF && a2 && k <= 16 && T * k <= 65535 && !*gq_unsupported(L);
}
int mx_fused_decode(const tsa_expert_layout& L, const uint8_t* pool, int64_t n_slots, const int32_t* slots,
                    const float* wts, const void* logits, int logits_dtype, int mode, const int32_t* expert_slot,
                    int64_t E, int32_t* idx_out, float* w_out, int64_t T, int k, const void* x, int x_dtype, void* y,
                    int y_dtype, uint8_t* ws, int64_t ws_bytes, hipStream_t st);
int64_t mx_tile_scale_bytes(int64_t K);
const char* mxt_unsupported(const tsa_expert_layout& L);
int mxt_decode(const tsa_expert_layout& L, const uint8_t* pool, int64_t n_slots, const int32_t* slots,
               const float* wts, const void* logits, int logits_dtype, int mode, const int32_t* expert_slot, int64_t E,
               int32_t* idx_out, float* w_out, int64_t T, int k, const void* x, void* y, int y_dtype, uint8_t* sync,
               uint8_t* ws, int64_t ws_bytes, hipStream_t st);

// Workspace: the sync area of the one-launch MXFP4 decode (MXT_SYNC_BYTES), then the
// intermediate h of every path (float [T, k, I] at most), then int32 slots / ids and float
// weights [T, k] for routed calls. Only the sync area carries state from one call to the
// next; it needs one value in every 32-bit word before the first call (zero it).
static int64_t h_region(const tsa_expert_layout& L, int64_t T, int k) {
    const int64_t v1 = (T * k * L.inter * 4 + 255) / 256 * 256;
    const int64_t fu = mx_fused_ws_bytes(L, T, k), ti = mxt_ws_bytes(L, T, k);
    return v1 > fu ? (v1 > ti ? v1 : ti) : (fu > ti ? fu : ti);
}
static int64_t ws_bytes(const tsa_expert_layout& L, int64_t T, int k) {
    return MXT_SYNC_BYTES + h_region(L, T, k) + 3 * ((T * k * 4 + 255) / 256 * 256);
}

namespace {
std::atomic<int> g_mxt_form{1};
std::atomic<uint32_t> g_mxt_wait_limit{1u << 18};
}  // namespace
int mxt_form() { return g_mxt_form.load(std::memory_order_relaxed); }
uint32_t mxt_wait_limit() { return g_mxt_wait_limit.load(std::memory_order_relaxed); }

int validate_layout(const tsa_expert_layout* L) {
    TSA_REQUIRE(L != nullptr, TSA_ERR_INVALID_ARG, "layout is null");
    TSA_REQUIRE(L->format == TSA_EXPERT_MXFP4 || L->format == TSA_EXPERT_GGUF, TSA_ERR_INVALID_ARG,
                "layout.format %d is not MXFP4(1) or GGUF(2)", L->format);
    TSA_REQUIRE(L->act == TSA_ACT_SILU || L->act == TSA_ACT_SWIGLU_OAI, TSA_ERR_INVALID_ARG, "layout.act %d unknown",
                L->act);
    TSA_REQUIRE(L->hidden > 0 && L->inter > 0 && L->slot_bytes > 0, TSA_ERR_SHAPE, "layout sizes must be positive");
    TSA_REQUIRE(L->hidden % 32 == 0 && L->inter % 32 == 0, TSA_ERR_SHAPE,
                "hidden (%lld) and intermediate (%lld) sizes must be multiples of 32", (long long)L->hidden,
                (long long)L->inter);
    TSA_REQUIRE(L->hidden * 4 <= 64 * 1024 && L->inter * 4 <= 64 * 1024, TSA_ERR_SHAPE,
                "hidden/intermediate sizes above 16384 are not supported");
    TSA_REQUIRE(L->prefill_mfma == TSA_PREFILL_FP6 || L->prefill_mfma == TSA_PREFILL_BF16, TSA_ERR_INVALID_ARG,
                "layout.prefill_mfma %d unknown", L->prefill_mfma);
    TSA_REQUIRE(L->mx_tiled == 0 || (L->mx_tiled == 1 && L->format == TSA_EXPERT_MXFP4), TSA_ERR_INVALID_ARG,
                "layout.mx_tiled must be 0, or 1 for MXFP4 experts (got %d)", L->mx_tiled);
    if (L->mx_tiled) {
        const char* why = mxt_unsupported(*L);
        TSA_REQUIRE(!*why, TSA_ERR_SHAPE, "%s", why);
    }
    if (L->format == TSA_EXPERT_MXFP4) {
        const int64_t H = L->hidden, I = L->inter;
        const bool tl = L->mx_tiled != 0;
        const int64_t need[4][2] = {{L->gate_off, 2 * I * H / 2},
                                    {L->gate_scales_off, tl ? 2 * I / 16 * mx_tile_scale_bytes(H) : 2 * I * H / 32},
                                    {L->down_off, H * I / 2},
                                    {L->down_scales_off, tl ? H / 16 * mx_tile_scale_bytes(I) : H * I / 32}};
        for (auto& r : need)
            TSA_REQUIRE(r[0] >= 0 && r[0] + r[1] <= L->slot_bytes, TSA_ERR_WEIGHT_TOO_SMALL,
                        "tensor at offset %lld (%lld bytes) exceeds slot_bytes %lld", (long long)r[0],
                        (long long)r[1], (long long)L->slot_bytes);
        if (L->gate_bias_off >= 0 || L->down_bias_off >= 0) {
            TSA_REQUIRE(valid_dtype(L->bias_dtype), TSA_ERR_INVALID_ARG, "bad bias dtype %d", L->bias_dtype);
            const int bs = dtype_size(L->bias_dtype);
            TSA_REQUIRE((L->gate_bias_off < 0 || L->gate_bias_off % bs == 0) &&
                            (L->down_bias_off < 0 || L->down_bias_off % bs == 0) && L->slot_bytes % bs == 0,
                        TSA_ERR_INVALID_ARG, "bias offsets and slot_bytes must be multiples of the bias element size");
            TSA_REQUIRE(L->gate_bias_off < 0 || L->gate_bias_off + 2 * I * bs <= L->slot_bytes,
                        TSA_ERR_WEIGHT_TOO_SMALL, "gate_up bias exceeds the slot");
            TSA_REQUIRE(L->down_bias_off < 0 || L->down_bias_off + H * bs <= L->slot_bytes, TSA_ERR_WEIGHT_TOO_SMALL,
                        "down bias exceeds the slot");
        }
    } else {
        int be, ts;
        const int types[3] = {L->gate_type, L->up_type, L->down_type};
        const int64_t offs[3] = {L->gate_off, L->up_off, L->down_off};
        for (int i = 0; i < 3; ++i) {
            TSA_REQUIRE(gguf_geometry(types[i], &be, &ts), TSA_ERR_UNSUPPORTED_TYPE,
                        "Unsupported ggml_type: %d. Supported: Q8_0(8), Q4_K(12), Q5_K(13), Q6_K(14)", types[i]);
            TSA_REQUIRE((L->hidden * L->inter) % be == 0, TSA_ERR_SHAPE, "matrix is not a whole number of blocks");
            const int64_t nbytes = L->hidden * L->inter / be * ts;
            TSA_REQUIRE(offs[i] >= 0 && offs[i] + nbytes <= L->slot_bytes, TSA_ERR_WEIGHT_TOO_SMALL,
                        "weight_data too small: projection %d needs bytes [%lld, %lld) of a %lld-byte slot", i,
                        (long long)offs[i], (long long)(offs[i] + nbytes), (long long)L->slot_bytes);
        }
        TSA_REQUIRE(L->gate_type == L->up_type, TSA_ERR_UNSUPPORTED_TYPE,
                    "the fused decode needs gate and up in one ggml type (got %d and %d)", L->gate_type, L->up_type);
    }
    return TSA_OK;
}

}  // namespace tsa

using namespace tsa;

static int two_launch_decode(const tsa_expert_layout& L, const uint8_t* pl, int64_t n_slots, const int32_t* slots,
                             const float* weights, int64_t T, int k, const void* x, int x_dtype, void* y, int y_dtype,
                             uint8_t* ws, hipStream_t st);

__global__ void __launch_bounds__(256) tsa_map_slots_kernel(const int32_t* __restrict__ idx, int64_t n,
                                                             const int32_t* __restrict__ expert_slot, int64_t E,
                                                             int32_t* __restrict__ slots) {
    const int64_t a = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (a >= n) return;
    const int e = idx[a];
    slots[a] = (e >= 0 && e < E) ? expert_slot[e] : -1;
}

// Checkpoint-order MXFP4 pools that the MFMA decode takes (bf16 activations, the layout's
// sizes and 16-byte alignment, the pool and x aligned); others keep mx_fused_decode.
static bool mxt_checkpoint_ok(const tsa_expert_layout& L, const uint8_t* pl, const void* x, int x_dtype, int k) {
    return L.format == TSA_EXPERT_MXFP4 && !L.mx_tiled && x_dtype == TSA_BF16 && k <= 16 && !*mxt_unsupported(L) &&
           ((reinterpret_cast<uintptr_t>(pl) | reinterpret_cast<uintptr_t>(x)) & 15) == 0;
}

// Tiled MXFP4 layouts (and checkpoint-order ones, mxt_checkpoint_ok): the MFMA decode over
// chunks of up to 4 tokens (stream-ordered on the shared workspace).
static int tiled_decode(const tsa_expert_layout& L, const uint8_t* pl, int64_t n_slots, const int32_t* slots,
                        const float* weights, const void* logits, int logits_dtype, int mode,
                        const int32_t* expert_slot, int64_t E, int32_t* idx_out, float* w_out, int64_t T, int k,
                        const void* x, int x_dtype, void* y, int y_dtype, uint8_t* sync, uint8_t* ws,
                        int64_t ws_bytes, hipStream_t st) {
    TSA_REQUIRE(x_dtype == TSA_BF16, TSA_ERR_INVALID_ARG, "tiled MXFP4 experts take bf16 activations (got dtype %d)",
                x_dtype);
    TSA_REQUIRE(k <= 16, TSA_ERR_SHAPE, "tiled MXFP4 decode supports top-k <= 16 (got %d)", k);
    const int64_t H = L.hidden, ys = dtype_size(y_dtype);
    for (int64_t t0 = 0; t0 < T; t0 += 4) {
        const int64_t tc = T - t0 < 4 ? T - t0 : 4;
        const void* lg = logits ? static_cast<const uint8_t*>(logits) + t0 * E * dtype_size(logits_dtype) : nullptr;
        int rc = mxt_decode(L, pl, n_slots, slots ? slots + t0 * k : nullptr, weights ? weights + t0 * k : nullptr, lg,
                            logits_dtype, mode, expert_slot, E, idx_out ? idx_out + t0 * k : nullptr,
                            w_out ? w_out + t0 * k : nullptr, tc, k, static_cast<const uint16_t*>(x) + t0 * H,
                            static_cast<uint8_t*>(y) + t0 * H * ys, y_dtype, sync, ws, ws_bytes, st);
        if (rc) return rc;
    }
    return TSA_OK;
}

extern "C" int tsa_moe_decode_workspace_size(const tsa_expert_layout* layout, int64_t T, int k, int64_t* bytes) {
    clear_error();
    int rc = validate_layout(layout);
    if (rc) return rc;
    TSA_REQUIRE(T >= 0 && k >= 1 && bytes, TSA_ERR_INVALID_ARG, "bad T/k/bytes");
    *bytes = ws_bytes(*layout, T, k);
    return TSA_OK;
}

extern "C" int tsa_moe_decode(const tsa_expert_layout* layout, const void* pool, int64_t n_slots, const int32_t* slots,
                              const float* weights, int64_t T, int k, const void* x, int x_dtype, void* y, int y_dtype,
                              void* workspace, int64_t workspace_bytes, void* stream) {
    clear_error();
    int rc = validate_layout(layout);
    if (rc) return rc;
    const tsa_expert_layout& L = *layout;
    TSA_REQUIRE(valid_dtype(x_dtype) && valid_dtype(y_dtype), TSA_ERR_INVALID_ARG, "bad dtype (x %d, y %d)", x_dtype,
                y_dtype);
    TSA_REQUIRE(T >= 0 && k >= 1 && k <= 64 && n_slots >= 0, TSA_ERR_INVALID_ARG, "bad T (%lld) / k (%d) / n_slots",
                (long long)T, k);
    if (T == 0) return TSA_OK;
    TSA_REQUIRE(pool && slots && weights && x && y, TSA_ERR_INVALID_ARG, "null pointer");
    TSA_REQUIRE(workspace && workspace_bytes >= ws_bytes(L, T, k), TSA_ERR_WORKSPACE,
                "workspace too small: got %lld bytes, need %lld", (long long)workspace_bytes,
                (long long)ws_bytes(L, T, k));
    hipStream_t st = as_stream(stream);
    const uint8_t* pl = static_cast<const uint8_t*>(pool);
    uint8_t* sync = static_cast<uint8_t*>(workspace);
    uint8_t* ws = sync + MXT_SYNC_BYTES;
    const int64_t wsb = workspace_bytes - MXT_SYNC_BYTES;
    if (L.mx_tiled || (T <= 64 && mxt_checkpoint_ok(L, pl, x, x_dtype, k)))
        return tiled_decode(L, pl, n_slots, slots, weights, nullptr, 0, 0, nullptr, 0, nullptr, nullptr, T, k, x,
                            x_dtype, y, y_dtype, sync, ws, wsb, st);
    if (T * k > 65535) {  // the other paths launch one grid row per assignment: token chunks
        const int64_t tc = 65535 / k;
        for (int64_t t0 = 0; t0 < T; t0 += tc) {
            const int64_t n = T - t0 < tc ? T - t0 : tc;
            rc = tsa_moe_decode(layout, pool, n_slots, slots + t0 * k, weights + t0 * k, n, k,
                                static_cast<const uint8_t*>(x) + t0 * L.hidden * dtype_size(x_dtype), x_dtype,
                                static_cast<uint8_t*>(y) + t0 * L.hidden * dtype_size(y_dtype), y_dtype, workspace,
                                workspace_bytes, stream);
            if (rc) return rc;
        }
        return TSA_OK;
    }
    rc = mx_fused_decode(L, pl, n_slots, slots, weights, nullptr, 0, 0, nullptr, 0, nullptr, nullptr, T, k, x, x_dtype,
                         y, y_dtype, ws, wsb, st);
    if (rc <= 0) return rc;
    return two_launch_decode(L, pl, n_slots, slots, weights, T, k, x, x_dtype, y, y_dtype, ws, st);
}

static int two_launch_decode(const tsa_expert_layout& L, const uint8_t* pl, int64_t n_slots, const int32_t* slots,
                             const float* weights, int64_t T, int k, const void* x, int x_dtype, void* y, int y_dtype,
                             uint8_t* ws, hipStream_t st) {
    const Launch s = shapes(L, T, k);
    float* h = reinterpret_cast<float*>(ws);
    const bool a16 = ((reinterpret_cast<uintptr_t>(pl) | L.slot_bytes | L.gate_off | L.up_off | L.down_off) & 15) == 0;
    hipError_t e = hipSuccess;
    if (L.format == TSA_EXPERT_MXFP4) {
        if (a16) {
            hipLaunchKernelGGL((mx_phase_a<16>), s.ga, dim3(256), s.lds_a, st, L, pl, n_slots, slots, k, x, x_dtype, h);
            hipLaunchKernelGGL((mx_phase_b<16>), s.gb, dim3(256), s.lds_b, st, L, pl, n_slots, slots, weights, k, h, y,
                               y_dtype);
        } else {
            hipLaunchKernelGGL((mx_phase_a<1>), s.ga, dim3(256), s.lds_a, st, L, pl, n_slots, slots, k, x, x_dtype, h);
            hipLaunchKernelGGL((mx_phase_b<1>), s.gb, dim3(256), s.lds_b, st, L, pl, n_slots, slots, weights, k, h, y,
                               y_dtype);
        }
        TSA_LAUNCH_CHECK();
        return TSA_OK;
    }
    if (use_gq(L, pl, T, k))
        return gq_decode(L, pl, n_slots, slots, weights, nullptr, 0, 0, nullptr, 0, nullptr, nullptr, T, k, x, x_dtype,
                         y, y_dtype, ws, h_region(L, T, k), st);
    const bool a2 = ((reinterpret_cast<uintptr_t>(pl) | L.slot_bytes | L.gate_off | L.up_off | L.down_off) & 1) == 0;
    switch (L.gate_type) {
        case 8: e = a2 ? launch_gguf_a<8, 2>(s, L, pl, n_slots, slots, k, x, x_dtype, h, st)
                       : launch_gguf_a<8, 1>(s, L, pl, n_slots, slots, k, x, x_dtype, h, st); break;
        case 12: e = a16 ? launch_gguf_a<12, 16>(s, L, pl, n_slots, slots, k, x, x_dtype, h, st)
                         : launch_gguf_a<12, 1>(s, L, pl, n_slots, slots, k, x, x_dtype, h, st); break;
        case 13: e = a16 ? launch_gguf_a<13, 16>(s, L, pl, n_slots, slots, k, x, x_dtype, h, st)
                         : launch_gguf_a<13, 1>(s, L, pl, n_slots, slots, k, x, x_dtype, h, st); break;
        default: e = a2 ? launch_gguf_a<14, 2>(s, L, pl, n_slots, slots, k, x, x_dtype, h, st)
                        : launch_gguf_a<14, 1>(s, L, pl, n_slots, slots, k, x, x_dtype, h, st); break;
    }
    TSA_HIP_CHECK(e);
    switch (L.down_type) {
        case 8: e = a2 ? launch_gguf_b<8, 2>(s, L, pl, n_slots, slots, weights, k, h, y, y_dtype, st)
                       : launch_gguf_b<8, 1>(s, L, pl, n_slots, slots, weights, k, h, y, y_dtype, st); break;
        case 12: e = a16 ? launch_gguf_b<12, 16>(s, L, pl, n_slots, slots, weights, k, h, y, y_dtype, st)
                         : launch_gguf_b<12, 1>(s, L, pl, n_slots, slots, weights, k, h, y, y_dtype, st); break;
        case 13: e = a16 ? launch_gguf_b<13, 16>(s, L, pl, n_slots, slots, weights, k, h, y, y_dtype, st)
                         : launch_gguf_b<13, 1>(s, L, pl, n_slots, slots, weights, k, h, y, y_dtype, st); break;
        default: e = a2 ? launch_gguf_b<14, 2>(s, L, pl, n_slots, slots, weights, k, h, y, y_dtype, st)
                        : launch_gguf_b<14, 1>(s, L, pl, n_slots, slots, weights, k, h, y, y_dtype, st); break;
    }
    TSA_HIP_CHECK(e);
    return TSA_OK;
}

// The routed decode; one_launch_ok false keeps the tiled MXFP4 decode on two launches
// whatever tsa_set_decode_options chose (the workspace's sync area is then never used).
static int decode_routed(const tsa_expert_layout* layout, const void* pool, int64_t n_slots,
                         const int32_t* expert_slot, int64_t E, const void* logits, int logits_dtype, int mode,
                         int64_t T, int k, const void* x, int x_dtype, void* y, int y_dtype, int32_t* idx_out,
                         float* w_out, void* workspace, int64_t workspace_bytes, void* stream, bool one_launch_ok) {
    clear_error();
    int rc = validate_layout(layout);
    if (rc) return rc;
    const tsa_expert_layout& L = *layout;
    TSA_REQUIRE(valid_dtype(x_dtype) && valid_dtype(y_dtype) && valid_dtype(logits_dtype), TSA_ERR_INVALID_ARG,
                "bad dtype (x %d, y %d, logits %d)", x_dtype, y_dtype, logits_dtype);
    TSA_REQUIRE(mode >= 0 && mode <= 2, TSA_ERR_INVALID_ARG, "bad routing mode %d", mode);
    TSA_REQUIRE(E >= 1 && E <= 1024 && k >= 1 && k <= 64 && k <= E && T >= 0, TSA_ERR_SHAPE,
                "bad routing shape (E %lld, k %d, T %lld)", (long long)E, k, (long long)T);
    if (T == 0) return TSA_OK;
    TSA_REQUIRE(pool && expert_slot && logits && x && y, TSA_ERR_INVALID_ARG, "null pointer");
    const int64_t need = ws_bytes(L, T, k);
    TSA_REQUIRE(workspace && workspace_bytes >= need, TSA_ERR_WORKSPACE, "workspace too small: got %lld bytes, need %lld",
                (long long)workspace_bytes, (long long)need);
    hipStream_t st = as_stream(stream);
    const uint8_t* pl = static_cast<const uint8_t*>(pool);
    uint8_t* ws = static_cast<uint8_t*>(workspace) + MXT_SYNC_BYTES;
    uint8_t* sync = one_launch_ok ? static_cast<uint8_t*>(workspace) : nullptr;
    const int64_t wsb = workspace_bytes - MXT_SYNC_BYTES;
    if ((L.mx_tiled || (T <= 64 && mxt_checkpoint_ok(L, pl, x, x_dtype, k))) && E <= 256)
        return tiled_decode(L, pl, n_slots, nullptr, nullptr, logits, logits_dtype, mode, expert_slot, E, idx_out,
                            w_out, T, k, x, x_dtype, y, y_dtype, sync, ws, wsb, st);
    if (!L.mx_tiled && T * k > 65535) {  // the row-per-assignment paths: token chunks, routed one by one
        const int64_t tc = 65535 / k;
        for (int64_t t0 = 0; t0 < T; t0 += tc) {
            const int64_t n = T - t0 < tc ? T - t0 : tc;
            rc = decode_routed(layout, pool, n_slots, expert_slot, E,
                               static_cast<const uint8_t*>(logits) + t0 * E * dtype_size(logits_dtype), logits_dtype,
                               mode, n, k, static_cast<const uint8_t*>(x) + t0 * L.hidden * dtype_size(x_dtype),
                               x_dtype, static_cast<uint8_t*>(y) + t0 * L.hidden * dtype_size(y_dtype), y_dtype,
                               idx_out ? idx_out + t0 * k : nullptr, w_out ? w_out + t0 * k : nullptr, workspace,
                               workspace_bytes, stream, one_launch_ok);
            if (rc) return rc;
        }
        return TSA_OK;
    }
    if (!L.mx_tiled) {
        rc = mx_fused_decode(L, pl, n_slots, nullptr, nullptr, logits, logits_dtype, mode, expert_slot, E, idx_out,
                             w_out, T, k, x, x_dtype, y, y_dtype, ws, wsb, st);
        if (rc <= 0) return rc;
    }
    if (use_gq(L, pl, T, k) && E <= 256 && T <= 4)
        return gq_decode(L, pl, n_slots, nullptr, nullptr, logits, logits_dtype, mode, expert_slot, E, idx_out, w_out,
                         T, k, x, x_dtype, y, y_dtype, ws, wsb, st);
    // separate routing, slot mapping and the two-launch decode
    const int64_t tk = (T * k * 4 + 255) / 256 * 256;
    uint8_t* extra = ws + h_region(L, T, k);
    int32_t* slots = reinterpret_cast<int32_t*>(extra);
    int32_t* idx = idx_out ? idx_out : reinterpret_cast<int32_t*>(extra + tk);
    float* w = w_out ? w_out : reinterpret_cast<float*>(extra + 2 * tk);
    rc = tsa_route_topk(logits, logits_dtype, T, E, k, mode, idx, w, stream);
    if (rc) return rc;
    hipLaunchKernelGGL(tsa_map_slots_kernel, dim3((unsigned)((T * k + 255) / 256)), dim3(256), 0, st, idx, T * k,
                       expert_slot, E, slots);
    TSA_LAUNCH_CHECK();
    if (L.mx_tiled)
        return tiled_decode(L, pl, n_slots, slots, w, nullptr, 0, 0, nullptr, 0, nullptr, nullptr, T, k, x, x_dtype, y,
                            y_dtype, sync, ws, wsb, st);
    return two_launch_decode(L, pl, n_slots, slots, w, T, k, x, x_dtype, y, y_dtype, ws, st);
}

extern "C" int tsa_moe_decode_routed(const tsa_expert_layout* layout, const void* pool, int64_t n_slots,
                                     const int32_t* expert_slot, int64_t E, const void* logits, int logits_dtype,
                                     int mode, int64_t T, int k, const void* x, int x_dtype, void* y, int y_dtype,
                                     int32_t* idx_out, float* w_out, void* workspace, int64_t workspace_bytes,
                                     void* stream) {
    return decode_routed(layout, pool, n_slots, expert_slot, E, logits, logits_dtype, mode, T, k, x, x_dtype, y,
                         y_dtype, idx_out, w_out, workspace, workspace_bytes, stream, true);
}

extern "C" int tsa_set_decode_options(int tiled_form, uint32_t wait_limit) {
    clear_error();
    TSA_REQUIRE(tiled_form == 0 || tiled_form == 1, TSA_ERR_INVALID_ARG, "tiled_form must be 0 or 1 (got %d)",
                tiled_form);
    g_mxt_form.store(tiled_form, std::memory_order_relaxed);
    g_mxt_wait_limit.store(wait_limit, std::memory_order_relaxed);
    return TSA_OK;
}

extern "C" int tsa_moe_decode_workspace_status(const void* workspace, int64_t workspace_bytes, int* poisoned,
                                               void* stream) {
    clear_error();
    TSA_REQUIRE(workspace && poisoned && workspace_bytes >= MXT_SYNC_BYTES, TSA_ERR_INVALID_ARG,
                "need a decode workspace (at least %lld bytes) and an output", (long long)MXT_SYNC_BYTES);
    uint32_t gen = 0;
    hipStream_t st = as_stream(stream);
    TSA_HIP_CHECK(hipMemcpyAsync(&gen, workspace, 4, hipMemcpyDeviceToHost, st));
    TSA_HIP_CHECK(hipStreamSynchronize(st));
    *poisoned = gen == MXT_GEN_POISON;
    return TSA_OK;
}

// ---- allocation-free routed decode: the workspace is a file-scope device array, one per
// GPU (held until the process ends), whose address is looked up once per device with that
// device current. Calls on one GPU share it, so calls that overlap on one GPU race (order
// them on one stream). Only its sync area carries state between calls; being zero at load,
// it needs no clearing.
static constexpr int64_t kNoAllocScratchBytes = 8ll << 20;
static __device__ __align__(256) uint8_t scratch[kNoAllocScratchBytes];

namespace {
constexpr int kMaxScratchDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxScratchDevices] = {};

// The current device's copy of `scratch` (device address).
int scratch_for_current_device(uint8_t** out) {
    int dev = -1;
    TSA_HIP_CHECK(hipGetDevice(&dev));
    TSA_REQUIRE(dev >= 0 && dev < kMaxScratchDevices, TSA_ERR_INVALID_ARG, "device %d is beyond the scratch table", dev);
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (!g_scratch_ptr[dev]) {
        void* ptr = nullptr;
        TSA_HIP_CHECK(hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch)));
        TSA_REQUIRE(ptr != nullptr, TSA_ERR_HIP, "no device address for the decode scratch");
        g_scratch_ptr[dev] = ptr;
    }
    *out = static_cast<uint8_t*>(g_scratch_ptr[dev]);
    return TSA_OK;
}
}  // namespace

extern "C" int tsa_moe_decode_routed_noalloc(const tsa_expert_layout* layout, const void* pool, int64_t n_slots,
                                             const int32_t* expert_slot, int64_t E, const void* logits,
                                             int logits_dtype, int mode, int64_t T, int k, const void* x, int x_dtype,
                                             void* y, int y_dtype, int32_t* idx_out, float* w_out, void* stream) {
    clear_error();
    int rc = validate_layout(layout);
    if (rc) return rc;
    TSA_REQUIRE(T >= 0 && k >= 1 && k <= 64, TSA_ERR_SHAPE, "bad T (%lld) / k (%d)", (long long)T, k);
    if (T == 0) return TSA_OK;
    const int64_t need = ws_bytes(*layout, T, k);
    TSA_REQUIRE(need <= kNoAllocScratchBytes, TSA_ERR_WORKSPACE,
                "the allocation-free decode has %lld scratch bytes per device; T %lld x top-%d needs %lld "
                "(use tsa_moe_decode_routed with a workspace)",
                (long long)kNoAllocScratchBytes, (long long)T, k, (long long)need);
    uint8_t* ws = nullptr;
    rc = scratch_for_current_device(&ws);
    if (rc) return rc;
    // always two launches: the shared array's sync area could not be cleared by a caller
    // after a one-launch wait gave up
    return decode_routed(layout, pool, n_slots, expert_slot, E, logits, logits_dtype, mode, T, k, x, x_dtype, y,
                         y_dtype, idx_out, w_out, ws, kNoAllocScratchBytes, stream, false);
}
