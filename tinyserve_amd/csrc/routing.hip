// Router top-k: one wave64 per token; up to 16 logits per lane (E <= 1024), or for E <= 256
// the decode kernels' DPP selection.
// Router logits (router_logits_kernel): the MoE block's linear gate ahead of it.
//
// Selection is by logit value, descending, ties to the lower expert id, NaN ranked
// above every number (as torch.topk ranks it); the softmax is monotone in the logits, so
// the selected set and order equal a top-k over the softmax probabilities
// (tinyserve/_model_hooks.py:456-473) for logits without NaN.
#include "fused_common.h"

namespace tsa {
namespace {

constexpr int MAX_PER_LANE = 16;

// (key, id) pairs: the larger key wins, equal keys go to the lower id.
__device__ __forceinline__ void argmax_merge(uint32_t& key, int& i, uint32_t okey, int oi) {
    if (okey > key || (okey == key && oi < i)) { key = okey; i = oi; }
}

__global__ void __launch_bounds__(256) route_topk_kernel(const void* __restrict__ logits, int ldt, int64_t T, int E,
                                                         int k, int mode, int32_t* __restrict__ idx,
                                                         float* __restrict__ wout) {
    const int lane = threadIdx.x & 63;
    const int64_t t = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (t >= T) return;
    float v[MAX_PER_LANE];
    float vmax = -INFINITY;
#pragma unroll
    for (int j = 0; j < MAX_PER_LANE; ++j) {
        const int e = lane + 64 * j;
        v[j] = e < E ? load_act(logits, ldt, t * E + e) : -INFINITY;
        vmax = fmaxf(vmax, v[j]);
    }
    // full-softmax denominator (modes 1, 2)
    float zsum = 0.0f;
    if (mode != TSA_ROUTE_TOPK_SOFTMAX) {
        float gmax = vmax;
#pragma unroll
        for (int off = 32; off >= 1; off >>= 1) gmax = fmaxf(gmax, __shfl_xor(gmax, off, 64));
        float s = 0.0f;
#pragma unroll
        for (int j = 0; j < MAX_PER_LANE; ++j)
            if (lane + 64 * j < E) s += expf(v[j] - gmax);
        zsum = wave_sum(s);
        vmax = gmax;
    }
    // Selection by route_key (NaN first, then descending logit), ties to the lower id. Every
    // logit's key is above the 0 a lane starts from, so with k <= E each round finds one.
    unsigned taken = 0;  // bit j: element lane + 64 j already selected
    float sel_v = 0.0f;  // lane j < k keeps the j-th selected logit
    int sel_i = 0;
    for (int r = 0; r < k; ++r) {
        uint32_t bk = 0u;
        int bi = 0x7FFFFFFF;
#pragma unroll
        for (int j = 0; j < MAX_PER_LANE; ++j) {
            const int e = lane + 64 * j;
            if (e < E && !((taken >> j) & 1u)) argmax_merge(bk, bi, route_key(v[j]), e);
        }
#pragma unroll
        for (int off = 32; off >= 1; off >>= 1) {
            const uint32_t ok = (uint32_t)__shfl_xor((int)bk, off, 64);
            const int oi = __shfl_xor(bi, off, 64);
            argmax_merge(bk, bi, ok, oi);
        }
        if ((bi & 63) == lane) taken |= 1u << (bi >> 6);
        if (lane == r) { sel_v = route_key_value(bk); sel_i = bi; }
    }
    // weights
    float wgt;
    if (mode == TSA_ROUTE_TOPK_SOFTMAX) {
        const float top = __shfl(sel_v, 0, 64);  // the first selected logit is the maximum
        const float ex = lane < k ? expf(sel_v - top) : 0.0f;
        wgt = ex / wave_sum(ex);
    } else {
        const float p = lane < k ? expf(sel_v - vmax) / zsum : 0.0f;
        wgt = mode == TSA_ROUTE_SOFTMAX_TOPK_RENORM ? p / wave_sum(p) : p;
    }
    if (lane < k) {
        idx[t * k + lane] = sel_i;
        wout[t * k + lane] = wgt;
    }
}

// E <= 256: the same selection from DPP wave maxima and ballots (route_select, as the decode
// kernels route), up to 4 logits per lane, and the weights from the selected logits.
struct RouteParams {
    const void* logits;
    int logits_dtype, route_mode, E, k;
};
__global__ void __launch_bounds__(256) route_topk_dpp_kernel(const void* __restrict__ logits, int ldt, int64_t T,
                                                             int E, int k, int mode, int32_t* __restrict__ idx,
                                                             float* __restrict__ wout) {
    const int lane = threadIdx.x & 63;
    const int64_t t = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (t >= T) return;
    const RouteParams p{logits, ldt, mode, E, k};
    float v[4];
    load4(logits, ldt, t * E, E, lane, v);
    const int es[4] = {lane, lane + 64, lane + 128, lane + 192};
    uint32_t myk;
    int mysel, myslot;
    select_topk(p, lane, v, es, k, myk, mysel, myslot);
    const float myval = route_key_value(myk);  // lane r < k: the r-th selected logit
    const float top = route_key_value((uint32_t)__builtin_amdgcn_readfirstlane((int)myk));
    float w;
    if (mode == TSA_ROUTE_SOFTMAX_TOPK) {  // full softmax, not renormalised
        float sum = 0.0f;
#pragma unroll
        for (int j = 0; j < 4; ++j)
            if (lane + 64 * j < E) sum += expf(v[j] - top);
        const float z = wave_sum(sum);  // every lane takes part in the exchange
        w = lane < k ? expf(myval - top) / z : 0.0f;
    } else {  // softmax over the k selected (= the renormalised full softmax)
        const float ex = lane < k ? expf(myval - top) : 0.0f;
        w = ex / wave_sum(ex);
    }
    if (lane < k) {
        idx[t * k + lane] = mysel;
        wout[t * k + lane] = w;
    }
}

// 8 consecutive values of a row (16-byte aligned for 2-byte dtypes, 32 for f32) as fp32.
__device__ __forceinline__ void load8(const void* base, int dtype, int64_t i, float (&v)[8]) {
    if (dtype == TSA_F32) {
        const float4 a = *reinterpret_cast<const float4*>(static_cast<const float*>(base) + i);
        const float4 b = *reinterpret_cast<const float4*>(static_cast<const float*>(base) + i + 4);
        v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w; v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
        return;
    }
    const uint4 w = *reinterpret_cast<const uint4*>(static_cast<const uint16_t*>(base) + i);
    const uint32_t u[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        const uint32_t lo = u[q] & 0xFFFFu, hi = u[q] >> 16;
        v[2 * q] = dtype == TSA_BF16 ? bf16_bits_to_f32(lo) : f16_bits_to_f32(lo);
        v[2 * q + 1] = dtype == TSA_BF16 ? bf16_bits_to_f32(hi) : f16_bits_to_f32(hi);
    }
}

// out[t, e] = sum_h x[t, h] w[e, h] (+ bias[e]), fp32 accumulation, rounded once to the
// output dtype (as the router nn.Linear computes it). Workgroup = 4 waves, wave = one
// expert row e against RT = 8 tokens: lane l takes the 8-value chunks l, l + 64, ... of the
// row (each load instruction reads 1 KB of w contiguously), each chunk is used for all 8
// tokens, and one multi-row wave reduction (wave_sum_rows<8>) finishes the 8 dot products.
constexpr int RT = 8;
__global__ void __launch_bounds__(256) router_logits_kernel(const void* __restrict__ x, int xdt, int64_t T, int H,
                                                            const void* __restrict__ w, int wdt,
                                                            const void* __restrict__ bias, int bdt, int E,
                                                            void* __restrict__ out, int odt) {
    const int lane = threadIdx.x & 63;
    const int e = (int)blockIdx.x * 4 + (int)(threadIdx.x >> 6);
    const int64_t t0 = (int64_t)blockIdx.y * RT;
    if (e >= E) return;  // whole waves
    const int nt = T - t0 < RT ? (int)(T - t0) : RT;
    float acc[RT];
#pragma unroll
    for (int r = 0; r < RT; ++r) acc[r] = 0.0f;
    for (int c = 8 * lane; c < H; c += 512) {
        float wv[8];
        load8(w, wdt, (int64_t)e * H + c, wv);
#pragma unroll
        for (int r = 0; r < RT; ++r) {
            if (r < nt) {
                float xv[8];
                load8(x, xdt, (t0 + r) * H + c, xv);
#pragma unroll
                for (int i = 0; i < 8; ++i) acc[r] = fmaf(xv[i], wv[i], acc[r]);
            }
        }
    }
    const float tot = wave_sum_rows<RT>(acc, lane);  // lane 8 r: token t0 + r
    const int r = lane >> 3;
    if ((lane & 7) == 0 && r < nt) {
        const float b = bias ? load_act(bias, bdt, e) : 0.0f;
        store_out(out, odt, (t0 + r) * E + e, tot + b);
    }
}

// The same for a decode step (T <= 4 tokens, all in one launch row): latency-bound, so each
// lane issues every load of its part of the row and of the tokens' x (chunks l, l + 64, ..,
// CH per pass: one pass for H <= 512 CH) as raw words before it converts any, one memory
// round trip instead of one per chunk. The dtypes are template arguments (WDT for w, XDT
// for x): with a runtime dtype branch around each load the compiler waits for it before the
// next, and the branchy code is fetched cold into the instruction cache on every call. Chunks
// past H are clamped to a valid address and contribute zero.
template <int DT>
__device__ __forceinline__ void raw8(const void* base, int64_t i, uint4& a, uint4& b) {
    if (DT == TSA_F32) {
        a = *reinterpret_cast<const uint4*>(static_cast<const float*>(base) + i);
        b = *reinterpret_cast<const uint4*>(static_cast<const float*>(base) + i + 4);
    } else {
        a = *reinterpret_cast<const uint4*>(static_cast<const uint16_t*>(base) + i);
    }
}
template <int DT>
__device__ __forceinline__ float raw_value(const uint4& a, const uint4& b, int j) {
    if (DT == TSA_F32) {
        const uint4& q = j < 4 ? a : b;
        return __uint_as_float((j & 3) == 0 ? q.x : (j & 3) == 1 ? q.y : (j & 3) == 2 ? q.z : q.w);
    }
    const uint32_t u = (j >> 1) == 0 ? a.x : (j >> 1) == 1 ? a.y : (j >> 1) == 2 ? a.z : a.w;
    const uint32_t h = (j & 1) ? u >> 16 : u & 0xFFFFu;
    return DT == TSA_BF16 ? bf16_bits_to_f32(h) : f16_bits_to_f32(h);
}
template <int NT, int WDT, int XDT>
__global__ void __launch_bounds__(256) router_logits_decode_kernel(const void* __restrict__ x, int H,
                                                                   const void* __restrict__ w,
                                                                   const void* __restrict__ bias, int bdt, int E,
                                                                   void* __restrict__ out, int odt) {
    constexpr int CH = 6;
    const int lane = threadIdx.x & 63;
    const int e = (int)blockIdx.x * 4 + (int)(threadIdx.x >> 6);
    if (e >= E) return;  // whole waves
    float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    for (int c0 = 0; c0 < H; c0 += 512 * CH) {
        uint4 wa[CH], wb[CH], xa[NT][CH], xb[NT][CH];
#pragma unroll
        for (int i = 0; i < CH; ++i) {
            const int c = min(c0 + 8 * lane + 512 * i, H - 8);
            raw8<WDT>(w, (int64_t)e * H + c, wa[i], wb[i]);
#pragma unroll
            for (int r = 0; r < NT; ++r) raw8<XDT>(x, (int64_t)r * H + c, xa[r][i], xb[r][i]);
        }
#pragma unroll
        for (int i = 0; i < CH; ++i) {
            const float on = c0 + 8 * lane + 512 * i < H ? 1.0f : 0.0f;  // clamped chunks add zero
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                const float wv = raw_value<WDT>(wa[i], wb[i], j) * on;
#pragma unroll
                for (int r = 0; r < NT; ++r) acc[r] = fmaf(raw_value<XDT>(xa[r][i], xb[r][i], j), wv, acc[r]);
            }
        }
    }
    const float tot = wave_sum_rows<4>(acc, lane);  // lane 16 r: token r
    const int r = lane >> 4;
    if ((lane & 15) == 0 && r < NT) {
        const float b = bias ? load_act(bias, bdt, e) : 0.0f;
        store_out(out, odt, (int64_t)r * E + e, tot + b);
    }
}

template <int NT, int WDT>
void launch_router_decode_w(const void* x, int xdt, int H, const void* w, const void* bias, int bdt, int E, void* out,
                            int odt, hipStream_t st) {
    const dim3 g((unsigned)((E + 3) / 4)), b(256);
    if (xdt == TSA_F32)
        hipLaunchKernelGGL((router_logits_decode_kernel<NT, WDT, TSA_F32>), g, b, 0, st, x, H, w, bias, bdt, E, out, odt);
    else if (xdt == TSA_F16)
        hipLaunchKernelGGL((router_logits_decode_kernel<NT, WDT, TSA_F16>), g, b, 0, st, x, H, w, bias, bdt, E, out, odt);
    else
        hipLaunchKernelGGL((router_logits_decode_kernel<NT, WDT, TSA_BF16>), g, b, 0, st, x, H, w, bias, bdt, E, out, odt);
}
template <int NT>
void launch_router_decode(const void* x, int xdt, int H, const void* w, int wdt, const void* bias, int bdt, int E,
                          void* out, int odt, hipStream_t st) {
    if (wdt == TSA_F32)
        launch_router_decode_w<NT, TSA_F32>(x, xdt, H, w, bias, bdt, E, out, odt, st);
    else if (wdt == TSA_F16)
        launch_router_decode_w<NT, TSA_F16>(x, xdt, H, w, bias, bdt, E, out, odt, st);
    else
        launch_router_decode_w<NT, TSA_BF16>(x, xdt, H, w, bias, bdt, E, out, odt, st);
}

}  // namespace
}  // namespace tsa

using namespace tsa;

extern "C" int tsa_router_logits(const void* x, int x_dtype, int64_t T, int64_t H, const void* w, int w_dtype,
                                 const void* bias, int bias_dtype, int64_t E, void* out, int out_dtype, void* stream) {
    clear_error();
    TSA_REQUIRE(valid_dtype(x_dtype) && valid_dtype(w_dtype) && valid_dtype(out_dtype) &&
                    (!bias || valid_dtype(bias_dtype)),
                TSA_ERR_INVALID_ARG, "bad dtype (x %d, w %d, bias %d, out %d)", x_dtype, w_dtype, bias_dtype,
                out_dtype);
    TSA_REQUIRE(T >= 0 && E >= 1 && E <= (1 << 20) && H >= 8 && H % 8 == 0 && H <= (1 << 20), TSA_ERR_SHAPE,
                "router shapes: T %lld, H %lld (a multiple of 8), E %lld", (long long)T, (long long)H, (long long)E);
    if (T == 0) return TSA_OK;
    TSA_REQUIRE(x && w && out, TSA_ERR_INVALID_ARG, "null pointer");
    const auto aligned = [](const void* p, int dt) {
        return (reinterpret_cast<uintptr_t>(p) & (dt == TSA_F32 ? 31u : 15u)) == 0;
    };
    TSA_REQUIRE(aligned(x, x_dtype) && aligned(w, w_dtype), TSA_ERR_INVALID_ARG,
                "x and w must be 16-byte aligned (32 for f32)");
    TSA_REQUIRE(T <= (int64_t)65535 * RT, TSA_ERR_SHAPE, "router: more than %d tokens per call", 65535 * RT);
    if (T <= 4) {
        hipStream_t st = as_stream(stream);
        switch (T) {
            case 1: launch_router_decode<1>(x, x_dtype, (int)H, w, w_dtype, bias, bias_dtype, (int)E, out, out_dtype, st); break;
            case 2: launch_router_decode<2>(x, x_dtype, (int)H, w, w_dtype, bias, bias_dtype, (int)E, out, out_dtype, st); break;
            case 3: launch_router_decode<3>(x, x_dtype, (int)H, w, w_dtype, bias, bias_dtype, (int)E, out, out_dtype, st); break;
            default: launch_router_decode<4>(x, x_dtype, (int)H, w, w_dtype, bias, bias_dtype, (int)E, out, out_dtype, st); break;
        }
        TSA_LAUNCH_CHECK();
        return TSA_OK;
    }
    hipLaunchKernelGGL(router_logits_kernel, dim3((unsigned)((E + 3) / 4), (unsigned)((T + RT - 1) / RT)), dim3(256), 0,
                       as_stream(stream), x, x_dtype, T, (int)H, w, w_dtype, bias, bias_dtype, (int)E, out, out_dtype);
    TSA_LAUNCH_CHECK();
    return TSA_OK;
}

extern "C" int tsa_route_topk(const void* logits, int logits_dtype, int64_t T, int64_t E, int k, int mode,
                              int32_t* idx, float* weights, void* stream) {
    clear_error();
    TSA_REQUIRE(valid_dtype(logits_dtype), TSA_ERR_INVALID_ARG, "bad logits dtype %d", logits_dtype);
    TSA_REQUIRE(mode >= 0 && mode <= 2, TSA_ERR_INVALID_ARG, "bad routing mode %d", mode);
    TSA_REQUIRE(E >= 1 && E <= 64 * MAX_PER_LANE, TSA_ERR_SHAPE, "num_experts (%lld) must be in [1, %d]",
                (long long)E, 64 * MAX_PER_LANE);
    TSA_REQUIRE(k >= 1 && k <= 64 && k <= E, TSA_ERR_SHAPE, "top_k (%d) must be in [1, min(64, num_experts)]", k);
    TSA_REQUIRE(T >= 0, TSA_ERR_INVALID_ARG, "negative token count");
    if (T == 0) return TSA_OK;
    TSA_REQUIRE(logits && idx && weights, TSA_ERR_INVALID_ARG, "null pointer");
    if (E <= 256)
        hipLaunchKernelGGL(route_topk_dpp_kernel, dim3((unsigned)((T + 3) / 4)), dim3(256), 0, as_stream(stream), logits,
                           logits_dtype, T, (int)E, k, mode, idx, weights);
    else
        hipLaunchKernelGGL(route_topk_kernel, dim3((unsigned)((T + 3) / 4)), dim3(256), 0, as_stream(stream), logits,
                           logits_dtype, T, (int)E, k, mode, idx, weights);
    TSA_LAUNCH_CHECK();
    return TSA_OK;
}
