// Router top-k: one wave64 per token; up to 16 logits per lane (E <= 1024).
//
// Selection is by logit value, descending, ties to the lower expert id; the
// softmax is monotone in the logits, so the selected set and order equal a top-k
// over the softmax probabilities (tinyserve/_model_hooks.py:456-473).
#include "tsa_common.h"

namespace tsa {
namespace {

constexpr int MAX_PER_LANE = 16;

__device__ __forceinline__ void argmax_merge(float& v, int& i, float ov, int oi) {
    if (ov > v || (ov == v && oi < i)) { v = ov; i = oi; }
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
    unsigned taken = 0;  // bit j: element lane + 64 j already selected
    float sel_v = 0.0f;  // lane j < k keeps the j-th selected logit
    int sel_i = 0;
    for (int r = 0; r < k; ++r) {
        float bv = -INFINITY;
        int bi = 0x7FFFFFFF;
#pragma unroll
        for (int j = 0; j < MAX_PER_LANE; ++j) {
            const int e = lane + 64 * j;
            if (e < E && !((taken >> j) & 1u)) argmax_merge(bv, bi, v[j], e);
        }
#pragma unroll
        for (int off = 32; off >= 1; off >>= 1) {
            const float ov = __shfl_xor(bv, off, 64);
            const int oi = __shfl_xor(bi, off, 64);
            argmax_merge(bv, bi, ov, oi);
        }
        if ((bi & 63) == lane) taken |= 1u << (bi >> 6);
        if (lane == r) { sel_v = bv; sel_i = bi; }
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

}  // namespace
}  // namespace tsa

using namespace tsa;

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
    hipLaunchKernelGGL(route_topk_kernel, dim3((unsigned)((T + 3) / 4)), dim3(256), 0, as_stream(stream), logits,
                       logits_dtype, T, (int)E, k, mode, idx, weights);
    TSA_LAUNCH_CHECK();
    return TSA_OK;
}
