// Device helpers shared by the fused single-launch MoE decode kernels: DPP wave
// reductions, in-kernel top-k routing, workspace counters and the GPT-OSS activation.
#pragma once

#include "tsa_common.h"
#include "formats.h"

namespace tsa {
namespace {

constexpr int FUSED_MAXT = 4;   // tokens per fused launch
constexpr int FUSED_MAXK = 16;  // experts per token
constexpr int SPIN_LIMIT = 1 << 23;  // ~2 s of s_sleep(4); never reached in a healthy run
static_assert(FUSED_MAXT * FUSED_MAXK <= WS_MAX_PAIRS, "one header counter per (token, expert) pair");

// ---------------------------------------------------------------- DPP wave reductions
template <int CTRL, int ROW_MASK, int BANK_MASK>
__device__ __forceinline__ float dpp_f(float v, float old) {
    return __int_as_float(
        __builtin_amdgcn_update_dpp(__float_as_int(old), __float_as_int(v), CTRL, ROW_MASK, BANK_MASK, false));
}
template <int CTRL, int ROW_MASK, int BANK_MASK>
__device__ __forceinline__ int dpp_i(int v, int old) {
    return __builtin_amdgcn_update_dpp(old, v, CTRL, ROW_MASK, BANK_MASK, false);
}

// Lane l accumulates v[l-1], v[l-2], v[l-3] of the ORIGINAL values (row_shr 1,2,3), then
// the partials of lanes l-4 (banks 1-3) and l-8 (banks 2-3), so lane 15 of each 16-lane
// row holds the row sum; row_bcast 15 / 31 fold the rows into lane 63, which is read back
// as a wave-uniform value. (Max/min use the same pattern; idempotence lets them fold the
// running value at every step.)
__device__ __forceinline__ float wave_sum_u(float v) {
    const float o = v;
    v += dpp_f<0x111, 0xF, 0xF>(o, 0.0f);
    v += dpp_f<0x112, 0xF, 0xF>(o, 0.0f);
    v += dpp_f<0x113, 0xF, 0xF>(o, 0.0f);
    v += dpp_f<0x114, 0xF, 0xE>(v, 0.0f);
    v += dpp_f<0x118, 0xF, 0xC>(v, 0.0f);
    v += dpp_f<0x142, 0xA, 0xF>(v, 0.0f);
    v += dpp_f<0x143, 0xC, 0xF>(v, 0.0f);
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 63));
}

__device__ __forceinline__ float wave_max_u(float v) {
    const float ni = -INFINITY;
    v = fmaxf(v, dpp_f<0x111, 0xF, 0xF>(v, ni));
    v = fmaxf(v, dpp_f<0x112, 0xF, 0xF>(v, ni));
    v = fmaxf(v, dpp_f<0x113, 0xF, 0xF>(v, ni));
    v = fmaxf(v, dpp_f<0x114, 0xF, 0xE>(v, ni));
    v = fmaxf(v, dpp_f<0x118, 0xF, 0xC>(v, ni));
    v = fmaxf(v, dpp_f<0x142, 0xA, 0xF>(v, ni));
    v = fmaxf(v, dpp_f<0x143, 0xC, 0xF>(v, ni));
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 63));
}

__device__ __forceinline__ int wave_min_u(int v) {
    const int big = 0x7FFFFFFF;
    v = min(v, dpp_i<0x111, 0xF, 0xF>(v, big));
    v = min(v, dpp_i<0x112, 0xF, 0xF>(v, big));
    v = min(v, dpp_i<0x113, 0xF, 0xF>(v, big));
    v = min(v, dpp_i<0x114, 0xF, 0xE>(v, big));
    v = min(v, dpp_i<0x118, 0xF, 0xC>(v, big));
    v = min(v, dpp_i<0x142, 0xA, 0xF>(v, big));
    v = min(v, dpp_i<0x143, 0xC, 0xF>(v, big));
    return __builtin_amdgcn_readlane(v, 63);
}

// Slot tables live in LDS, so the compiler treats values read from them as per-lane;
// a buffer resource built from such a value is wrapped in a waterfall loop per load.
// Every lane reads the same entry, so lane 0's value is the wave's.
__device__ __forceinline__ int uniform(int v) { return __builtin_amdgcn_readfirstlane(v); }

__device__ __forceinline__ unsigned ld_relaxed(unsigned* p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Completion counter of pair i = t*k + j (header layout in tsa_common.h).
__device__ __forceinline__ unsigned* pair_ctr(unsigned* bar, int i) {
    return bar + (WS_CTR_OFF + i * WS_CTR_STRIDE) / 4;
}

// v[j] = element base + min(lane + 64 j, n - 1) of a float/bf16/fp16 array: four
// unconditional loads issued together (a per-element dtype branch would serialise them).
__device__ __forceinline__ void load4(const void* src, int dtype, int64_t base, int n, int lane, float v[4]) {
    int idx[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) idx[j] = min(lane + 64 * j, n - 1);
    if (dtype == TSA_F32) {
        const float* f = static_cast<const float*>(src) + base;
        const float a = f[idx[0]], b = f[idx[1]], c = f[idx[2]], d = f[idx[3]];
        v[0] = a; v[1] = b; v[2] = c; v[3] = d;
    } else {
        const uint16_t* h = static_cast<const uint16_t*>(src) + base;
        const uint32_t a = h[idx[0]], b = h[idx[1]], c = h[idx[2]], d = h[idx[3]];
        const bool bf = dtype == TSA_BF16;
        v[0] = bf ? bf16_bits_to_f32(a) : f16_bits_to_f32(a);
        v[1] = bf ? bf16_bits_to_f32(b) : f16_bits_to_f32(b);
        v[2] = bf ? bf16_bits_to_f32(c) : f16_bits_to_f32(c);
        v[3] = bf ? bf16_bits_to_f32(d) : f16_bits_to_f32(d);
    }
}

// A bias element, without a dtype branch around the load (the bits are converted after).
__device__ __forceinline__ float load_bias(const uint8_t* src, int dtype, int64_t i) {
    if (dtype == TSA_F32) return reinterpret_cast<const float*>(src)[i];
    const uint32_t b = reinterpret_cast<const uint16_t*>(src)[i];
    return dtype == TSA_BF16 ? bf16_bits_to_f32(b) : f16_bits_to_f32(b);
}

// One wave routes token t (E <= 256): slots of the selected experts into s_slot (es[j] =
// expert_slot[lane + 64 j], loaded by the caller), weights into s_w; lane r < k returns
// the r-th selected expert id.
template <class P>
__device__ int route_token(const P& p, int t, int lane, const int es[4], int* s_slot, float* s_w) {
    float v[4];
    load4(p.logits, p.logits_dtype, (int64_t)t * p.E, p.E, lane, v);
#pragma unroll
    for (int j = 0; j < 4; ++j)
        if (lane + 64 * j >= p.E) v[j] = -INFINITY;
    unsigned taken = 0;
    float myval = -INFINITY;  // lane r < k: the r-th selected logit
    int mysel = -1;           // lane r < k: the r-th selected id
    for (int r = 0; r < p.k; ++r) {
        float bv = -INFINITY;
        int bi = 0x7FFFFFFF;
#pragma unroll
        for (int j = 0; j < 4; ++j) {  // j ascending keeps the lowest id on ties within a lane
            const int e = lane + 64 * j;
            if (e < p.E && !((taken >> j) & 1u) && (v[j] > bv || bi == 0x7FFFFFFF)) { bv = v[j]; bi = e; }
        }
        const float m = wave_max_u(bv);
        const int e = wave_min_u(bv == m ? bi : 0x7FFFFFFF);
        const int je = e >> 6;
        if ((e & 63) == lane) {
            taken |= 1u << je;
            s_slot[t * p.k + r] = je == 0 ? es[0] : je == 1 ? es[1] : je == 2 ? es[2] : es[3];
        }
        if (lane == r) { myval = m; mysel = e; }
    }
    float w;
    if (p.route_mode == TSA_ROUTE_TOPK_SOFTMAX) {
        const float top = __int_as_float(__builtin_amdgcn_readfirstlane(__float_as_int(myval)));  // lane 0 = max
        const float ex = lane < p.k ? expf(myval - top) : 0.0f;
        w = ex / wave_sum_u(ex);
    } else {
        const float vmax = wave_max_u(fmaxf(fmaxf(v[0], v[1]), fmaxf(v[2], v[3])));
        float s = 0.0f;
#pragma unroll
        for (int j = 0; j < 4; ++j)
            if (lane + 64 * j < p.E) s += expf(v[j] - vmax);
        const float zsum = wave_sum_u(s);
        const float pr = lane < p.k ? expf(myval - vmax) / zsum : 0.0f;
        w = p.route_mode == TSA_ROUTE_SOFTMAX_TOPK_RENORM ? pr / wave_sum_u(pr) : pr;
    }
    if (lane < p.k) s_w[t * p.k + lane] = w;
    return mysel;
}

__device__ __forceinline__ float swiglu_oai(const tsa_expert_layout& L, float gate, float up) {
    const float g = fminf(gate, L.swiglu_limit);
    const float u = fminf(fmaxf(up, -L.swiglu_limit), L.swiglu_limit);
    return (u + 1.0f) * g * sigmoidf_(L.swiglu_alpha * g);
}

}  // namespace
}  // namespace tsa
