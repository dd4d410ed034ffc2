// Device helpers shared by the MoE decode kernels: DPP wave reductions, in-kernel top-k
// routing and the GPT-OSS activation.
#pragma once

#include "tsa_common.h"
#include "formats.h"

namespace tsa {
namespace {

constexpr int FUSED_MAXT = 4;   // tokens per fused launch
constexpr int FUSED_MAXK = 16;  // experts per token

// ---------------------------------------------------------------- DPP wave reductions
template <int CTRL, int ROW_MASK, int BANK_MASK>
__device__ __forceinline__ float dpp_f(float v, float old) {
    return __int_as_float(
        __builtin_amdgcn_update_dpp(__float_as_int(old), __float_as_int(v), CTRL, ROW_MASK, BANK_MASK, false));
}

// Sums each of R rows (R = 4 or 8; one partial per row per lane) over the 64 lanes: on
// return every lane holds its group's total, row (lane >> log2(64 / R)), so lane (64 / R) r
// holds row r. Halving steps first: v_permlane32_swap / v_permlane16_swap hand each half of
// the wave the other half's partials of the rows it keeps (rows 0 .. n/2-1 stay in the lower
// lanes), then (R = 8) lanes 8 apart via row_ror:8, which is xor 8 inside a 16-lane row; DPP
// sums the remaining lane group. All VALU, no LDS round trip: about R + 6 cross-lane steps
// instead of R full wave reductions.
__device__ __forceinline__ void permlane_halves(float& lo, float& hi, int off) {
    // lo: the rows the lower lanes keep, hi: the rows the upper lanes keep; on return
    // lo = lo + partner's lo in the lower lanes and hi + partner's hi in the upper ones
    const auto r = off == 32 ? __builtin_amdgcn_permlane32_swap(__float_as_uint(lo), __float_as_uint(hi), false, false)
                             : __builtin_amdgcn_permlane16_swap(__float_as_uint(lo), __float_as_uint(hi), false, false);
    lo = __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

template <int R>
__device__ __forceinline__ float wave_sum_rows(const float (&a)[R], int lane) {
    static_assert(R == 4 || R == 8, "4 or 8 rows");
    float v[R];
#pragma unroll
    for (int i = 0; i < R; ++i) v[i] = a[i];
#pragma unroll
    for (int i = 0; i < R / 2; ++i) permlane_halves(v[i], v[R / 2 + i], 32);
#pragma unroll
    for (int i = 0; i < R / 4; ++i) permlane_halves(v[i], v[R / 4 + i], 16);
    float t = v[0];
    if (R == 8) {
        const bool hi = (lane & 8) != 0;
        const float keep = hi ? v[1] : v[0], send = hi ? v[0] : v[1];
        t = keep + dpp_f<0x128, 0xF, 0xF>(send, 0.0f);  // row_ror:8
    }
    t += dpp_f<0xB1, 0xF, 0xF>(t, 0.0f);   // quad_perm [1,0,3,2]
    t += dpp_f<0x4E, 0xF, 0xF>(t, 0.0f);   // quad_perm [2,3,0,1]: every lane holds its quad's sum
    t += dpp_f<0x141, 0xF, 0xF>(t, 0.0f);  // row_half_mirror (lane i reads 7 - i): octet sums
    if (R == 4) t += dpp_f<0x140, 0xF, 0xF>(t, 0.0f);  // row_mirror (lane i reads 15 - i): 16-lane sums
    return t;
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

// Inclusive sum of v over the workgroup's threads in thread order (up to 16 waves): a
// shuffle scan per wave, then each wave adds the totals of the waves before it (wsum: 16
// ints of LDS). total = the sum over all threads. Every thread must call it; two barriers,
// the second so that wsum may be reused.
__device__ __forceinline__ int block_incl_sum(int v, int* wsum, int& total) {
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6, nw = blockDim.x >> 6;
    for (int d = 1; d < 64; d <<= 1) {
        const int t = __shfl_up(v, d, 64);
        if (lane >= d) v += t;
    }
    if (lane == 63) wsum[w] = v;
    __syncthreads();
    int off = 0, tot = 0;
    for (int i = 0; i < nw; ++i) {
        const int s = wsum[i];
        off += i < w ? s : 0;
        tot += s;
    }
    total = tot;
    __syncthreads();
    return v + off;
}

// Slot tables live in LDS, so the compiler treats values read from them as per-lane;
// a buffer resource built from such a value is wrapped in a waterfall loop per load.
// Every lane reads the same entry, so lane 0's value is the wave's.
__device__ __forceinline__ int uniform(int v) { return __builtin_amdgcn_readfirstlane(v); }

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

// Orderable key of a logit: a larger float has a larger key, -0 and +0 share one key, NaN
// gets the largest key (torch.topk, which the reference's routing calls, ranks NaN above
// every number), and every logit's key is above the key 0 of padding and of entries
// already selected.
__device__ __forceinline__ uint32_t route_key(float v) {
    uint32_t u = __float_as_uint(v);
    u = u == 0x80000000u ? 0u : u;
    const uint32_t key = (u & 0x80000000u) ? ~u : (u | 0x80000000u);
    return v != v ? 0xFFFFFFFFu : key;
}
__device__ __forceinline__ float route_key_value(uint32_t key) {
    return __uint_as_float((key & 0x80000000u) ? (key & 0x7FFFFFFFu) : ~key);
}

// Sum over lanes 0..15 (the first DPP row), returned to every lane.
__device__ __forceinline__ float row16_sum(float v) {
    const float o = v;
    v += dpp_f<0x111, 0xF, 0xF>(o, 0.0f);
    v += dpp_f<0x112, 0xF, 0xF>(o, 0.0f);
    v += dpp_f<0x113, 0xF, 0xF>(o, 0.0f);
    v += dpp_f<0x114, 0xF, 0xE>(v, 0.0f);
    v += dpp_f<0x118, 0xF, 0xC>(v, 0.0f);
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 15));
}

__device__ __forceinline__ uint32_t wave_max_u32(uint32_t v) {
    v = max(v, (uint32_t)dpp_i<0x111, 0xF, 0xF>((int)v, 0));
    v = max(v, (uint32_t)dpp_i<0x112, 0xF, 0xF>((int)v, 0));
    v = max(v, (uint32_t)dpp_i<0x113, 0xF, 0xF>((int)v, 0));
    v = max(v, (uint32_t)dpp_i<0x114, 0xF, 0xE>((int)v, 0));
    v = max(v, (uint32_t)dpp_i<0x118, 0xF, 0xC>((int)v, 0));
    v = max(v, (uint32_t)dpp_i<0x142, 0xA, 0xF>((int)v, 0));
    v = max(v, (uint32_t)dpp_i<0x143, 0xC, 0xF>((int)v, 0));
    return (uint32_t)__builtin_amdgcn_readlane((int)v, 63);
}

// Top-k selection over NV logits per lane (expert e = lane + 64 j), k <= 16, in rounds:
// each takes the largest remaining key with a DPP wave max, its lowest expert id among
// equal keys with ballots, and removes it (key 0, below the key of every logit). The
// selections come out in rank order: NaN first, then descending logit, ties to the lower id.
// Lane r < nr ends with the key, id and slot (es) of the r-th selection; nr <= k rounds run
// (a caller that needs only the r-th selection stops after round r).
template <int NV, class P>
__device__ void route_select(const P& p, int lane, const float v[4], const int es[4], int nr, uint32_t& myk,
                             int& mysel, int& myslot) {
    uint32_t key[NV];
#pragma unroll
    for (int j = 0; j < NV; ++j) key[j] = lane + 64 * j < p.E ? route_key(v[j]) : 0u;
    myk = 0u;
    mysel = -1;
    myslot = -1;
    for (int r = 0; r < nr; ++r) {
        uint32_t m = key[0];
#pragma unroll
        for (int j = 1; j < NV; ++j) m = max(m, key[j]);
        const uint32_t top = wave_max_u32(m);
        int id = -1, slot = -1;
#pragma unroll
        for (int j = 0; j < NV; ++j) {
            const uint64_t hit = __ballot(key[j] == top);
            if (hit && id < 0) {
                const int l = __ffsll((unsigned long long)hit) - 1;
                id = 64 * j + l;
                slot = __builtin_amdgcn_readlane(es[j], l);
            }
        }
#pragma unroll
        for (int j = 0; j < NV; ++j) key[j] = lane + 64 * j == id ? 0u : key[j];
        if (lane == r) {
            myk = top;
            mysel = id;
            myslot = slot;
        }
    }
}

// One wave routes token t (E <= 256, k <= 16): slots of the selected experts into s_slot
// (es[j] = expert_slot[lane + 64 j], loaded by the caller), weights into s_w; lane r < k
// returns the r-th selected expert id. Selection is by logit, descending, ties to the lower
// id; the softmax is monotone, so this is also the top-k of the probabilities
// (tinyserve/_model_hooks.py:456-473). Softmax over all experts, top-k and renormalisation
// equals the softmax over the k selected logits, so that mode shares the top-k-softmax
// path; only the unnormalised mode needs the sum over all experts. v[j] = logit lane + 64 j
// of the token, loaded by the caller (as load4 gives them).
template <class P>
__device__ int route_token_v(const P& p, int t, int lane, const float v[4], const int es[4], int* s_slot, float* s_w) {
    uint32_t myk;
    int mysel, myslot;
    switch ((p.E + 63) >> 6) {
        case 1: route_select<1>(p, lane, v, es, p.k, myk, mysel, myslot); break;
        case 2: route_select<2>(p, lane, v, es, p.k, myk, mysel, myslot); break;
        case 3: route_select<3>(p, lane, v, es, p.k, myk, mysel, myslot); break;
        default: route_select<4>(p, lane, v, es, p.k, myk, mysel, myslot); break;
    }
    if (lane < p.k) s_slot[t * p.k + lane] = myslot;
    const float myval = route_key_value(myk);  // lane r < k: the r-th selected logit
    const float top = route_key_value((uint32_t)__builtin_amdgcn_readfirstlane((int)myk));  // the maximum
    float w;
    if (p.route_mode == TSA_ROUTE_SOFTMAX_TOPK) {
        float s = 0.0f;
#pragma unroll
        for (int j = 0; j < 4; ++j)
            if (lane + 64 * j < p.E) s += __expf(v[j] - top);
        const float z = wave_sum_u(s);
        w = lane < p.k ? __expf(myval - top) / z : 0.0f;
    } else {
        const float ex = lane < p.k ? __expf(myval - top) : 0.0f;
        w = ex / row16_sum(ex);
    }
    if (lane < p.k) s_w[t * p.k + lane] = w;
    return mysel;
}

// The token's first nr selections within one wave (route_select: rounds of a DPP wave max):
// lane r < nr ends with the key, expert id and slot of the r-th selection (NaN first, then
// descending logit, ties to the lower id). lg / es: the token's logits and slot table as
// load4 lays them out.
template <class P>
__device__ __forceinline__ void select_topk(const P& p, int lane, const float lg[4], const int es[4], int nr,
                                            uint32_t& myk, int& mysel, int& myslot) {
    switch ((p.E + 63) >> 6) {
        case 1: route_select<1>(p, lane, lg, es, nr, myk, mysel, myslot); break;
        case 2: route_select<2>(p, lane, lg, es, nr, myk, mysel, myslot); break;
        case 3: route_select<3>(p, lane, lg, es, nr, myk, mysel, myslot); break;
        default: route_select<4>(p, lane, lg, es, nr, myk, mysel, myslot); break;
    }
}

// route_token_v with the token's logits loaded here.
template <class P>
__device__ int route_token(const P& p, int t, int lane, const int es[4], int* s_slot, float* s_w) {
    float v[4];
    load4(p.logits, p.logits_dtype, (int64_t)t * p.E, p.E, lane, v);
    return route_token_v(p, t, lane, v, es, s_slot, s_w);
}

__device__ __forceinline__ float swiglu_oai(const tsa_expert_layout& L, float gate, float up) {
    const float g = fminf(gate, L.swiglu_limit);
    const float u = fminf(fmaxf(up, -L.swiglu_limit), L.swiglu_limit);
    return (u + 1.0f) * g * sigmoidf_(L.swiglu_alpha * g);
}

// The same for epilogues that evaluate many values per lane: the sigmoid from v_exp_f32 and
// v_rcp_f32 (each within about 1 ulp) instead of the range-reduced expf and the IEEE
// divide, about a third of the VALU instructions. The relative error is of order 1e-6,
// far below the bf16 rounding of the result.
__device__ __forceinline__ float swiglu_oai_fast(const tsa_expert_layout& L, float gate, float up) {
    const float g = fminf(gate, L.swiglu_limit);
    const float u = fminf(fmaxf(up, -L.swiglu_limit), L.swiglu_limit);
    const float e = __builtin_amdgcn_exp2f(-1.44269504088896341f * (L.swiglu_alpha * g));
    return (u + 1.0f) * g * __builtin_amdgcn_rcpf(1.0f + e);
}

// SiLU(gate) * up with the same v_exp_f32 / v_rcp_f32 sigmoid (relative error of order 1e-6).
__device__ __forceinline__ float silu_mul_fast(float gate, float up) {
    const float e = __builtin_amdgcn_exp2f(-1.44269504088896341f * gate);
    return gate * __builtin_amdgcn_rcpf(1.0f + e) * up;
}

// Two floats to packed bf16 (lo in the low half) by v_cvt_pk_bf16_f32: round to nearest
// even, as f32_to_bf16_bits for every non-NaN input.
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
    typedef float f2_t __attribute__((ext_vector_type(2)));
    return __builtin_bit_cast(uint32_t, __builtin_convertvector((f2_t{lo, hi}), bf16x2_t));
}

}  // namespace
}  // namespace tsa
