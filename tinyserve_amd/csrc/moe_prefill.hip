// Prefill side of the MoE path: expert-major grouping of (token, j) assignments and the
// batched expert FFN over many tokens.
#include "tsa_common.h"

namespace tsa {
int validate_layout(const tsa_expert_layout* L);

namespace {

constexpr int GROUP_THREADS = 1024;
constexpr int GROUP_WAVES = GROUP_THREADS / 64;
constexpr int MAX_GROUP_E = 1024;

// Single-workgroup stable counting sort of assignment ids by expert.
// Pass 1 counts; pass 2 walks the assignments in rounds of 1024 (in order), ranks
// each one among equal experts of lower index inside its wave (ballot), then across
// the waves of the round (per-wave distinct-expert counts in LDS), then across rounds
// (running offsets), so the result is token-major within every expert.
__global__ void __launch_bounds__(GROUP_THREADS) group_kernel(const int32_t* __restrict__ idx, int64_t n, int E,
                                                              int32_t* __restrict__ counts,
                                                              int32_t* __restrict__ offsets,
                                                              int32_t* __restrict__ perm) {
    __shared__ int cnt[MAX_GROUP_E];
    __shared__ int run[MAX_GROUP_E];
    __shared__ int wave_cnt[GROUP_WAVES][64];
    __shared__ int wave_eid[GROUP_WAVES][64];
    __shared__ int wave_nuniq[GROUP_WAVES];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    for (int e = tid; e < E; e += GROUP_THREADS) cnt[e] = 0;
    __syncthreads();
    for (int64_t a = tid; a < n; a += GROUP_THREADS) {
        const int e = idx[a];
        if (e >= 0 && e < E) atomicAdd(&cnt[e], 1);
    }
    __syncthreads();
    if (tid == 0) {  // exclusive scan; E <= 1024 so a serial scan is negligible
        int acc = 0;
        for (int e = 0; e < E; ++e) {
            offsets[e] = acc;
            counts[e] = cnt[e];
            run[e] = acc;
            acc += cnt[e];
        }
        offsets[E] = acc;
    }
    __syncthreads();
    for (int64_t base = 0; base < n; base += GROUP_THREADS) {
        const int64_t a = base + tid;
        int e = a < n ? idx[a] : -1;
        if (e >= E) e = -1;
        unsigned long long remaining = __ballot(e >= 0);
        int my_rank = 0, nuniq = 0;
        while (remaining) {
            const int leader = __ffsll((unsigned long long)remaining) - 1;
            const int le = __shfl(e, leader, 64);
            const unsigned long long m = __ballot(e == le) & remaining;
            if (e == le) my_rank = __popcll(m & ((1ull << lane) - 1ull));
            if (lane == 0) {
                wave_eid[wave][nuniq] = le;
                wave_cnt[wave][nuniq] = __popcll(m);
            }
            remaining &= ~m;
            ++nuniq;
        }
        if (lane == 0) wave_nuniq[wave] = nuniq;
        __syncthreads();
        if (e >= 0) {
            int before = 0;  // same expert in earlier waves of this round
            for (int w = 0; w < wave; ++w)
                for (int u = 0; u < wave_nuniq[w]; ++u)
                    if (wave_eid[w][u] == e) before += wave_cnt[w][u];
            perm[run[e] + before + my_rank] = (int32_t)a;
        }
        __syncthreads();
        if (lane == 0)
            for (int u = 0; u < nuniq; ++u) atomicAdd(&run[wave_eid[wave][u]], wave_cnt[wave][u]);
        __syncthreads();
    }
}

__global__ void __launch_bounds__(256) map_slots_kernel(const int32_t* __restrict__ idx, int64_t n,
                                                        const int32_t* __restrict__ expert_slot, int64_t E,
                                                        int32_t* __restrict__ slots) {
    const int64_t a = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (a >= n) return;
    const int e = idx[a];
    slots[a] = (e >= 0 && e < E) ? expert_slot[e] : -1;
}

}  // namespace
}  // namespace tsa

using namespace tsa;

extern "C" int tsa_group_by_expert(const int32_t* idx, int64_t T, int k, int64_t E, int32_t* counts, int32_t* offsets,
                                   int32_t* perm, void* stream) {
    clear_error();
    TSA_REQUIRE(T >= 0 && k >= 1 && E >= 1 && E <= MAX_GROUP_E, TSA_ERR_SHAPE,
                "bad grouping shape (T %lld, k %d, E %lld; E must be <= %d)", (long long)T, k, (long long)E,
                MAX_GROUP_E);
    TSA_REQUIRE(T * k < (int64_t)1 << 31, TSA_ERR_SHAPE, "too many assignments");
    TSA_REQUIRE(idx && counts && offsets && (perm || T == 0), TSA_ERR_INVALID_ARG, "null pointer");
    hipLaunchKernelGGL(group_kernel, dim3(1), dim3(GROUP_THREADS), 0, as_stream(stream), idx, T * k, (int)E, counts,
                       offsets, perm);
    TSA_LAUNCH_CHECK();
    return TSA_OK;
}

static int64_t prefill_ws(const tsa_expert_layout& L, int64_t T, int k) {
    int64_t dec = 0;
    tsa_moe_decode_workspace_size(&L, T, k, &dec);
    return ((T * k * 4 + 255) / 256) * 256 + dec;
}

extern "C" int tsa_moe_prefill_workspace_size(const tsa_expert_layout* layout, int64_t T, int k, int64_t E,
                                              int64_t* bytes) {
    clear_error();
    int rc = validate_layout(layout);
    if (rc) return rc;
    TSA_REQUIRE(T >= 0 && k >= 1 && E >= 1 && bytes, TSA_ERR_INVALID_ARG, "bad T/k/E/bytes");
    *bytes = prefill_ws(*layout, T, k);
    return TSA_OK;
}

extern "C" int tsa_moe_prefill(const tsa_expert_layout* layout, const void* pool, int64_t n_slots,
                               const int32_t* expert_slot, int64_t E, const int32_t* idx, const float* weights,
                               int64_t T, int k, const void* x, int x_dtype, void* y, int y_dtype, void* workspace,
                               int64_t workspace_bytes, void* stream) {
    clear_error();
    int rc = validate_layout(layout);
    if (rc) return rc;
    TSA_REQUIRE(T >= 0 && k >= 1 && E >= 1, TSA_ERR_INVALID_ARG, "bad T/k/E");
    if (T == 0) return TSA_OK;
    TSA_REQUIRE(expert_slot && idx && weights, TSA_ERR_INVALID_ARG, "null pointer");
    const int64_t need = prefill_ws(*layout, T, k);
    TSA_REQUIRE(workspace && workspace_bytes >= need, TSA_ERR_WORKSPACE, "workspace too small: got %lld bytes, need %lld",
                (long long)workspace_bytes, (long long)need);
    int32_t* slots = static_cast<int32_t*>(workspace);
    const int64_t off = ((T * k * 4 + 255) / 256) * 256;
    hipLaunchKernelGGL(map_slots_kernel, dim3((unsigned)((T * k + 255) / 256)), dim3(256), 0, as_stream(stream), idx,
                       T * k, expert_slot, E, slots);
    TSA_LAUNCH_CHECK();
    return tsa_moe_decode(layout, pool, n_slots, slots, weights, T, k, x, x_dtype, y, y_dtype,
                          static_cast<uint8_t*>(workspace) + off, workspace_bytes - off, stream);
}
