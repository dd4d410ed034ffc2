// Prefill side of the MoE path: expert-major grouping of (token, j) assignments and the
// batched expert FFN over many tokens.
#include "fused_common.h"

namespace tsa {
int validate_layout(const tsa_expert_layout* L);
bool pf_mxt_supported(const tsa_expert_layout& L, int x_dtype, int64_t T, int k);
int64_t pf_mxt_workspace_bytes(const tsa_expert_layout& L, int64_t T, int k, int64_t E);
int pf_mxt_prefill(const tsa_expert_layout& L, const uint8_t* pool, int64_t n_slots, const int32_t* expert_slot,
                   int64_t E, const int32_t* idx, const float* weights, int64_t T, int k, const uint16_t* x, void* y,
                   int y_dtype, uint8_t* ws, hipStream_t stream);
bool gf_supported(const tsa_expert_layout& L, int x_dtype, int64_t T, int k);
int64_t gf_workspace_bytes(const tsa_expert_layout& L, int64_t T, int k, int64_t E);
int gf_prefill(const tsa_expert_layout& L, const uint8_t* pool, int64_t n_slots, const int32_t* expert_slot, int64_t E,
               const int32_t* idx, const float* weights, int64_t T, int k, const uint16_t* x, void* y, int y_dtype,
               uint8_t* ws, hipStream_t stream);

namespace {

constexpr int GROUP_THREADS = 512;
constexpr int GROUP_WAVES = GROUP_THREADS / 64;
constexpr int MAX_GROUP_E = 1024;
constexpr int GROUP_AHEAD = 8;  // id batches loaded ahead per wave

// Optional tile table written by group_kernel (the grouped GGUF GEMMs' work list): per
// resident expert in id order, entries of up to `rows` sorted rows {slot, first sorted row,
// rows, 0}; n_entries[0] = their count.
struct GroupTiles {
    const int32_t* expert_slot;
    int64_t n_slots;
    int rows;
    int* n_entries;
    int4* table;
};

// LDS of group_kernel for E experts: per (wave, expert) counters, the experts' offsets, and
// per (wave, expert) 64-bit lane masks (8-byte aligned).
__host__ __device__ constexpr int group_lds_bytes(int E) { return ((GROUP_WAVES + 1) * E * 4 + 7) / 8 * 8 + GROUP_WAVES * E * 8; }

// Single-workgroup stable counting sort of assignment ids by expert. Wave w owns one
// contiguous chunk of the assignments (a multiple of 64 long) and walks it in batches of
// 64. Pass 1 counts per (wave, expert) with LDS atomic adds (a wave owns its row of
// counters; the order of the adds does not matter). An exclusive scan over the waves, per
// expert, then gives each wave its first rank inside the expert, and a scan over the
// experts the offsets. Pass 2 walks the same batches in the same order and places each
// assignment at offset + the wave's running rank + its rank among the batch's lanes of the
// same expert: every lane ORs its bit into its wave's mask of the expert and reads the mask
// back (LDS runs one wave's instructions in order), the lowest lane of each group then
// clears the mask and advances the running rank. Every expert's run keeps assignment order
// (token-major), as the reference's grouping does. With tiles.table set it also writes the
// tile table between the passes (each thread two experts; the slots are loaded first).
__global__ void __launch_bounds__(GROUP_THREADS) group_kernel(const int32_t* __restrict__ idx, int64_t n, int E,
                                                              int32_t* __restrict__ counts,
                                                              int32_t* __restrict__ offsets,
                                                              int32_t* __restrict__ perm, GroupTiles tiles) {
    extern __shared__ __align__(16) unsigned char gsm[];
    int* wcnt = reinterpret_cast<int*>(gsm);  // [wave][expert]
    int* eoff = wcnt + GROUP_WAVES * E;
    unsigned long long* wmask = reinterpret_cast<unsigned long long*>(gsm + ((GROUP_WAVES + 1) * E * 4 + 7) / 8 * 8);
    __shared__ int wsum[16];
    __shared__ int n_all;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const unsigned long long below = (1ull << lane) - 1ull;
    static_assert(2 * GROUP_THREADS >= MAX_GROUP_E, "two experts per thread for the tile table");
    int es[2] = {-1, -1};  // the tile table's experts 2 tid, 2 tid + 1: their slots, loaded early
    if (tiles.table) {
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            const int e = 2 * tid + i;
            if (e < E) {
                es[i] = tiles.expert_slot[e];
                if (es[i] >= tiles.n_slots) es[i] = -1;
            }
        }
    }
    for (int i = tid; i < GROUP_WAVES * E; i += GROUP_THREADS) {
        wcnt[i] = 0;
        wmask[i] = 0ull;
    }
    __syncthreads();
    int* cnt = wcnt + wave * E;
    unsigned long long* msk = wmask + wave * E;
    const int64_t chunk = ((n + GROUP_WAVES - 1) / GROUP_WAVES + 63) / 64 * 64;
    const int64_t a0 = wave * chunk, a1 = a0 + chunk < n ? a0 + chunk : n;
    // Batches of 64 assignments in order; the ids of GROUP_AHEAD batches are loaded together
    // so the wave waits for one memory round trip per GROUP_AHEAD batches, not per batch.
    for (int64_t b0 = a0; b0 < a1; b0 += 64 * GROUP_AHEAD) {
        int ev[GROUP_AHEAD];
#pragma unroll
        for (int j = 0; j < GROUP_AHEAD; ++j) {
            const int64_t a = b0 + 64 * j + lane;
            ev[j] = a < a1 ? idx[a] : -1;
        }
#pragma unroll
        for (int j = 0; j < GROUP_AHEAD; ++j)
            if (ev[j] >= 0 && ev[j] < E) atomicAdd(&cnt[ev[j]], 1);
    }
    __syncthreads();
    for (int e = tid; e < E; e += GROUP_THREADS) {
        int run = 0;
        for (int w = 0; w < GROUP_WAVES; ++w) {
            const int c = wcnt[w * E + e];
            wcnt[w * E + e] = run;
            run += c;
        }
        eoff[e] = run;
    }
    __syncthreads();
    if (wave == 0) {  // offsets: exclusive scan of the totals, 16 experts per lane at most
        const int per = (E + 63) / 64;
        int loc = 0;
        for (int j = 0; j < per; ++j)
            if (lane * per + j < E) loc += eoff[lane * per + j];
        int inc = loc;
        for (int d = 1; d < 64; d <<= 1) {
            const int v = __shfl_up(inc, d, 64);
            if (lane >= d) inc += v;
        }
        int run = inc - loc;
        for (int j = 0; j < per; ++j) {
            const int e = lane * per + j;
            if (e < E) {
                const int c = eoff[e];
                counts[e] = c;
                offsets[e] = run;
                eoff[e] = run;
                run += c;
            }
        }
        if (lane == 63) {
            offsets[E] = inc;
            n_all = inc;
        }
    }
    __syncthreads();
    if (tiles.table) {  // eoff holds the offsets; a count is the next offset minus its own
        int c[2], nt[2];
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            const int e = 2 * tid + i;
            c[i] = e < E && es[i] >= 0 ? (e + 1 < E ? eoff[e + 1] : n_all) - eoff[e] : 0;
            nt[i] = (c[i] + tiles.rows - 1) / tiles.rows;
        }
        int total;
        int first = block_incl_sum(nt[0] + nt[1], wsum, total) - nt[0] - nt[1];
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            const int e = 2 * tid + i;
            for (int j = 0; j < nt[i]; ++j) {
                const int r = c[i] - tiles.rows * j;
                tiles.table[first++] = make_int4(es[i], eoff[e] + tiles.rows * j, r < tiles.rows ? r : tiles.rows, 0);
            }
        }
        if (tid == 0) tiles.n_entries[0] = total;
    }
    for (int64_t b0 = a0; b0 < a1; b0 += 64 * GROUP_AHEAD) {
        int ev[GROUP_AHEAD];
#pragma unroll
        for (int j = 0; j < GROUP_AHEAD; ++j) {
            const int64_t a = b0 + 64 * j + lane;
            ev[j] = a < a1 ? idx[a] : -1;
        }
#pragma unroll
        for (int j = 0; j < GROUP_AHEAD; ++j) {
            const int e = ev[j];
            if (e >= 0 && e < E) {
                atomicOr(&msk[e], 1ull << lane);
                const unsigned long long m = msk[e];  // after every lane's OR: this batch's lanes of e
                const int at = eoff[e] + cnt[e] + __popcll(m & below);
                perm[at] = (int32_t)(b0 + 64 * j + lane);
                if (!(m & below)) {  // after every lane of the group read the mask and the count
                    msk[e] = 0ull;
                    cnt[e] += __popcll(m);
                }
            }
        }
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

// tile_rows > 0: also the tile table of the resident experts (table: int4 entries).
int launch_group_kernel(const int32_t* idx, int64_t n, int E, int32_t* counts, int32_t* offsets, int32_t* perm,
                        hipStream_t stream, const int32_t* expert_slot, int64_t n_slots, int tile_rows,
                        int* n_entries, void* table) {
    const int lds = group_lds_bytes(E);
    const hipError_t e = ensure_dynamic_lds(reinterpret_cast<const void*>(&group_kernel), lds);
    TSA_REQUIRE(e == hipSuccess, TSA_ERR_HIP, "hipFuncSetAttribute(LDS %d): %s", lds, hipGetErrorString(e));
    const GroupTiles tiles{expert_slot, n_slots, tile_rows, n_entries, tile_rows > 0 ? static_cast<int4*>(table) : nullptr};
    hipLaunchKernelGGL(group_kernel, dim3(1), dim3(GROUP_THREADS), lds, stream, idx, n, E, counts, offsets, perm,
                       tiles);
    TSA_LAUNCH_CHECK();
    return TSA_OK;
}

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
    return launch_group_kernel(idx, T * k, (int)E, counts, offsets, perm, as_stream(stream), nullptr, 0, 0, nullptr,
                               nullptr);
}

// Workspace of the token-chunked decode path: the assignments' slots, then a decode workspace.
static int64_t chunked_ws(const tsa_expert_layout& L, int64_t T, int k) {
    int64_t dec = 0;
    tsa_moe_decode_workspace_size(&L, T, k, &dec);
    return ((T * k * 4 + 255) / 256) * 256 + dec;
}

// MXFP4 tiled pools with bf16 activations take the grouped MFMA GEMMs, and so do GGUF pools
// (gf_supported: bf16 activations, dimensions multiples of 32, enough assignments); every
// other call runs the decode kernels over chunks of tokens. The workspace covers the
// largest form the layout can take (the x dtype is not known here).
static int64_t prefill_ws(const tsa_expert_layout& L, int64_t T, int k, int64_t E) {
    const int64_t c = chunked_ws(L, T, k);
    int64_t g = 0;
    if (L.format == TSA_EXPERT_MXFP4 && L.mx_tiled) g = pf_mxt_workspace_bytes(L, T, k, E);
    if (gf_supported(L, TSA_BF16, T, k)) g = gf_workspace_bytes(L, T, k, E);
    return g > c ? g : c;
}

extern "C" int tsa_moe_prefill_workspace_size(const tsa_expert_layout* layout, int64_t T, int k, int64_t E,
                                              int64_t* bytes) {
    clear_error();
    int rc = validate_layout(layout);
    if (rc) return rc;
    TSA_REQUIRE(T >= 0 && k >= 1 && E >= 1 && bytes, TSA_ERR_INVALID_ARG, "bad T/k/E/bytes");
    *bytes = prefill_ws(*layout, T, k, E);
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
    TSA_REQUIRE(E <= 1024, TSA_ERR_SHAPE, "E %lld exceeds 1024", (long long)E);
    const int64_t need = prefill_ws(*layout, T, k, E);
    TSA_REQUIRE(workspace && workspace_bytes >= need, TSA_ERR_WORKSPACE, "workspace too small: got %lld bytes, need %lld",
                (long long)workspace_bytes, (long long)need);
    if (pf_mxt_supported(*layout, x_dtype, T, k)) {
        TSA_REQUIRE(x && y, TSA_ERR_INVALID_ARG, "null pointer");
        return pf_mxt_prefill(*layout, static_cast<const uint8_t*>(pool), n_slots, expert_slot, E, idx, weights, T, k,
                              static_cast<const uint16_t*>(x), y, y_dtype, static_cast<uint8_t*>(workspace),
                              as_stream(stream));
    }
    if (gf_supported(*layout, x_dtype, T, k) && (reinterpret_cast<uintptr_t>(pool) & 15u) == 0 &&
        (reinterpret_cast<uintptr_t>(x) & 15u) == 0) {
        TSA_REQUIRE(x && y, TSA_ERR_INVALID_ARG, "null pointer");
        return gf_prefill(*layout, static_cast<const uint8_t*>(pool), n_slots, expert_slot, E, idx, weights, T, k,
                          static_cast<const uint16_t*>(x), y, y_dtype, static_cast<uint8_t*>(workspace),
                          as_stream(stream));
    }
    int32_t* slots = static_cast<int32_t*>(workspace);
    const int64_t off = ((T * k * 4 + 255) / 256) * 256;
    hipLaunchKernelGGL(map_slots_kernel, dim3((unsigned)((T * k + 255) / 256)), dim3(256), 0, as_stream(stream), idx,
                       T * k, expert_slot, E, slots);
    TSA_LAUNCH_CHECK();
    return tsa_moe_decode(layout, pool, n_slots, slots, weights, T, k, x, x_dtype, y, y_dtype,
                          static_cast<uint8_t*>(workspace) + off, workspace_bytes - off, stream);
}
