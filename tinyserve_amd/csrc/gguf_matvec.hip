// One GGUF matrix times a few token vectors: y[t, n] = sum_k deq(W)[n, k] x[t, k], the
// matvec behind tsa_gguf_matvec for small token counts (tinyserve/csrc/ggml_ops.cu:461-569:
// fp32 result of the dequantised weights times the activations; the weight stream is flat,
// so rows may start inside a super-block).
//
// Workgroup = nw waves (4, 8 or 16) and one token (grid.y); wave w takes rw consecutive rows
// (rw <= 4). The host picks rw for the lanes' rounds and the SIMDs' share (gq_cost) and
// then the most waves per workgroup the LDS allows: every workgroup stages the whole
// activation row, so fewer, larger workgroups read it fewer times.
// The wave copies the byte range of its rows' super-blocks into its LDS area with
// buffer-to-LDS loads, the workgroup stages the token's activations as bf16 with the per-16
// and per-32 sums (gguf_dot.h), and each lane reduces whole units with v_dot2_f32_bf16 over
// bf16-exact codes; one wave sum per row.
#include "gguf_dot.h"

namespace tsa {
namespace {

constexpr int MV_RW = 4;         // rows per wave, at most
constexpr int MV_MAX_WAVES = 16;  // waves per workgroup, at most

struct MvParams {
    const uint8_t* w;
    uint32_t w_records;  // bytes of w the loads may touch (buffer bound)
    const void* x;
    int x_dtype;
    void* y;
    int y_dtype;
    int N, K, rw;
    int raw_off, raw_stride;  // LDS offset and per-wave stride of the super-block areas
};

template <int TY, bool WRAP, bool SPLIT>
__device__ __forceinline__ void mv_units(const uint8_t* rbuf, uint32_t shift, uint32_t s0, uint32_t u0, uint32_t nu,
                                         int n0, int K, uint32_t lo, uint32_t hi, const GqVec& xv, int lane,
                                         float (&acc)[MV_RW]) {
    using U = GqUnit<TY>;
    constexpr uint32_t VS = TY == 8 ? 32 : 256, SB = U::SB;
    for (uint32_t i = lane; i < nu; i += 64) {
        const uint32_t u = u0 + i;
        const uint32_t g0 = u * U::V, row = g0 / (uint32_t)K, kk0 = g0 - row * (uint32_t)K;
        const uint8_t* sb = rbuf + shift + (g0 / VS - s0) * SB;
        float pa = 0.0f, pb = 0.0f;
        gq_unit<TY, WRAP, SPLIT>(sb, u, kk0, K, lo, hi, xv, pa, pb);
        const int r = (int)row - n0;
        acc_add(acc, r, pa);
        if (WRAP) acc_add(acc, r + 1, pb);
    }
}

template <int TY>
__global__ void __launch_bounds__(64 * MV_MAX_WAVES) gq_matvec_kernel(MvParams p) {
    extern __shared__ __align__(16) uint8_t smem[];
    const int tid = threadIdx.x, lane = tid & 63, wave = uniform(tid >> 6);
    const int K = p.K, N = p.N, t = blockIdx.y;
    const bool split = p.x_dtype != TSA_BF16;
    const GqVec xv = gq_vec(smem, K, split);
    // the weight rows first (they do not depend on x), then x: the two latencies overlap
    const int n0 = ((int)blockIdx.x * (int)(blockDim.x >> 6) + wave) * p.rw;
    const int n1 = n0 + p.rw < N ? n0 + p.rw : N;
    using U = GqUnit<TY>;
    constexpr uint32_t VS = TY == 8 ? 32 : 256, SB = U::SB;
    const uint32_t lo = (uint32_t)n0 * K, hi = (uint32_t)(n0 < N ? n1 : n0) * K;
    const uint32_t u0 = lo / U::V, nu = (hi + U::V - 1) / U::V - u0;
    const uint32_t s0 = lo / VS, raw = gq_raw_bytes(gq_sb_count<TY>(lo, hi), SB);
    uint8_t* rbuf = smem + p.raw_off + wave * p.raw_stride;
    // copies read 16-byte-aligned memory: the buffer starts at the boundary at or below w
    const uint32_t mis = (uint32_t)reinterpret_cast<uintptr_t>(p.w) & 15u;
    const uint32_t first = mis + s0 * SB, shift = first & 15u;
    if (n0 < N)
        gq_stage_raw(p.w - mis, gq_records(p.w_records, mis), first - shift, raw, (uint32_t)reinterpret_cast<uintptr_t>(rbuf), lane);
    gq_stage(smem, p.x, p.x_dtype, (int64_t)t * K, K, tid, blockDim.x);
    gq_wait_dma();
    __syncthreads();
    if (n0 >= N) return;
    float acc[MV_RW];
#pragma unroll
    for (int r = 0; r < MV_RW; ++r) acc[r] = 0.0f;
    const bool wrap = K % U::V != 0;
    if (!wrap && !split)
        mv_units<TY, false, false>(rbuf, shift, s0, u0, nu, n0, K, lo, hi, xv, lane, acc);
    else if (!wrap)
        mv_units<TY, false, true>(rbuf, shift, s0, u0, nu, n0, K, lo, hi, xv, lane, acc);
    else if (!split)
        mv_units<TY, true, false>(rbuf, shift, s0, u0, nu, n0, K, lo, hi, xv, lane, acc);
    else
        mv_units<TY, true, true>(rbuf, shift, s0, u0, nu, n0, K, lo, hi, xv, lane, acc);
    const float tot = wave_sum_rows<MV_RW>(acc, lane);  // lane 16 r: row r
    const int r = lane >> 4;
    if ((lane & 15) == 0 && n0 + r < n1) store_out(p.y, p.y_dtype, (int64_t)t * N + n0 + r, tot);
}

const void* mv_kernel(int type) {
    switch (type) {
        case 8: return reinterpret_cast<const void*>(&gq_matvec_kernel<8>);
        case 12: return reinterpret_cast<const void*>(&gq_matvec_kernel<12>);
        case 13: return reinterpret_cast<const void*>(&gq_matvec_kernel<13>);
        case 14: return reinterpret_cast<const void*>(&gq_matvec_kernel<14>);
    }
    return nullptr;
}

struct MvShape {
    int rw = 0, nw = 4;
    size_t lds = 0;
    int raw_off = 0, raw_stride = 0;
};

// Rows per wave: the least gq_cost within the LDS budget (ties to more rows).
MvShape mv_shape(int type, int64_t T, int64_t K, int64_t N, bool split, int cus) {
    const uint32_t sb = type == 8 ? 34u : type == 12 ? 144u : type == 13 ? 176u : 210u;
    const uint32_t vs = type == 8 ? 32u : 256u, v = gq_unit_values(type);
    const size_t vec = ((size_t)gq_vec_bytes((int)K, split) + 15) / 16 * 16;
    MvShape best;
    double best_cost = 0.0;
    for (int rw = 1; rw <= MV_RW; ++rw) {
        const uint32_t raw = gq_raw_bytes((uint32_t)((rw * K + vs - 1) / vs) + 1, sb);
        if (vec + 4 * (size_t)raw > 160 * 1024) break;
        const double cost = gq_cost(gq_units(rw, K, v), (double)((N + rw - 1) / rw) * (double)T, cus);
        if (best.rw == 0 || cost <= best_cost) {
            best_cost = cost;
            best.rw = rw;
            best.raw_off = (int)vec;
            best.raw_stride = (int)raw;
        }
    }
    if (best.rw == 0) return best;
    // waves per workgroup: the most that fit in LDS while the grid still covers half the
    // CUs (every workgroup stages the activations, so fewer, larger workgroups win until
    // about half the CUs hold one: workload 1, rw 1, measured 7.5 us with 16 waves against
    // 7.9 with 8)
    const int64_t waves_needed = (N + best.rw - 1) / best.rw;
    for (int nw = MV_MAX_WAVES; nw >= 4; nw /= 2) {
        const size_t lds = vec + (size_t)nw * best.raw_stride;
        if (lds <= 160 * 1024 && (nw == 4 || 2 * (waves_needed + nw - 1) / nw * T >= cus)) {
            best.nw = nw;
            best.lds = lds;
            break;
        }
    }
    return best;
}

}  // namespace

// Requirements of the super-block matvec beyond tsa_gguf_matvec's own checks: "" if met.
const char* gq_matvec_unsupported(int type, const void* w, int64_t T, int64_t K, int64_t N, int x_dtype) {
    if (!mv_kernel(type)) return "unsupported ggml type";
    if (reinterpret_cast<uintptr_t>(w) & 1) return "weights must be 2-byte aligned";
    if (T < 1 || T > 65535) return "token count out of range";
    if (K % 32 || K > 16384) return "in_features must be a multiple of 32 and at most 16384";
    if (N * K >= ((int64_t)1 << 31)) return "matrices of 2^31 values or more are not supported";
    if (mv_shape(type, T, K, N, x_dtype != TSA_BF16, 256).rw == 0) return "activation row too large for LDS";
    return "";
}

int gq_matvec(int type, const uint8_t* w, int64_t w_bytes, const void* x, int x_dtype, int64_t T, int64_t K, void* y,
              int y_dtype, int64_t N, hipStream_t st) {
    const char* why = gq_matvec_unsupported(type, w, T, K, N, x_dtype);
    TSA_REQUIRE(!*why, TSA_ERR_SHAPE, "GGUF matvec: %s", why);
    const MvShape sh = mv_shape(type, T, K, N, x_dtype != TSA_BF16, num_cus());
    MvParams p{};
    p.w = w;
    p.w_records = (uint32_t)(w_bytes < 0xFFFFFFF0ll ? w_bytes : 0xFFFFFFF0ll);
    p.x = x;
    p.x_dtype = x_dtype;
    p.y = y;
    p.y_dtype = y_dtype;
    p.N = (int)N;
    p.K = (int)K;
    p.rw = sh.rw;
    p.raw_off = sh.raw_off;
    p.raw_stride = sh.raw_stride;
    const void* fn = mv_kernel(type);
    TSA_HIP_CHECK(ensure_dynamic_lds(fn, (int)sh.lds));
    void* args[] = {&p};
    const dim3 grid((unsigned)((N + sh.nw * sh.rw - 1) / (sh.nw * sh.rw)), (unsigned)T);
    TSA_HIP_CHECK(hipLaunchKernel(fn, grid, dim3(64 * sh.nw), args, sh.lds, st));
    return TSA_OK;
}

}  // namespace tsa
