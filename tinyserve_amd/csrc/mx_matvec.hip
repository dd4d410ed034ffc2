// MXFP4 matvec on the matrix cores, straight from the checkpoint order: y[t, n] =
// sum_k W[n, k] x[t, k] (+ bias[n]) for bf16 x, up to 8 tokens per launch column.
//
// A 16-row slice of W in the checkpoint order ([N, K/32, 16] blocks, [N, K/32] e8m0 scales)
// is, lane by lane, the fp4 B operand of v_mfma_scale_f32_16x16x128_f8f6f4: for 128-wide
// K piece m, lane 16q + i loads the 16 bytes of row n0 + i, block 4m + q (32 consecutive
// K values, the instruction's fp4 layout for column i, K block q) and that block's scale
// byte, which the instruction takes as the lane's B scale. The A operand carries x as two
// block-scaled fp8 terms per value (mx_terms.h), token t in rows 2t and 2t + 1, so one
// instruction multiplies a piece of 16 rows by up to 8 tokens and the matrix core applies
// both operands' block scales. A wave's load instruction reads 64 contiguous bytes of each
// of 16 rows; consecutive pieces continue each row.
//
// Workgroup = W waves = one 16-row slice; wave w takes pieces [w MS, w MS + MS), loads its
// share of x, issues all its block and scale loads, converts its share of x into terms in
// its own LDS area (no barrier: no other wave reads them), runs its MFMAs, and the W
// partial sums meet in LDS.
//
// Semantics: tinyserve/mxfp4.py:20-53 (values FP4_LUT[code] 2^(scale - 127)),
// tinyserve/triton_dot_scaled.py:68-122 (x . deq(W)^T + bias, fp32 accumulation, bf16 out).
#include "fused_common.h"
#include "mfma_tile.h"
#include "mx_terms.h"

namespace tsa {
namespace {

constexpr int MXM_MAXT = 8;  // tokens per launch column: rows 2t, 2t + 1 of A
constexpr int MXM_XPRE = 2;  // x loads per lane issued ahead of the weights

struct MxmParams {
    const uint8_t* blocks;
    const uint8_t* scales;
    const void* bias;
    int bias_dtype;
    const uint16_t* x;  // bf16 [T, K]
    void* y;
    int y_dtype;
    int64_t T, N;
    int K, G, P;  // values, 32-value blocks and 128-wide pieces per row
    uint32_t blk_bytes, sc_bytes;
};

// LDS of a wave: per token its terms of the wave's MS pieces (hi 128 MS bytes, then lo) and
// an A-scale table over all blocks (only the wave's blocks are written and read); after the
// W waves' areas, the partial sums [W][MXM_MAXT][16] floats.
__host__ __device__ __forceinline__ int mxm_tb(int P) { return 16 * ((P + 3) / 4); }
__host__ __device__ __forceinline__ int mxm_wave_bytes(int MS, int P, int nt) {
    return (nt * (256 * MS + mxm_tb(P)) + 15) / 16 * 16;
}
__host__ __device__ __forceinline__ int mxm_lds(int W, int MS, int P, int nt) {
    return W * mxm_wave_bytes(MS, P, nt) + W * MXM_MAXT * 16 * 4;
}

template <int OPA>
__device__ __forceinline__ v4f mxm_mfma(const mxt_v8i& A, const mxt_v8i& B, const v4f& C, int sa, int sb) {
    return __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(A, B, C, 0, 4, OPA, sa, 0, sb);
}

template <int W, int MS>
__global__ void __launch_bounds__(64 * W) mxfp4_mv_mfma_kernel(MxmParams p) {
    extern __shared__ __align__(16) uint8_t smem[];
    const int tid = threadIdx.x, lane = tid & 63, wave = uniform(tid >> 6);
    const int64_t n0 = (int64_t)blockIdx.x * 16;
    const int64_t t0 = (int64_t)blockIdx.y * MXM_MAXT;
    const int nt = (int)(p.T - t0 < MXM_MAXT ? p.T - t0 : MXM_MAXT);
    const int i = lane & 15, q = lane >> 4;
    const int m0 = wave * MS;
    constexpr int LP = 128 * MS;  // bytes of one term over the wave's pieces
    const int tb = mxm_tb(p.P);
    uint8_t* area = smem + wave * mxm_wave_bytes(MS, p.P, nt);
    uint8_t* tables = area + nt * 2 * LP;

    // The wave's x chunks over its pieces below P (mv of them): item u = lane + 64 j is chunk
    // c0 + u % sw of token u / sw, c0 = 16 m0, sw = 16 mv (a block's four chunks are four
    // consecutive lanes, all valid or none: sw, 64 and C are multiples of 4). The first
    // MXM_XPRE are loaded before the weights, so the wait for them leaves the weight loads in
    // flight (a wave's loads complete in order).
    const int mv = m0 < p.P ? (p.P - m0 < MS ? p.P - m0 : MS) : 0;
    const int C = p.K / 8, c0 = 16 * m0, sw = 16 * mv, items = nt * sw;
    auto item_ok = [&](int u) { return u < items && c0 + u % sw < C; };
    auto item_src = [&](int u) {
        return reinterpret_cast<const u32x4*>(p.x + (t0 + u / sw) * p.K + 8 * (c0 + u % sw));
    };
    u32x4 xv[MXM_XPRE];
#pragma unroll
    for (int j = 0; j < MXM_XPRE; ++j) {
        const int u = lane + 64 * j;
        xv[j] = item_ok(u) ? *item_src(u) : u32x4{0u, 0u, 0u, 0u};
    }

    // this wave's pieces of row n0 + i: block 4m + q and its scale (zero past the row's
    // blocks or the matrix: out-of-range buffer offsets read zero)
    const __amdgpu_buffer_rsrc_t rb =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t*>(p.blocks), (short)0, (int)p.blk_bytes, 0x00020000);
    const __amdgpu_buffer_rsrc_t rs =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t*>(p.scales), (short)0, (int)p.sc_bytes, 0x00020000);
    u32x4 bq[MS];
    uint32_t bs[MS];
    const int64_t row = n0 + i;
#pragma unroll
    for (int j = 0; j < MS; ++j) {
        const int g = 4 * (m0 + j) + q;
        const bool ok = m0 + j < p.P && g < p.G && row < p.N;
        const uint32_t c = ok ? (uint32_t)(row * p.G + g) : 0xFFFFFFF0u;
        bq[j] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rb, ok ? 16u * c : 0xFFFFFFF0u, 0, 0));
        bs[j] = __builtin_amdgcn_raw_buffer_load_b8(rs, c, 0, 0);
    }

    // x as block-scaled terms in the wave's area; chunks past K get zero terms, blocks past
    // G a unit scale (their weights read zero, and every scale the MFMA takes is finite)
    auto convert = [&](int u, const u32x4& v) {
        const int t = u / sw, cl = u % sw, c = c0 + cl;
        uint8_t* hi = area + t * 2 * LP + 8 * cl;
        if (c < C) {
            block_terms(v, c >> 2, (c & 3) == 0, hi, hi + LP, tables + t * tb);
        } else {
            *reinterpret_cast<uint2*>(hi) = uint2{0u, 0u};
            *reinterpret_cast<uint2*>(hi + LP) = uint2{0u, 0u};
            if ((c & 3) == 0) tables[t * tb + ascale_byte(c >> 2)] = 127;
        }
    };
#pragma unroll
    for (int j = 0; j < MXM_XPRE; ++j)
        if (lane + 64 * j < items) convert(lane + 64 * j, xv[j]);
    for (int u = lane + 64 * MXM_XPRE; u < items; u += 64) convert(u, item_ok(u) ? *item_src(u) : u32x4{0u, 0u, 0u, 0u});
    // the wave reads what its own lanes wrote: LDS operations of a wave complete in order
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");

    // A rows: token r / 2, term r % 2; rows of absent tokens are zero (with token 0's
    // scales, all finite)
    const int r = lane & 15, ta = r >> 1;
    const bool live = ta < nt;
    const uint8_t* src = area + (live ? ta : 0) * 2 * LP + (r & 1) * LP + 16 * q;
    const uint8_t* aw = tables + (live ? ta : 0) * tb + 4 * q;
    v4f acc = v4f{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int j = 0; j < MS; ++j) {
        const int m = m0 + j;
        if (m >= p.P) break;  // wave-uniform
        u32x4 lo = lds16(src + 128 * j), hi = lds16(src + 128 * j + 64);
        if (!live) lo = hi = u32x4{0u, 0u, 0u, 0u};
        const mxt_v8i A = {(int)lo[0], (int)lo[1], (int)lo[2], (int)lo[3], (int)hi[0], (int)hi[1], (int)hi[2], (int)hi[3]};
        const mxt_v8i B = {(int)bq[j][0], (int)bq[j][1], (int)bq[j][2], (int)bq[j][3], 0, 0, 0, 0};
        const int sa = (int)*(const lds_u32*)(aw + 16 * (m >> 2));
        const int sb = (int)bs[j];
        switch (m & 3) {
            case 0: acc = mxm_mfma<0>(A, B, acc, sa, sb); break;
            case 1: acc = mxm_mfma<1>(A, B, acc, sa, sb); break;
            case 2: acc = mxm_mfma<2>(A, B, acc, sa, sb); break;
            default: acc = mxm_mfma<3>(A, B, acc, sa, sb); break;
        }
    }
    // lane 16g + i holds D rows 4g .. 4g + 3 of column i: tokens 2g (rows 4g, 4g + 1) and
    // 2g + 1 (rows 4g + 2, 4g + 3)
    float* part = reinterpret_cast<float*>(smem + W * mxm_wave_bytes(MS, p.P, nt));
    const int te = 2 * q, to = 2 * q + 1;
    if (te < nt) part[(wave * MXM_MAXT + te) * 16 + i] = acc[0] + acc[1];
    if (to < nt) part[(wave * MXM_MAXT + to) * 16 + i] = acc[2] + acc[3];
    __syncthreads();
    if (tid < 16 * nt) {
        const int t = tid >> 4, n = tid & 15;
        if (n0 + n < p.N) {
            float s = 0.0f;
#pragma unroll
            for (int w = 0; w < W; ++w) s += part[(w * MXM_MAXT + t) * 16 + n];
            if (p.bias) s += load_act(p.bias, p.bias_dtype, n0 + n);
            store_out(p.y, p.y_dtype, (t0 + t) * p.N + n0 + n, s);
        }
    }
}

template <int W, int MS>
const void* mxm_fn() { return reinterpret_cast<const void*>(&mxfp4_mv_mfma_kernel<W, MS>); }

}  // namespace

// Whether the matrix-core matvec takes a call: bf16 x, K a multiple of 32 up to 4096,
// 16-byte-aligned blocks and x, matrices under 4 GB (32-bit buffer offsets).
bool mxm_supported(const void* blocks, const void* x, int x_dtype, int64_t N, int64_t K) {
    return x_dtype == TSA_BF16 && K % 32 == 0 && K >= 32 && K <= 4096 &&
           (reinterpret_cast<uintptr_t>(blocks) & 15) == 0 && (reinterpret_cast<uintptr_t>(x) & 15) == 0 &&
           N * K / 2 < 0xFFFFFFF0ll;
}

int mxm_matvec(const uint8_t* blocks, const uint8_t* scales, const void* bias, int bias_dtype, const void* x,
               int64_t T, void* y, int y_dtype, int64_t N, int64_t K, hipStream_t st) {
    MxmParams p{};
    p.blocks = blocks;
    p.scales = scales;
    p.bias = bias;
    p.bias_dtype = bias_dtype;
    p.x = static_cast<const uint16_t*>(x);
    p.y = y;
    p.y_dtype = y_dtype;
    p.T = T;
    p.N = N;
    p.K = (int)K;
    p.G = (int)(K / 32);
    p.P = (p.G + 3) / 4;
    p.blk_bytes = (uint32_t)(N * K / 2);
    p.sc_bytes = (uint32_t)(N * K / 32);
    // 8 waves per 16-row slice, pieces spread evenly (MS <= 4 at K <= 4096)
    constexpr int W = 8;
    const int ms = (p.P + W - 1) / W;
    const int MS = ms <= 1 ? 1 : ms <= 2 ? 2 : ms <= 3 ? 3 : 4;
    const void* fn = MS == 1 ? mxm_fn<W, 1>() : MS == 2 ? mxm_fn<W, 2>() : MS == 3 ? mxm_fn<W, 3>() : mxm_fn<W, 4>();
    const int nt = T < MXM_MAXT ? (int)T : MXM_MAXT;
    const int lds = mxm_lds(W, MS, p.P, nt);
    const hipError_t e = ensure_dynamic_lds(fn, lds);
    TSA_REQUIRE(e == hipSuccess, TSA_ERR_HIP, "hipFuncSetAttribute(LDS %d): %s", lds, hipGetErrorString(e));
    void* args[] = {&p};
    TSA_HIP_CHECK(hipLaunchKernel(fn, dim3((unsigned)((N + 15) / 16), (unsigned)((T + MXM_MAXT - 1) / MXM_MAXT)),
                                  dim3(64 * W), args, lds, st));
    return TSA_OK;
}

}  // namespace tsa
