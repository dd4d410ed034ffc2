// Dequant-matvec kernels for small token counts (decode): y[t, n] = sum_k W[n, k] x[t, k].
//
// Launch shape: 256 threads (4 wave64s) per workgroup, ROWS_PER_WG output rows per
// workgroup, up to TCH tokens per launch column (grid.y walks token chunks). The
// activations of the chunk are staged once into LDS as float32; each wave owns whole
// rows and its 64 lanes stride over the row's 32-value units (GGUF) or 16-byte groups
// (MXFP4), so a wave's loads of one row are contiguous. Lanes reduce with a wave sum.
#include "rowdot.h"

namespace tsa {
namespace {

constexpr int ROWS_PER_WG = 8;
constexpr int MAX_X_LDS_BYTES = 64 * 1024;

// The chunk's tn token rows of x (contiguous in memory) as float32 into xs, rows past tn
// zero. From a 16-byte-aligned source in 16-byte loads, four per thread issued before any
// is converted (one element per load, as below, costs a memory round trip per element).
template <int TCH>
__device__ __forceinline__ int stage_x(float* xs, const void* x, int x_dtype, int64_t t0, int64_t T, int64_t K) {
    const int tn = (int)((T - t0) < TCH ? (T - t0) : TCH);
    const int es = x_dtype == TSA_F32 ? 4 : 2, per = 16 / es;  // elements per 16-byte chunk
    const uint8_t* src = static_cast<const uint8_t*>(x) + t0 * K * es;
    if ((reinterpret_cast<uintptr_t>(src) & 15u) == 0) {  // K % 32 == 0: rows are whole chunks
        const int64_t nch = (int64_t)tn * K / per;
        for (int64_t c0 = 0; c0 < nch; c0 += 4 * (int64_t)blockDim.x) {
            uint4 v[4];
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                const int64_t c = c0 + u * (int64_t)blockDim.x + threadIdx.x;
                v[u] = c < nch ? reinterpret_cast<const uint4*>(src)[c] : make_uint4(0u, 0u, 0u, 0u);
            }
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                const int64_t c = c0 + u * (int64_t)blockDim.x + threadIdx.x;
                if (c >= nch) continue;
                const uint32_t w[4] = {v[u].x, v[u].y, v[u].z, v[u].w};
                float* d = xs + c * per;
                if (x_dtype == TSA_F32) {
                    *reinterpret_cast<float4*>(d) = make_float4(__uint_as_float(w[0]), __uint_as_float(w[1]),
                                                                __uint_as_float(w[2]), __uint_as_float(w[3]));
                } else {
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        const float lo = x_dtype == TSA_BF16 ? bf16_bits_to_f32(w[i] & 0xFFFFu) : f16_bits_to_f32(w[i]);
                        const float hi = x_dtype == TSA_BF16 ? bf16_bits_to_f32(w[i] >> 16) : f16_bits_to_f32(w[i] >> 16);
                        *reinterpret_cast<float2*>(d + 2 * i) = make_float2(lo, hi);
                    }
                }
            }
        }
        for (int64_t i = (int64_t)tn * K + threadIdx.x; i < (int64_t)TCH * K; i += blockDim.x) xs[i] = 0.0f;
    } else {
        for (int64_t i = threadIdx.x; i < (int64_t)TCH * K; i += blockDim.x) {
            const int64_t t = i / K;
            xs[i] = t < tn ? load_act(x, x_dtype, (t0 + t) * K + (i - t * K)) : 0.0f;
        }
    }
    __syncthreads();
    return tn;
}

template <int TYPE, int A, int TCH>
__global__ void __launch_bounds__(256) gguf_matvec_kernel(const uint8_t* __restrict__ w, const void* __restrict__ x,
                                                          int x_dtype, int64_t T, int64_t K, void* __restrict__ y,
                                                          int y_dtype, int64_t N) {
    using Tr = GgufTraits<TYPE>;
    extern __shared__ float xs[];
    const int64_t t0 = (int64_t)blockIdx.y * TCH;
    const int tn = stage_x<TCH>(xs, x, x_dtype, t0, T, K);
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int64_t upr = K / 32;
    for (int r = wave; r < ROWS_PER_WG; r += 4) {
        const int64_t n = (int64_t)blockIdx.x * ROWS_PER_WG + r;
        if (n >= N) break;
        float acc[TCH];
#pragma unroll
        for (int t = 0; t < TCH; ++t) acc[t] = 0.0f;
        for (int64_t j = lane; j < upr; j += 64) {
            const int64_t U = n * upr + j;
            float v[32];
            decode_unit<TYPE, A>(w + (U / Tr::UPB) * Tr::TS, (int)(U % Tr::UPB), v);
#pragma unroll
            for (int t = 0; t < TCH; ++t) {
                const float4* xv = reinterpret_cast<const float4*>(xs + t * K + 32 * j);
                float a = 0.0f;
#pragma unroll
                for (int i = 0; i < 8; ++i) {
                    const float4 q = xv[i];
                    a += v[4 * i] * q.x + v[4 * i + 1] * q.y + v[4 * i + 2] * q.z + v[4 * i + 3] * q.w;
                }
                acc[t] += a;
            }
        }
#pragma unroll
        for (int t = 0; t < TCH; ++t) {
            const float s = wave_sum(acc[t]);
            if (lane == 0 && t < tn) store_out(y, y_dtype, (t0 + t) * N + n, s);
        }
    }
}

template <int A, int TCH>
__global__ void __launch_bounds__(256) mxfp4_matvec_kernel(const uint8_t* __restrict__ blocks,
                                                           const uint8_t* __restrict__ scales,
                                                           const void* __restrict__ bias, int bias_dtype,
                                                           const void* __restrict__ x, int x_dtype, int64_t T,
                                                           void* __restrict__ y, int y_dtype, int64_t N, int64_t K) {
    extern __shared__ float xs[];
    const int64_t t0 = (int64_t)blockIdx.y * TCH;
    const int tn = stage_x<TCH>(xs, x, x_dtype, t0, T, K);
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int64_t G = K / 32;
    for (int r = wave; r < ROWS_PER_WG; r += 4) {
        const int64_t n = (int64_t)blockIdx.x * ROWS_PER_WG + r;
        if (n >= N) break;
        float acc[TCH];
#pragma unroll
        for (int t = 0; t < TCH; ++t) acc[t] = 0.0f;
        for (int64_t g = lane; g < G; g += 64) {
            const int64_t c = n * G + g;
            uint32_t q[4];
            if constexpr (A >= 16) {
                const uint4 v = reinterpret_cast<const uint4*>(blocks)[c];
                q[0] = v.x; q[1] = v.y; q[2] = v.z; q[3] = v.w;
            } else {
                __builtin_memcpy(q, blocks + 16 * c, 16);
            }
            const float s = e8m0_to_f32(scales[c]);
#pragma unroll
            for (int t = 0; t < TCH; ++t) acc[t] += mx16_dot(q, xs + t * K + 32 * g) * s;
        }
        const float b = bias ? load_act(bias, bias_dtype, n) : 0.0f;
#pragma unroll
        for (int t = 0; t < TCH; ++t) {
            const float s = wave_sum(acc[t]);
            if (lane == 0 && t < tn) store_out(y, y_dtype, (t0 + t) * N + n, s + b);
        }
    }
}

// MXFP4 on 16-byte-aligned blocks: each wave owns MR rows and issues every block and scale
// load of them (GH 16-byte groups per lane and row, G <= 64 GH) before the first is used, so
// a lane has MR * GH loads in flight rather than one; the activations are staged meanwhile.
// Same arithmetic as mxfp4_matvec_kernel (per group: the fp4 dot in fp32, times the scale).
template <int GH, int MR, int TCH>
__global__ void __launch_bounds__(256) mxfp4_mv_kernel(const uint8_t* __restrict__ blocks,
                                                       const uint8_t* __restrict__ scales,
                                                       const void* __restrict__ bias, int bias_dtype,
                                                       const void* __restrict__ x, int x_dtype, int64_t T,
                                                       void* __restrict__ y, int y_dtype, int64_t N, int64_t K) {
    extern __shared__ float xs[];
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int64_t G = K / 32;
    const int64_t n0 = ((int64_t)blockIdx.x * 4 + wave) * MR;
    uint4 q[MR][GH];
    uint32_t sc[MR][GH];
#pragma unroll
    for (int r = 0; r < MR; ++r)
#pragma unroll
        for (int h = 0; h < GH; ++h) {
            const int64_t g = lane + 64 * h, c = (n0 + r) * G + g;
            const bool ok = g < G && n0 + r < N;
            q[r][h] = ok ? reinterpret_cast<const uint4*>(blocks)[c] : make_uint4(0u, 0u, 0u, 0u);
            sc[r][h] = ok ? scales[c] : 127u;
        }
    const int64_t t0 = (int64_t)blockIdx.y * TCH;
    const int tn = stage_x<TCH>(xs, x, x_dtype, t0, T, K);
    float acc[MR][TCH];
#pragma unroll
    for (int r = 0; r < MR; ++r)
#pragma unroll
        for (int t = 0; t < TCH; ++t) acc[r][t] = 0.0f;
#pragma unroll
    for (int h = 0; h < GH; ++h) {
        const int64_t g = lane + 64 * h;
        if (g >= G) break;
#pragma unroll
        for (int r = 0; r < MR; ++r) {
            const uint32_t qq[4] = {q[r][h].x, q[r][h].y, q[r][h].z, q[r][h].w};
            const float s = e8m0_to_f32(sc[r][h]);
#pragma unroll
            for (int t = 0; t < TCH; ++t) acc[r][t] += mx16_dot(qq, xs + t * K + 32 * g) * s;
        }
    }
#pragma unroll
    for (int r = 0; r < MR; ++r) {
        const int64_t n = n0 + r;
        const float b = bias && n < N ? load_act(bias, bias_dtype, n) : 0.0f;
#pragma unroll
        for (int t = 0; t < TCH; ++t) {
            const float s = wave_sum(acc[r][t]);
            if (lane == 0 && t < tn && n < N) store_out(y, y_dtype, (t0 + t) * N + n, s + b);
        }
    }
}

template <int GH, int MR>
hipError_t launch_mv(const uint8_t* bl, const uint8_t* sc, const void* bias, int bias_dtype, const void* x,
                     int x_dtype, int64_t T, void* y, int y_dtype, int64_t N, int64_t K, int tch, hipStream_t st) {
    const dim3 block(256), grid((unsigned)((N + 4 * MR - 1) / (4 * MR)), (unsigned)((T + tch - 1) / tch));
    const size_t lds = (size_t)tch * K * sizeof(float);
    switch (tch) {
        case 4: hipLaunchKernelGGL((mxfp4_mv_kernel<GH, MR, 4>), grid, block, lds, st, bl, sc, bias, bias_dtype, x, x_dtype, T, y, y_dtype, N, K); break;
        case 2: hipLaunchKernelGGL((mxfp4_mv_kernel<GH, MR, 2>), grid, block, lds, st, bl, sc, bias, bias_dtype, x, x_dtype, T, y, y_dtype, N, K); break;
        default: hipLaunchKernelGGL((mxfp4_mv_kernel<GH, MR, 1>), grid, block, lds, st, bl, sc, bias, bias_dtype, x, x_dtype, T, y, y_dtype, N, K); break;
    }
    return hipGetLastError();
}

// Groups per lane GH = ceil(G / 64) (K <= 16384: G <= 512), rows per wave MR so that a lane
// holds 4 groups (8 at G > 256). For 5760 x 2880 (GH 2) rows per wave 1 / 2 / 4 / 8 measured
// 9.67 / 7.73 / 8.45 / 9.45 us.
hipError_t launch_mx_aligned(const uint8_t* bl, const uint8_t* sc, const void* bias, int bias_dtype, const void* x,
                             int x_dtype, int64_t T, void* y, int y_dtype, int64_t N, int64_t K, int tch,
                             hipStream_t st) {
    const int64_t G = K / 32;
    if (G <= 64) return launch_mv<1, 4>(bl, sc, bias, bias_dtype, x, x_dtype, T, y, y_dtype, N, K, tch, st);
    if (G <= 128) return launch_mv<2, 2>(bl, sc, bias, bias_dtype, x, x_dtype, T, y, y_dtype, N, K, tch, st);
    if (G <= 256) return launch_mv<4, 1>(bl, sc, bias, bias_dtype, x, x_dtype, T, y, y_dtype, N, K, tch, st);
    return launch_mv<8, 1>(bl, sc, bias, bias_dtype, x, x_dtype, T, y, y_dtype, N, K, tch, st);
}

template <int TYPE, int A>
hipError_t launch_gguf(const uint8_t* w, const void* x, int x_dtype, int64_t T, int64_t K, void* y, int y_dtype,
                       int64_t N, int tch, hipStream_t st) {
    const dim3 block(256), grid((unsigned)((N + ROWS_PER_WG - 1) / ROWS_PER_WG), (unsigned)((T + tch - 1) / tch));
    const size_t lds = (size_t)tch * K * sizeof(float);
    switch (tch) {
        case 4: hipLaunchKernelGGL((gguf_matvec_kernel<TYPE, A, 4>), grid, block, lds, st, w, x, x_dtype, T, K, y, y_dtype, N); break;
        case 2: hipLaunchKernelGGL((gguf_matvec_kernel<TYPE, A, 2>), grid, block, lds, st, w, x, x_dtype, T, K, y, y_dtype, N); break;
        default: hipLaunchKernelGGL((gguf_matvec_kernel<TYPE, A, 1>), grid, block, lds, st, w, x, x_dtype, T, K, y, y_dtype, N); break;
    }
    return hipGetLastError();
}

template <int A>
hipError_t launch_mx(const uint8_t* bl, const uint8_t* sc, const void* bias, int bias_dtype, const void* x, int x_dtype,
                     int64_t T, void* y, int y_dtype, int64_t N, int64_t K, int tch, hipStream_t st) {
    const dim3 block(256), grid((unsigned)((N + ROWS_PER_WG - 1) / ROWS_PER_WG), (unsigned)((T + tch - 1) / tch));
    const size_t lds = (size_t)tch * K * sizeof(float);
    switch (tch) {
        case 4: hipLaunchKernelGGL((mxfp4_matvec_kernel<A, 4>), grid, block, lds, st, bl, sc, bias, bias_dtype, x, x_dtype, T, y, y_dtype, N, K); break;
        case 2: hipLaunchKernelGGL((mxfp4_matvec_kernel<A, 2>), grid, block, lds, st, bl, sc, bias, bias_dtype, x, x_dtype, T, y, y_dtype, N, K); break;
        default: hipLaunchKernelGGL((mxfp4_matvec_kernel<A, 1>), grid, block, lds, st, bl, sc, bias, bias_dtype, x, x_dtype, T, y, y_dtype, N, K); break;
    }
    return hipGetLastError();
}

int pick_tch(int64_t T, int64_t K) {
    int tch = T >= 4 ? 4 : (T >= 2 ? 2 : 1);
    while (tch > 1 && (int64_t)tch * K * 4 > MAX_X_LDS_BYTES) tch >>= 1;
    return tch;
}

}  // namespace
}  // namespace tsa

namespace tsa {
bool mxm_supported(const void* blocks, const void* x, int x_dtype, int64_t N, int64_t K);
int mxm_matvec(const uint8_t* blocks, const uint8_t* scales, const void* bias, int bias_dtype, const void* x,
               int64_t T, void* y, int y_dtype, int64_t N, int64_t K, hipStream_t st);
const char* gq_matvec_unsupported(int type, const void* w, int64_t T, int64_t K, int64_t N, int x_dtype);
int gq_matvec(int type, const uint8_t* w, int64_t w_bytes, const void* x, int x_dtype, int64_t T, int64_t K, void* y,
              int y_dtype, int64_t N, hipStream_t st);
const char* gs_unsupported(int type, int64_t K);
int gs_matvec(int type, const uint8_t* w, int64_t w_bytes, const void* x, int x_dtype, int64_t T, int64_t K, void* y,
              int y_dtype, int64_t N, hipStream_t st);
}  // namespace tsa

using namespace tsa;

// Up to this many tokens per call run on the super-block streaming matvec (gguf_matvec.hip,
// one workgroup column per token); more tokens reuse each decoded unit across a chunk of
// tokens in the row kernel above.
constexpr int64_t GQ_MATVEC_MAX_T = 8;

extern "C" int tsa_gguf_matvec(int ggml_type, const void* w, int64_t w_bytes, const void* x, int x_dtype, int64_t T,
                               int64_t K, void* y, int y_dtype, int64_t N, void* stream) {
    clear_error();
    int be, ts;
    TSA_REQUIRE(gguf_geometry(ggml_type, &be, &ts), TSA_ERR_UNSUPPORTED_TYPE,
                "Unsupported ggml_type: %d. Supported: Q8_0(8), Q4_K(12), Q5_K(13), Q6_K(14)", ggml_type);
    TSA_REQUIRE(valid_dtype(x_dtype) && valid_dtype(y_dtype), TSA_ERR_INVALID_ARG, "bad dtype (x %d, y %d)", x_dtype,
                y_dtype);
    TSA_REQUIRE(N >= 0 && K >= 0 && T >= 0, TSA_ERR_INVALID_ARG, "negative size");
    TSA_REQUIRE(K % 32 == 0, TSA_ERR_SHAPE, "in_features (%lld) must be divisible by block_elements (32)", (long long)K);
    TSA_REQUIRE((N * K) % be == 0, TSA_ERR_SHAPE,
                "out_features*in_features (%lld) must be a whole number of blocks (%d values each)",
                (long long)(N * K), be);
    const int64_t expected = N * K / be * ts;
    TSA_REQUIRE(w_bytes >= expected, TSA_ERR_WEIGHT_TOO_SMALL, "weight_data too small: got %lld bytes, expected %lld",
                (long long)w_bytes, (long long)expected);
    TSA_REQUIRE(K * 4 <= MAX_X_LDS_BYTES, TSA_ERR_SHAPE, "in_features (%lld) exceeds the supported maximum (%d)",
                (long long)K, MAX_X_LDS_BYTES / 4);
    if (N == 0 || T == 0) return TSA_OK;
    TSA_REQUIRE(w && x && y, TSA_ERR_INVALID_ARG, "null pointer");
    const uint8_t* wb = static_cast<const uint8_t*>(w);
    hipStream_t st = as_stream(stream);
    // the sub-block stream (moe_decode_gs.hip) first, then the super-block matvec
    if (T <= GQ_MATVEC_MAX_T && !*gs_unsupported(ggml_type, K) && (reinterpret_cast<uintptr_t>(w) & 1) == 0 &&
        (reinterpret_cast<uintptr_t>(x) & 15) == 0 && N * K < ((int64_t)1 << 31) &&
        T * K * (x_dtype == TSA_F32 ? 4 : 2) < ((int64_t)1 << 32) - 16)
        return gs_matvec(ggml_type, wb, w_bytes, x, x_dtype, T, K, y, y_dtype, N, st);
    if (T <= GQ_MATVEC_MAX_T && !*gq_matvec_unsupported(ggml_type, w, T, K, N, x_dtype))
        return gq_matvec(ggml_type, wb, w_bytes, x, x_dtype, T, K, y, y_dtype, N, st);
    const bool a16 = (reinterpret_cast<uintptr_t>(w) & 15) == 0, a2 = (reinterpret_cast<uintptr_t>(w) & 1) == 0;
    const int tch = pick_tch(T, K);
    hipError_t e;
    switch (ggml_type) {
        case 8: e = a2 ? launch_gguf<8, 2>(wb, x, x_dtype, T, K, y, y_dtype, N, tch, st)
                       : launch_gguf<8, 1>(wb, x, x_dtype, T, K, y, y_dtype, N, tch, st); break;
        case 12: e = a16 ? launch_gguf<12, 16>(wb, x, x_dtype, T, K, y, y_dtype, N, tch, st)
                         : launch_gguf<12, 1>(wb, x, x_dtype, T, K, y, y_dtype, N, tch, st); break;
        case 13: e = a16 ? launch_gguf<13, 16>(wb, x, x_dtype, T, K, y, y_dtype, N, tch, st)
                         : launch_gguf<13, 1>(wb, x, x_dtype, T, K, y, y_dtype, N, tch, st); break;
        default: e = a2 ? launch_gguf<14, 2>(wb, x, x_dtype, T, K, y, y_dtype, N, tch, st)
                        : launch_gguf<14, 1>(wb, x, x_dtype, T, K, y, y_dtype, N, tch, st); break;
    }
    TSA_HIP_CHECK(e);
    return TSA_OK;
}

extern "C" int tsa_mxfp4_matvec(const void* blocks, const void* scales, const void* bias, int bias_dtype,
                                const void* x, int x_dtype, int64_t T, void* y, int y_dtype, int64_t N, int64_t K,
                                void* stream) {
    clear_error();
    TSA_REQUIRE(valid_dtype(x_dtype) && valid_dtype(y_dtype) && (!bias || valid_dtype(bias_dtype)),
                TSA_ERR_INVALID_ARG, "bad dtype (x %d, y %d, bias %d)", x_dtype, y_dtype, bias_dtype);
    TSA_REQUIRE(N >= 0 && K >= 0 && T >= 0, TSA_ERR_INVALID_ARG, "negative size");
    TSA_REQUIRE(K % 32 == 0, TSA_ERR_SHAPE, "in_features (%lld) must be a multiple of 32", (long long)K);
    TSA_REQUIRE(K * 4 <= MAX_X_LDS_BYTES, TSA_ERR_SHAPE, "in_features (%lld) exceeds the supported maximum (%d)",
                (long long)K, MAX_X_LDS_BYTES / 4);
    if (N == 0 || T == 0) return TSA_OK;
    TSA_REQUIRE(blocks && scales && x && y, TSA_ERR_INVALID_ARG, "null pointer");
    const uint8_t* bl = static_cast<const uint8_t*>(blocks);
    const uint8_t* sc = static_cast<const uint8_t*>(scales);
    hipStream_t st = as_stream(stream);
    // bf16 tokens, a few at a time: the matrix-core form (mx_matvec.hip)
    if (T <= 32 && mxm_supported(blocks, x, x_dtype, N, K))
        return mxm_matvec(bl, sc, bias, bias_dtype, x, T, y, y_dtype, N, K, st);
    const int tch = pick_tch(T, K);
    hipError_t e = (reinterpret_cast<uintptr_t>(blocks) & 15) == 0
                       ? launch_mx_aligned(bl, sc, bias, bias_dtype, x, x_dtype, T, y, y_dtype, N, K, tch, st)
                       : launch_mx<1>(bl, sc, bias, bias_dtype, x, x_dtype, T, y, y_dtype, N, K, tch, st);
    TSA_HIP_CHECK(e);
    return TSA_OK;
}
