// Bit-exact dequantisation kernels: GGUF (Q8_0/Q4_K/Q5_K/Q6_K, F32/F16) and MXFP4.
//
// One thread decodes one 32-value unit and writes it; the unit decoders are shared
// with the matvec and MoE kernels (formats.h).
#include "formats.h"

namespace tsa {
namespace {

template <int TYPE, int A>
__global__ void __launch_bounds__(256) gguf_dequant_kernel(const uint8_t* __restrict__ data, int64_t n_units,
                                                           void* __restrict__ out, int out_dtype) {
    using Tr = GgufTraits<TYPE>;
    const int64_t unit = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (unit >= n_units) return;
    const int64_t blk = unit / Tr::UPB;
    const int u = (int)(unit % Tr::UPB);
    float v[32];
    decode_unit<TYPE, A>(data + blk * Tr::TS, u, v);
    const int64_t base = unit * 32;
    if (out_dtype == TSA_F32) {
        float4* o = reinterpret_cast<float4*>(static_cast<float*>(out) + base);
#pragma unroll
        for (int i = 0; i < 8; ++i) o[i] = make_float4(v[4 * i], v[4 * i + 1], v[4 * i + 2], v[4 * i + 3]);
    } else {
        uint32_t* o = reinterpret_cast<uint32_t*>(static_cast<uint16_t*>(out) + base);
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            const uint32_t lo = out_dtype == TSA_BF16 ? f32_to_bf16_bits(v[2 * i]) : f32_to_f16_bits(v[2 * i]);
            const uint32_t hi = out_dtype == TSA_BF16 ? f32_to_bf16_bits(v[2 * i + 1]) : f32_to_f16_bits(v[2 * i + 1]);
            o[i] = lo | (hi << 16);
        }
    }
}

// F32 / F16 "dequantisation" (tinyserve/gguf_dequant_torch.py:54-59): reinterpret and convert.
__global__ void __launch_bounds__(256) plain_dequant_kernel(const uint8_t* __restrict__ data, int src_f16,
                                                            int64_t n, void* __restrict__ out, int out_dtype) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    float v;
    if (src_f16) {
        uint16_t h;
        __builtin_memcpy(&h, data + 2 * i, 2);
        v = f16_bits_to_f32(h);
    } else {
        __builtin_memcpy(&v, data + 4 * i, 4);
    }
    store_out(out, out_dtype, i, v);
}

// One thread per 16-byte group chunk (32 values) of row n, group g.
__global__ void __launch_bounds__(256) mxfp4_dequant_kernel(const uint8_t* __restrict__ blocks,
                                                            const uint8_t* __restrict__ scales, int64_t N,
                                                            int64_t G, void* __restrict__ out, int out_dtype,
                                                            int transpose) {
    const int64_t c = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (c >= N * G) return;
    const int64_t n = c / G, g = c % G, K = G * 32;
    uint32_t w[4];
    __builtin_memcpy(w, blocks + c * 16, 16);
    const float s = e8m0_to_f32(scales[c]);
#pragma unroll
    for (int j = 0; j < 16; ++j) {
        const uint32_t byte = (w[j >> 2] >> (8 * (j & 3))) & 0xFFu;
        const float lo = e2m1_to_f32(byte & 15u) * s, hi = e2m1_to_f32(byte >> 4) * s;
        const int64_t k0 = 32 * g + 2 * j;
        if (!transpose) {
            store_out(out, out_dtype, n * K + k0, lo);
            store_out(out, out_dtype, n * K + k0 + 1, hi);
        } else {
            store_out(out, out_dtype, k0 * N + n, lo);
            store_out(out, out_dtype, (k0 + 1) * N + n, hi);
        }
    }
}

inline unsigned grid_for(int64_t n, int threads) { return (unsigned)((n + threads - 1) / threads); }

}  // namespace
}  // namespace tsa

using namespace tsa;

extern "C" int tsa_gguf_dequant(int ggml_type, const void* data, int64_t data_bytes, int64_t n_elems, void* out,
                                int out_dtype, void* stream) {
    clear_error();
    TSA_REQUIRE(valid_dtype(out_dtype), TSA_ERR_INVALID_ARG, "out_dtype %d is not F32(0)/F16(1)/BF16(2)", out_dtype);
    TSA_REQUIRE(n_elems >= 0 && data_bytes >= 0, TSA_ERR_INVALID_ARG, "negative size");
    if (n_elems == 0) return TSA_OK;
    TSA_REQUIRE(data != nullptr && out != nullptr, TSA_ERR_INVALID_ARG, "null pointer");
    hipStream_t st = as_stream(stream);
    if (ggml_type == 0 || ggml_type == 1) {
        const int64_t need = n_elems * (ggml_type == 0 ? 4 : 2);
        TSA_REQUIRE(data_bytes >= need, TSA_ERR_WEIGHT_TOO_SMALL, "data too small: got %lld bytes, expected %lld",
                    (long long)data_bytes, (long long)need);
        hipLaunchKernelGGL(plain_dequant_kernel, dim3(grid_for(n_elems, 256)), dim3(256), 0, st,
                           static_cast<const uint8_t*>(data), ggml_type == 1, n_elems, out, out_dtype);
        TSA_LAUNCH_CHECK();
        return TSA_OK;
    }
    int be, ts;
    TSA_REQUIRE(gguf_geometry(ggml_type, &be, &ts), TSA_ERR_UNSUPPORTED_TYPE,
                "Unsupported GGML quantization type %d. Supported: [0, 1, 8, 12, 13, 14]", ggml_type);
    TSA_REQUIRE(n_elems % be == 0, TSA_ERR_SHAPE, "n_elems (%lld) must be a multiple of the block size (%d)",
                (long long)n_elems, be);
    const int64_t need = n_elems / be * ts;
    TSA_REQUIRE(data_bytes >= need, TSA_ERR_WEIGHT_TOO_SMALL, "data too small: got %lld bytes, expected %lld",
                (long long)data_bytes, (long long)need);
    const int64_t n_units = n_elems / 32;
    const uint8_t* d = static_cast<const uint8_t*>(data);
    const bool a16 = (reinterpret_cast<uintptr_t>(data) & 15) == 0;
    const bool a2 = (reinterpret_cast<uintptr_t>(data) & 1) == 0;
    const bool out_ok = (reinterpret_cast<uintptr_t>(out) & (out_dtype == TSA_F32 ? 15 : 3)) == 0;
    TSA_REQUIRE(out_ok, TSA_ERR_INVALID_ARG, "out must be %d-byte aligned", out_dtype == TSA_F32 ? 16 : 4);
    const dim3 grid(grid_for(n_units, 256)), block(256);
    switch (ggml_type) {
        case 8:
            if (a2) hipLaunchKernelGGL((gguf_dequant_kernel<8, 2>), grid, block, 0, st, d, n_units, out, out_dtype);
            else hipLaunchKernelGGL((gguf_dequant_kernel<8, 1>), grid, block, 0, st, d, n_units, out, out_dtype);
            break;
        case 12:
            if (a16) hipLaunchKernelGGL((gguf_dequant_kernel<12, 16>), grid, block, 0, st, d, n_units, out, out_dtype);
            else hipLaunchKernelGGL((gguf_dequant_kernel<12, 1>), grid, block, 0, st, d, n_units, out, out_dtype);
            break;
        case 13:
            if (a16) hipLaunchKernelGGL((gguf_dequant_kernel<13, 16>), grid, block, 0, st, d, n_units, out, out_dtype);
            else hipLaunchKernelGGL((gguf_dequant_kernel<13, 1>), grid, block, 0, st, d, n_units, out, out_dtype);
            break;
        default:
            if (a2) hipLaunchKernelGGL((gguf_dequant_kernel<14, 2>), grid, block, 0, st, d, n_units, out, out_dtype);
            else hipLaunchKernelGGL((gguf_dequant_kernel<14, 1>), grid, block, 0, st, d, n_units, out, out_dtype);
            break;
    }
    TSA_LAUNCH_CHECK();
    return TSA_OK;
}

extern "C" int tsa_mxfp4_dequant(const void* blocks, const void* scales, int64_t N, int64_t K, void* out,
                                 int out_dtype, int transpose, void* stream) {
    clear_error();
    TSA_REQUIRE(valid_dtype(out_dtype), TSA_ERR_INVALID_ARG, "out_dtype %d is not F32(0)/F16(1)/BF16(2)", out_dtype);
    TSA_REQUIRE(N >= 0 && K >= 0, TSA_ERR_INVALID_ARG, "negative size");
    TSA_REQUIRE(K % 32 == 0, TSA_ERR_SHAPE, "in_features (%lld) must be a multiple of 32", (long long)K);
    if (N == 0 || K == 0) return TSA_OK;
    TSA_REQUIRE(blocks && scales && out, TSA_ERR_INVALID_ARG, "null pointer");
    const int64_t G = K / 32;
    hipLaunchKernelGGL(mxfp4_dequant_kernel, dim3(grid_for(N * G, 256)), dim3(256), 0, as_stream(stream),
                       static_cast<const uint8_t*>(blocks), static_cast<const uint8_t*>(scales), N, G, out, out_dtype,
                       transpose);
    TSA_LAUNCH_CHECK();
    return TSA_OK;
}
