// MXFP4 16-row MFMA tile order (device layout of the fast decode path).
//
// A wave multiplies 16 weight rows at a time with v_mfma_f32_16x16x32_bf16, whose A
// operand gives lane 16q+i row i and 8 consecutive K values of K-slice q. Each lane
// expands one 16-byte MXFP4 block (32 values) into four such operands, so one MFMA group
// m covers blocks 4m..4m+3 of 16 rows: exactly 1 KB. Storing each group's 1 KB in lane
// order makes every operand fetch one fully contiguous 16-byte-per-lane load, which
// streams from HBM like a memcpy (a row-major fetch of the same operands touches 16 rows
// per load and runs at ~60% of that rate on MI355X).
//
//   tile r (rows 16r..16r+15) = 256*G bytes, G = K/32 blocks per row;
//   block b of row 16r+i at tile offset 1024*(b/4) + 16*(16*(b%4) + i)
//   (a short last group just ends early, so the tile is dense);
//   its e8m0 scale is byte m%4 (m = b/4) of 32-bit word w = m/4 of lane l = 16*(b%4) + i;
//   a lane's W = ceil(ceil(G/4)/4) words are stored in chunks of 4: chunk c = w/4 holds
//   words 4c..4c+3 of every lane, lane-major, each lane's part width min(4, W - 4c) words,
//   so a wave fetches all its scales with one 16-byte (and one shorter) load per lane.
//   The tile-scale area is 256 * W bytes, zero where no block exists.
#include "tsa_common.h"

namespace tsa {

int64_t mx_tile_groups(int64_t K) { return (K / 32 + 3) / 4; }              // MFMA groups per row tile
int64_t mx_tile_scale_words(int64_t K) { return (mx_tile_groups(K) + 3) / 4; }  // per lane
int64_t mx_tile_scale_bytes(int64_t K) { return 256 * mx_tile_scale_words(K); }  // per row tile

namespace {

// One thread per (row, block): moves 16 bytes and one scale byte.
__global__ void __launch_bounds__(256) mx_tile_kernel(const uint8_t* __restrict__ blocks,
                                                      const uint8_t* __restrict__ scales, int64_t N, int64_t G,
                                                      int64_t W, uint8_t* __restrict__ tb, uint8_t* __restrict__ ts) {
    const int64_t c = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (c >= N * G) return;
    const int64_t n = c / G, b = c % G;
    const int64_t r = n / 16, i = n % 16;
    const int64_t lanepos = 16 * (b % 4) + i;
    const uint4 v = *reinterpret_cast<const uint4*>(blocks + 16 * c);
    *reinterpret_cast<uint4*>(tb + r * 256 * G + 1024 * (b / 4) + 16 * lanepos) = v;
    const int64_t w = b / 16, ch = w / 4, width = W - 4 * ch < 4 ? W - 4 * ch : 4;
    ts[r * 256 * W + 1024 * ch + 4 * width * lanepos + 4 * (w % 4) + (b / 4) % 4] = scales[c];
}

// Zero n bytes (the tiled scale area's padding words must read zero). A kernel, not
// hipMemsetAsync, so that the call can be captured into a HIP graph.
__global__ void __launch_bounds__(256) mx_zero_kernel(uint8_t* __restrict__ p, int64_t n) {
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x)
        p[i] = 0;
}

}  // namespace
}  // namespace tsa

using namespace tsa;

extern "C" int tsa_mxfp4_tile_sizes(int64_t N, int64_t K, int64_t* blocks_bytes, int64_t* scales_bytes) {
    clear_error();
    TSA_REQUIRE(blocks_bytes && scales_bytes, TSA_ERR_INVALID_ARG, "null output pointer");
    TSA_REQUIRE(N > 0 && K > 0 && N % 16 == 0 && K % 32 == 0, TSA_ERR_SHAPE,
                "tiled MXFP4 needs N %% 16 == 0 and K %% 32 == 0 (N %lld, K %lld)", (long long)N, (long long)K);
    *blocks_bytes = N * K / 2;
    *scales_bytes = N / 16 * mx_tile_scale_bytes(K);
    return TSA_OK;
}

extern "C" int tsa_mxfp4_tile(const void* blocks, const void* scales, int64_t N, int64_t K, void* tiled_blocks,
                              void* tiled_scales, void* stream) {
    int64_t bb = 0, sb = 0;
    int rc = tsa_mxfp4_tile_sizes(N, K, &bb, &sb);
    if (rc) return rc;
    TSA_REQUIRE(blocks && scales && tiled_blocks && tiled_scales, TSA_ERR_INVALID_ARG, "null pointer");
    TSA_REQUIRE(((reinterpret_cast<uintptr_t>(blocks) | reinterpret_cast<uintptr_t>(tiled_blocks)) & 15) == 0,
                TSA_ERR_INVALID_ARG, "blocks and tiled_blocks must be 16-byte aligned");
    hipStream_t st = as_stream(stream);
    hipLaunchKernelGGL(mx_zero_kernel, dim3((unsigned)((sb + 255) / 256 < 1024 ? (sb + 255) / 256 : 1024)), dim3(256),
                       0, st, static_cast<uint8_t*>(tiled_scales), sb);
    TSA_LAUNCH_CHECK();
    const int64_t G = K / 32, n = N * G;
    hipLaunchKernelGGL(mx_tile_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st,
                       static_cast<const uint8_t*>(blocks), static_cast<const uint8_t*>(scales), N, G,
                       mx_tile_scale_words(K), static_cast<uint8_t*>(tiled_blocks), static_cast<uint8_t*>(tiled_scales));
    TSA_LAUNCH_CHECK();
    return TSA_OK;
}
