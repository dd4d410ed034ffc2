// Shared host/device helpers of the tinyserve_amd HIP library (gfx950 only).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stdarg.h>
#include <stdio.h>

#include "../../include/tinyserve_amd.h"

namespace tsa {

// ---------------------------------------------------------------- host-side errors
// Thread-local message of the last failing call (read through tsa_last_error()).
void set_error(const char* fmt, ...) __attribute__((format(printf, 1, 2)));
void clear_error();

#define TSA_REQUIRE(cond, status, ...)      \
    do {                                    \
        if (!(cond)) {                      \
            ::tsa::set_error(__VA_ARGS__);  \
            return (status);                \
        }                                   \
    } while (0)

#define TSA_HIP_CHECK(expr)                                                         \
    do {                                                                            \
        hipError_t e_ = (expr);                                                     \
        if (e_ != hipSuccess) {                                                     \
            ::tsa::set_error("HIP error: %s (%s)", hipGetErrorString(e_), #expr);   \
            return TSA_ERR_HIP;                                                     \
        }                                                                           \
    } while (0)

// After a kernel launch: report launch-configuration errors without synchronising.
#define TSA_LAUNCH_CHECK() TSA_HIP_CHECK(hipGetLastError())

inline hipStream_t as_stream(void* s) { return reinterpret_cast<hipStream_t>(s); }

inline bool valid_dtype(int dt) { return dt == TSA_F32 || dt == TSA_F16 || dt == TSA_BF16; }
inline int dtype_size(int dt) { return dt == TSA_F32 ? 4 : 2; }

// GGUF block geometry for the hot-path types. Returns false for other ids.
inline bool gguf_geometry(int type, int* block_elems, int* type_size) {
    switch (type) {
        case 8:  *block_elems = 32;  *type_size = 34;  return true;   // Q8_0
        case 12: *block_elems = 256; *type_size = 144; return true;   // Q4_K
        case 13: *block_elems = 256; *type_size = 176; return true;   // Q5_K
        case 14: *block_elems = 256; *type_size = 210; return true;   // Q6_K
        default: return false;
    }
}

int num_cus();  // compute units of the current device (cached per device)
// Allow `fn` `bytes` of dynamic LDS on the current device (hipFuncSetAttribute once per
// device and kernel, for launches above the 64 KiB default; thread-safe).
hipError_t ensure_dynamic_lds(const void* fn, int bytes);

// The MoE decode workspace starts with a sync area of MXT_SYNC_BYTES, used only by the
// one-launch MXFP4 decode (moe_decode_mxt.hip): a call counter and one flag per workgroup of
// a launch (at most MXT_SYNC_GFLAGS gate_up and MXT_SYNC_DFLAGS down workgroups: T <= 4,
// k <= 16, inter, hidden <= 3072). The other decode paths start after it.
constexpr int64_t MXT_SYNC_BYTES = 32 << 10;
constexpr int MXT_SYNC_GFLAGS = 4 * 16 * 96;
constexpr int MXT_SYNC_DFLAGS = 4 * 192;
constexpr uint32_t MXT_GEN_POISON = 0x7E7E7E7Eu;  // the call counter after a wait gave up
// Process-wide settings of the tiled MXFP4 decode (tsa_set_decode_options): its form (0 one
// launch, 1 two launches) and how many polls a one-launch wait makes before it gives up.
int mxt_form();
uint32_t mxt_wait_limit();


// ---------------------------------------------------------------- device helpers
// IEEE binary16 bits -> float by v_cvt_f32_f16: exact for every half, subnormals included
// (HIP kernels run with f16/f64 denormals preserved; a signalling NaN comes back quiet).
__device__ __forceinline__ float f16_bits_to_f32(uint32_t h) {
    return (float)__builtin_bit_cast(_Float16, (uint16_t)(h & 0xFFFFu));
}

__device__ __forceinline__ float bf16_bits_to_f32(uint32_t b) { return __uint_as_float(b << 16); }

// float -> bfloat16 bits, round to nearest even; NaN -> canonical quiet NaN.
__device__ __forceinline__ uint16_t f32_to_bf16_bits(float f) {
    const uint32_t u = __float_as_uint(f);
    if ((u & 0x7FFFFFFFu) > 0x7F800000u) return 0x7FC0;
    return (uint16_t)((u + 0x7FFFu + ((u >> 16) & 1u)) >> 16);
}

__device__ __forceinline__ uint16_t f32_to_f16_bits(float f) {
    _Float16 h = (_Float16)f;  // v_cvt_f16_f32: round to nearest even
    return __builtin_bit_cast(uint16_t, h);
}

__device__ __forceinline__ float load_act(const void* p, int dtype, int64_t i) {
    if (dtype == TSA_F32) return static_cast<const float*>(p)[i];
    const uint16_t b = static_cast<const uint16_t*>(p)[i];
    return dtype == TSA_BF16 ? bf16_bits_to_f32(b) : f16_bits_to_f32(b);
}

__device__ __forceinline__ void store_out(void* p, int dtype, int64_t i, float v) {
    if (dtype == TSA_F32) static_cast<float*>(p)[i] = v;
    else if (dtype == TSA_BF16) static_cast<uint16_t*>(p)[i] = f32_to_bf16_bits(v);
    else static_cast<uint16_t*>(p)[i] = f32_to_f16_bits(v);
}

// Sum over the 64 lanes of a wavefront; every lane receives the total.
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off, 64);
    return v;
}

__device__ __forceinline__ float sigmoidf_(float x) { return 1.0f / (1.0f + expf(-x)); }

}  // namespace tsa
