// Library-level C ABI: version, status strings, per-thread last error, block geometry.
#include <map>
#include <mutex>
#include <utility>
#include <vector>

#include "tsa_common.h"

namespace tsa {

static thread_local char g_last_error[1024] = "";

void set_error(const char* fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
    va_end(ap);
}

void clear_error() { g_last_error[0] = '\0'; }

int num_cus() {
    static std::mutex mu;
    static std::vector<int> cache;
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) return 0;
    std::lock_guard<std::mutex> lock(mu);
    if ((int)cache.size() <= dev) cache.resize(dev + 1, 0);
    if (cache[dev] == 0) {
        int n = 0;
        if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess) cache[dev] = n;
    }
    return cache[dev];
}

hipError_t ensure_dynamic_lds(const void* fn, int bytes) {
    if (bytes <= 64 * 1024) return hipSuccess;
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return e;
    static std::mutex mu;
    static std::map<std::pair<int, const void*>, int> set;  // (device, kernel) -> bytes allowed
    std::lock_guard<std::mutex> lock(mu);
    int& have = set[{dev, fn}];
    if (have >= bytes) return hipSuccess;
    e = hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, bytes);
    if (e == hipSuccess) have = bytes;
    return e;
}

}  // namespace tsa

extern "C" int tsa_version(void) { return 1; }

extern "C" const char* tsa_last_error(void) { return tsa::g_last_error; }

extern "C" const char* tsa_status_string(int status) {
    switch (status) {
        case TSA_OK: return "ok";
        case TSA_ERR_INVALID_ARG: return "invalid argument";
        case TSA_ERR_UNSUPPORTED_TYPE: return "unsupported type";
        case TSA_ERR_SHAPE: return "unsupported shape";
        case TSA_ERR_WEIGHT_TOO_SMALL: return "weight buffer too small";
        case TSA_ERR_ACT_TOO_SMALL: return "activation buffer too small";
        case TSA_ERR_WORKSPACE: return "workspace too small";
        case TSA_ERR_HIP: return "HIP runtime error";
        default: return "unknown status";
    }
}

extern "C" int tsa_gguf_block_info(int ggml_type, int64_t* block_elems, int64_t* type_size) {
    tsa::clear_error();
    int be = 0, ts = 0;
    if (ggml_type == 0) { be = 1; ts = 4; }
    else if (ggml_type == 1) { be = 1; ts = 2; }
    else if (!tsa::gguf_geometry(ggml_type, &be, &ts)) {
        tsa::set_error("Unsupported ggml_type: %d. Supported: Q8_0(8), Q4_K(12), Q5_K(13), Q6_K(14)", ggml_type);
        return TSA_ERR_UNSUPPORTED_TYPE;
    }
    if (block_elems) *block_elems = be;
    if (type_size) *type_size = ts;
    return TSA_OK;
}
