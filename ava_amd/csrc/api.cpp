// Error reporting and version of the C ABI (include/ava.h).
#include <stdarg.h>
#include <string.h>

#include <mutex>
#include <set>
#include <utility>

#include "common.h"

namespace {
thread_local char g_err[512] = "";
}

namespace ava {

void set_error(const char *fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_err, sizeof g_err, fmt, ap);
    va_end(ap);
}

int fail(int code, const char *fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_err, sizeof g_err, fmt, ap);
    va_end(ap);
    return code;
}

int lds_opt_in(const void *fn, size_t bytes) {
    static std::mutex mu;
    static std::set<std::pair<int, const void *>> done;
    int dev = 0;
    AVA_HIP(hipGetDevice(&dev));
    std::lock_guard<std::mutex> lock(mu);
    if (done.count({dev, fn})) return AVA_OK;
    AVA_HIP(hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, (int)bytes));
    done.insert({dev, fn});
    return AVA_OK;
}

int device_cus(int *cus) {
    static std::mutex mu;
    static int n[64] = {};
    int dev = 0;
    AVA_HIP(hipGetDevice(&dev));
    AVA_REQUIRE(dev >= 0 && dev < 64, AVA_ERR_UNSUPPORTED, "device %d (0..63)", dev);
    std::lock_guard<std::mutex> lock(mu);
    if (!n[dev]) AVA_HIP(hipDeviceGetAttribute(&n[dev], hipDeviceAttributeMultiprocessorCount, dev));
    *cus = n[dev];
    return AVA_OK;
}

}  // namespace ava

extern "C" const char *ava_last_error(void) { return g_err; }

extern "C" const char *ava_version(void) { return "ava_amd 0.1 (gfx950)"; }

// FNV-1a over n bytes, continuing from h (the reference's model fingerprint, gpu/state.rs:1095-1107).
extern "C" uint64_t ava_fnv1a64(const void *p, size_t n, uint64_t h) {
    const unsigned char *b = static_cast<const unsigned char *>(p);
    for (size_t i = 0; i < n; ++i) {
        h ^= b[i];
        h *= 0x100000001b3ull;
    }
    return h;
}
