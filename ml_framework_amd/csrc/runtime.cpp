// runtime.cpp -- error reporting and the per-device workspace.
#include "runtime.h"

#include <stdarg.h>
#include <stdio.h>

#include <mutex>

namespace seera {

namespace {
thread_local char g_msg[512] = "";

struct DeviceScratch {
    void* ptr = nullptr;
    size_t bytes = 0;
};
constexpr int kMaxDevices = 64;
DeviceScratch g_scratch[kMaxDevices];
std::mutex g_scratch_mu;
}  // namespace

int fail(int code, const char* fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_msg, sizeof(g_msg), fmt, ap);
    va_end(ap);
    return code;
}

int fail_hip(hipError_t e, const char* what) {
    const int code = (e == hipErrorOutOfMemory || e == hipErrorMemoryAllocation)
                         ? SEERA_ERR_OUT_OF_MEMORY
                         : SEERA_ERR_HIP;
    return fail(code, "%s: %s (%d)", what, hipGetErrorString(e), (int)e);
}

void clear_error() { g_msg[0] = 0; }

const char* last_error() { return g_msg; }

int workspace(size_t bytes, void** out) {
    int dev = 0;
    SEERA_HIP_TRY(hipGetDevice(&dev));
    if (dev < 0 || dev >= kMaxDevices) return fail(SEERA_ERR_HIP, "device id %d out of range", dev);
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    DeviceScratch& s = g_scratch[dev];
    if (bytes > s.bytes) {
        if (s.ptr) {
            // Kernels queued earlier may still read the old buffer.
            SEERA_HIP_TRY(hipDeviceSynchronize());
            SEERA_HIP_TRY(hipFree(s.ptr));
            s.ptr = nullptr;
            s.bytes = 0;
        }
        // Round up to 1 MiB so small growth steps do not reallocate.
        const size_t want = (bytes + (1u << 20) - 1) & ~(size_t)((1u << 20) - 1);
        SEERA_HIP_TRY(hipMalloc(&s.ptr, want));
        s.bytes = want;
    }
    *out = s.ptr;
    return SEERA_OK;
}

}  // namespace seera
