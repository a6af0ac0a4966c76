// runtime.h -- host-side plumbing shared by the entry points: per-thread error
// messages, HIP status checking and the per-device scratch workspace.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#include "../../include/seera_hip.h"

namespace seera {

// Records a message for seera_hip_last_error() and returns `code`.
int fail(int code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));
int fail_hip(hipError_t e, const char* what);
void clear_error();

#define SEERA_HIP_TRY(expr)                                   \
    do {                                                      \
        hipError_t seera_e_ = (expr);                         \
        if (seera_e_ != hipSuccess) return fail_hip(seera_e_, #expr); \
    } while (0)

#define SEERA_TRY(expr)                 \
    do {                                \
        int seera_s_ = (expr);          \
        if (seera_s_ != SEERA_OK) return seera_s_; \
    } while (0)

// Device scratch owned by the library (split-K partials, re-laid-out weights).
// Grows on demand and is kept until process exit. A grow synchronizes the
// device first so no queued kernel still uses the old buffer. Not safe for
// concurrent calls from several host threads on one device.
int workspace(size_t bytes, void** out);

// Caching device allocator behind seera_hip_malloc / seera_hip_free (size
// classes per device; see runtime.cpp). A free synchronizes the device first
// when an *_async entry point may have left work queued.
int device_malloc(void** out, size_t nbytes);
int device_free(void* ptr);
int device_empty_cache();
void device_memory_stats(size_t* live_bytes, size_t* cached_bytes);
// Called by the *_async entry points after they enqueue work, and after every
// device-wide synchronization.
void note_async_work();
void note_device_synchronized();

// Launch-shape sanity: every grid the library builds must fit these limits.
constexpr int64_t kMaxGridX = 0x7fffffff;

}  // namespace seera
