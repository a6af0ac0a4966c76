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

// Device scratch owned by the library (split-K partials, re-laid-out weights,
// dW and bias partials): one buffer per (device, stream), so calls on two
// streams never share one. Grows on demand and is kept until process exit; a
// grow synchronizes the device first so no queued kernel still uses the old
// buffer, and while a HIP graph is live on the device the old buffer is kept
// (a replay still writes to it) until the device's last graph is destroyed.
// Growing while `st` is being captured fails with SEERA_ERR_INVALID_ARGUMENT.
int workspace(size_t bytes, void** out, hipStream_t st);
// A second buffer per (device, stream) under the same rules, for operands
// staged in a new layout before a call that itself takes workspace() (the two
// never alias). Not available under FixedWorkspace.
int staging_workspace(size_t bytes, void** out, hipStream_t st);
// The same, for a staging copy the caller can do without: where the buffer
// cannot be had without allocating under graph capture or a fixed workspace,
// or the device is out of memory for it, returns SEERA_OK with *got false and
// nothing reported, so the caller takes its path without the copy.
int staging_workspace_try(size_t bytes, void** out, hipStream_t st, bool* got);

// Compute units of the current device (256 if the query fails).
int device_cus();

// While alive, workspace() on this host thread hands out [ptr, ptr + bytes)
// instead of the library's buffers and fails (naming `owner`) for requests
// above `bytes`. Used by the entry point that must not allocate.
class FixedWorkspace {
public:
    FixedWorkspace(void* ptr, size_t bytes, const char* owner);
    ~FixedWorkspace();
    FixedWorkspace(const FixedWorkspace&) = delete;
    FixedWorkspace& operator=(const FixedWorkspace&) = delete;
};

// Called before a stream is destroyed: frees its workspace (or keeps it for
// the device's live graphs).
int stream_destroyed(hipStream_t st);
// Graph bookkeeping for the workspace rule above (capi.cpp calls these when
// an executable graph is instantiated and destroyed).
int graph_created(void* exec);
int graph_destroyed(void* exec);
// Bytes held by workspaces and the number of retired (graph-pinned) buffers.
void workspace_stats(size_t* held, size_t* retired_count);

// Caching device allocator behind seera_hip_malloc / seera_hip_free (size
// classes per device; see runtime.cpp). A free synchronizes the device first
// when an *_async entry point may have left work queued.
int device_malloc(void** out, size_t nbytes);
int device_free(void* ptr);
// Stream-ordered: the block is usable by work queued on `st` after the call;
// a block freed with device_free_async goes to work on its own stream at once
// and elsewhere once the work queued before the free has completed.
int device_malloc_async(void** out, size_t nbytes, hipStream_t st);
int device_free_async(void* ptr, hipStream_t st);
int device_empty_cache();
void device_memory_stats(size_t* live_bytes, size_t* cached_bytes);
// Called by the *_async entry points after they enqueue work, and after every
// device-wide synchronization.
void note_async_work();
void note_device_synchronized();

// Launch-shape sanity: every grid the library builds must fit these limits.
constexpr int64_t kMaxGridX = 0x7fffffff;

}  // namespace seera
