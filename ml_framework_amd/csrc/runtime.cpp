// runtime.cpp -- error reporting, the per-device workspace and the caching
// device allocator behind seera_hip_malloc / seera_hip_free.
#include "runtime.h"
#include "workspace_pool.h"

#include <stdarg.h>
#include <stdio.h>

#include <atomic>
#include <map>
#include <mutex>
#include <unordered_map>
#include <utility>
#include <vector>

namespace seera {

namespace {
thread_local char g_msg[512] = "";

// Workspaces: one per (device, stream), kept and grown by WorkspacePool
// (workspace_pool.h) over the HIP backend below.
struct HipBackend {
    int alloc(int, size_t bytes, void** out) {
        SEERA_HIP_TRY(hipMalloc(out, bytes));
        return SEERA_OK;
    }
    int release(int, void* p) {
        SEERA_HIP_TRY(hipFree(p));
        return SEERA_OK;
    }
    int sync(int dev) {
        int cur = 0;
        SEERA_HIP_TRY(hipGetDevice(&cur));
        if (cur != dev) SEERA_HIP_TRY(hipSetDevice(dev));
        const hipError_t e = hipDeviceSynchronize();
        if (cur != dev) SEERA_HIP_TRY(hipSetDevice(cur));
        SEERA_HIP_TRY(e);
        return SEERA_OK;
    }
};
HipBackend g_hip_backend;
WorkspacePool<HipBackend> g_pool(g_hip_backend);
std::mutex g_scratch_mu;

// A caller-supplied scratch region that workspace() hands out instead of the
// library's own buffers (seera_hip_matmul_noalloc), per host thread.
thread_local void* g_fixed_ptr = nullptr;
thread_local size_t g_fixed_bytes = 0;
thread_local const char* g_fixed_owner = nullptr;
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

FixedWorkspace::FixedWorkspace(void* ptr, size_t bytes, const char* owner) {
    g_fixed_ptr = ptr;
    g_fixed_bytes = bytes;
    g_fixed_owner = owner;
}
FixedWorkspace::~FixedWorkspace() {
    g_fixed_ptr = nullptr;
    g_fixed_bytes = 0;
    g_fixed_owner = nullptr;
}

int workspace(size_t bytes, void** out, hipStream_t st) {
    *out = nullptr;
    if (g_fixed_owner) {
        if (bytes > g_fixed_bytes)
            return fail(SEERA_ERR_INVALID_ARGUMENT,
                        "%s: this call needs %zu bytes of scratch, above its fixed maximum of %zu",
                        g_fixed_owner, bytes, g_fixed_bytes);
        *out = g_fixed_ptr;
        return SEERA_OK;
    }
    int dev = 0;
    SEERA_HIP_TRY(hipGetDevice(&dev));
    hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
    if (hipStreamIsCapturing(st, &cap) != hipSuccess) {
        // Not a capturable stream (the query is refused, e.g. for the legacy
        // null stream in some runtime states): it is not being captured.
        (void)hipGetLastError();
        cap = hipStreamCaptureStatusNone;
    }
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    const int e = g_pool.get(dev, st, bytes, cap != hipStreamCaptureStatusNone, out);
    if (e == WorkspacePool<HipBackend>::kGrowUnderCapture)
        return fail(SEERA_ERR_INVALID_ARGUMENT,
                    "the workspace must grow to %zu bytes during stream capture: make one eager "
                    "call of the same sizes on this stream before capturing",
                    bytes);
    return e;
}

int stream_destroyed(hipStream_t st) {
    if (!st) return SEERA_OK;
    int dev = 0;
    SEERA_HIP_TRY(hipStreamGetDevice(st, &dev));
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    return g_pool.stream_destroyed(dev, st);
}

int graph_created(void* exec) {
    int dev = 0;
    SEERA_HIP_TRY(hipGetDevice(&dev));
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    g_pool.graph_created(exec, dev);
    return SEERA_OK;
}

int graph_destroyed(void* exec) {
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    return g_pool.graph_destroyed(exec);
}

void workspace_stats(size_t* held, size_t* retired_count) {
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (held) *held = g_pool.held_bytes();
    if (retired_count) *retired_count = g_pool.retired_count();
}

// ---------------------------------------------------------------------------
// Caching device allocator. The reference allocates every tensor and every
// temporary with cudaMalloc and releases it with cudaFree (cuTen.py:77-84,
// cuda_bindings.cpp:23-59); on HIP both calls are slow and the free
// synchronizes the device. Here a freed block is kept in a per-device list of
// its size class and handed to the next request of that class:
//   <= 512 B          512 B
//   <= 1 MiB          the next power of two
//   larger            a multiple of 2 MiB
// A free must not hand out memory that queued kernels still use. Every
// blocking entry point synchronizes the device before it returns, so only the
// *_async ones can leave work behind: they raise a flag, and a free that finds
// it raised synchronizes the device first (what cudaFree does every time).
// When hipMalloc fails, the cached blocks of that device are released and the
// request is retried once.
// ---------------------------------------------------------------------------
namespace {
struct LiveBlock {
    int dev;
    size_t bytes;  // size class
};
std::mutex g_alloc_mu;
std::unordered_map<void*, LiveBlock> g_live;
std::map<std::pair<int, size_t>, std::vector<void*>> g_cached;
size_t g_live_bytes = 0, g_cached_bytes = 0;
std::atomic<bool> g_async_pending{false};

size_t size_class(size_t n) {
    if (n <= 512) return 512;
    if (n <= ((size_t)1 << 20)) {
        size_t c = 1024;
        while (c < n) c <<= 1;
        return c;
    }
    const size_t g = (size_t)2 << 20;
    return (n + g - 1) / g * g;
}

// Releases every cached block of `dev` (all devices when dev < 0). Caller
// holds g_alloc_mu.
int release_cached(int dev) {
    for (auto it = g_cached.begin(); it != g_cached.end();) {
        if (dev >= 0 && it->first.first != dev) {
            ++it;
            continue;
        }
        int cur = 0;
        SEERA_HIP_TRY(hipGetDevice(&cur));
        SEERA_HIP_TRY(hipSetDevice(it->first.first));
        // Erase each block as it is freed: after a failed hipFree the list
        // holds exactly the blocks that are still allocated.
        std::vector<void*>& blocks = it->second;
        while (!blocks.empty()) {
            const hipError_t e = hipFree(blocks.back());
            if (e != hipSuccess) {
                (void)hipSetDevice(cur);
                return fail_hip(e, "hipFree of a cached block");
            }
            blocks.pop_back();
            g_cached_bytes -= it->first.second;
        }
        SEERA_HIP_TRY(hipSetDevice(cur));
        it = g_cached.erase(it);
    }
    return SEERA_OK;
}
}  // namespace

void note_async_work() { g_async_pending.store(true, std::memory_order_release); }
void note_device_synchronized() { g_async_pending.store(false, std::memory_order_release); }

int device_malloc(void** out, size_t nbytes) {
    *out = nullptr;
    int dev = 0;
    SEERA_HIP_TRY(hipGetDevice(&dev));
    const size_t cls = size_class(nbytes);
    std::lock_guard<std::mutex> lock(g_alloc_mu);
    auto it = g_cached.find({dev, cls});
    if (it != g_cached.end() && !it->second.empty()) {
        *out = it->second.back();
        it->second.pop_back();
        g_cached_bytes -= cls;
    } else {
        hipError_t e = hipMalloc(out, cls);
        if (e == hipErrorOutOfMemory || e == hipErrorMemoryAllocation) {
            (void)hipGetLastError();  // clear the sticky allocation error
            SEERA_HIP_TRY(hipDeviceSynchronize());
            SEERA_TRY(release_cached(dev));
            e = hipMalloc(out, cls);
        }
        if (e != hipSuccess) {
            *out = nullptr;
            return fail_hip(e, "hipMalloc");
        }
    }
    g_live[*out] = LiveBlock{dev, cls};
    g_live_bytes += cls;
    return SEERA_OK;
}

int device_free(void* ptr) {
    if (!ptr) return SEERA_OK;
    std::lock_guard<std::mutex> lock(g_alloc_mu);
    auto it = g_live.find(ptr);
    if (it == g_live.end()) {
        // Not from this allocator: release it the plain way.
        SEERA_HIP_TRY(hipFree(ptr));
        return SEERA_OK;
    }
    if (g_async_pending.exchange(false, std::memory_order_acq_rel)) {
        const hipError_t e = hipDeviceSynchronize();
        if (e != hipSuccess) {
            g_async_pending.store(true);
            return fail_hip(e, "hipDeviceSynchronize before reusing a freed block");
        }
    }
    const LiveBlock b = it->second;
    g_live.erase(it);
    g_live_bytes -= b.bytes;
    g_cached[{b.dev, b.bytes}].push_back(ptr);
    g_cached_bytes += b.bytes;
    return SEERA_OK;
}

int device_empty_cache() {
    std::lock_guard<std::mutex> lock(g_alloc_mu);
    SEERA_HIP_TRY(hipDeviceSynchronize());
    return release_cached(-1);
}

void device_memory_stats(size_t* live_bytes, size_t* cached_bytes) {
    std::lock_guard<std::mutex> lock(g_alloc_mu);
    if (live_bytes) *live_bytes = g_live_bytes;
    if (cached_bytes) *cached_bytes = g_cached_bytes;
}

int device_cus() {
    int dev = 0, n = 0;
    if (hipGetDevice(&dev) != hipSuccess ||
        hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0)
        return 256;
    return n;
}

}  // namespace seera
