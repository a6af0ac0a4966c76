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
    int sync_stream(int dev, const void* stream) {
        int cur = 0;
        SEERA_HIP_TRY(hipGetDevice(&cur));
        if (cur != dev) SEERA_HIP_TRY(hipSetDevice(dev));
        const hipError_t e = hipStreamSynchronize(static_cast<hipStream_t>(const_cast<void*>(stream)));
        if (cur != dev) SEERA_HIP_TRY(hipSetDevice(cur));
        SEERA_HIP_TRY(e);
        return SEERA_OK;
    }
};

// Whether work queued on `st` now would be captured. A refused query counts
// as capturing when the refusal itself says a capture is under way
// (hipErrorStreamCaptureImplicit: the legacy null stream while another stream
// is capturing in global mode; hipErrorStreamCaptureUnsupported); any other
// refusal means the stream cannot be captured. The query's sticky error is
// cleared either way.
bool stream_capturing(hipStream_t st) {
    hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
    const hipError_t e = hipStreamIsCapturing(st, &cap);
    if (e != hipSuccess) {
        (void)hipGetLastError();
        return e == hipErrorStreamCaptureImplicit || e == hipErrorStreamCaptureUnsupported;
    }
    return cap != hipStreamCaptureStatusNone;
}
HipBackend g_hip_backend;
WorkspacePool<HipBackend> g_pool(g_hip_backend);
// Second buffer per (device, stream): operands re-laid out for a kernel that
// takes workspace() itself (staging_workspace).
WorkspacePool<HipBackend> g_stage_pool(g_hip_backend);
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

namespace {
int pool_get(WorkspacePool<HipBackend>& pool, size_t bytes, void** out, hipStream_t st) {
    int dev = 0;
    SEERA_HIP_TRY(hipGetDevice(&dev));
    const bool cap = stream_capturing(st);
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    const int e = pool.get(dev, st, bytes, cap, out);
    if (e == WorkspacePool<HipBackend>::kGrowUnderCapture)
        return fail(SEERA_ERR_INVALID_ARGUMENT,
                    "the workspace must grow to %zu bytes during stream capture: make one eager "
                    "call of the same sizes on this stream before capturing",
                    bytes);
    return e;
}
}  // namespace

int staging_workspace(size_t bytes, void** out, hipStream_t st) {
    *out = nullptr;
    if (g_fixed_owner)
        return fail(SEERA_ERR_INVALID_ARGUMENT, "%s: no staging buffer under a fixed workspace",
                    g_fixed_owner);
    return pool_get(g_stage_pool, bytes, out, st);
}

int staging_workspace_try(size_t bytes, void** out, hipStream_t st, bool* got) {
    *out = nullptr;
    *got = false;
    if (g_fixed_owner) return SEERA_OK;
    int dev = 0;
    SEERA_HIP_TRY(hipGetDevice(&dev));
    const bool cap = stream_capturing(st);
    int e;
    {
        std::lock_guard<std::mutex> lock(g_scratch_mu);
        e = g_stage_pool.get(dev, st, bytes, cap, out);
    }
    if (e == WorkspacePool<HipBackend>::kGrowUnderCapture) return SEERA_OK;
    if (e == SEERA_ERR_OUT_OF_MEMORY) {
        (void)hipGetLastError();  // the failed hipMalloc's status, so later launch checks do not see it
        clear_error();
        *out = nullptr;
        return SEERA_OK;
    }
    if (e != SEERA_OK) return e;
    *got = true;
    return SEERA_OK;
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
    return pool_get(g_pool, bytes, out, st);
}

void streams_gone_for_pending(hipStream_t st);

int stream_destroyed(hipStream_t st) {
    if (!st) return SEERA_OK;
    streams_gone_for_pending(st);
    int dev = 0;
    SEERA_HIP_TRY(hipStreamGetDevice(st, &dev));
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    const int e = g_pool.stream_destroyed(dev, st);
    const int e2 = g_stage_pool.stream_destroyed(dev, st);
    return e ? e : e2;
}

int graph_created(void* exec) {
    int dev = 0;
    SEERA_HIP_TRY(hipGetDevice(&dev));
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    g_pool.graph_created(exec, dev);
    g_stage_pool.graph_created(exec, dev);
    return SEERA_OK;
}

int graph_destroyed(void* exec) {
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    const int e = g_pool.graph_destroyed(exec);
    const int e2 = g_stage_pool.graph_destroyed(exec);
    return e ? e : e2;
}

void workspace_stats(size_t* held, size_t* retired_count) {
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (held) *held = g_pool.held_bytes() + g_stage_pool.held_bytes();
    if (retired_count) *retired_count = g_pool.retired_count() + g_stage_pool.retired_count();
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
// A block handed back by device_free_async: free for work queued on `stream`
// after the free, for anything else once `ev` (recorded on the stream at the
// free) has completed. stream_gone: the stream was destroyed (its handle may
// come back for a new stream), so only the event counts.
struct PendingBlock {
    void* ptr;
    hipStream_t stream;
    hipEvent_t ev;
    bool stream_gone;
};
std::mutex g_alloc_mu;
std::unordered_map<void*, LiveBlock> g_live;
std::map<std::pair<int, size_t>, std::vector<void*>> g_cached;
std::map<std::pair<int, size_t>, std::vector<PendingBlock>> g_pending;
std::map<int, std::vector<hipEvent_t>> g_spare_events;  // per device, recorded events to reuse
size_t g_live_bytes = 0, g_cached_bytes = 0, g_pending_bytes = 0;
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
// Takes a block of (dev, cls) from the pending list that work on `st` may use
// now: one freed on `st` itself (stream order puts this request after that
// free), else one whose free event has completed. Caller holds g_alloc_mu.
void* take_pending(int dev, size_t cls, hipStream_t st, bool same_stream_ok) {
    auto it = g_pending.find({dev, cls});
    if (it == g_pending.end()) return nullptr;
    std::vector<PendingBlock>& v = it->second;
    for (int pass = 0; pass < 2; ++pass) {
        for (size_t i = v.size(); i-- > 0;) {
            const PendingBlock& b = v[i];
            bool ok;
            if (pass == 0) {
                ok = same_stream_ok && !b.stream_gone && b.stream == st;
            } else {
                const hipError_t q = hipEventQuery(b.ev);
                if (q != hipSuccess && q != hipErrorNotReady) (void)hipGetLastError();
                ok = q == hipSuccess;
            }
            if (!ok) continue;
            void* p = b.ptr;
            g_spare_events[dev].push_back(b.ev);
            v.erase(v.begin() + (ptrdiff_t)i);
            g_pending_bytes -= cls;
            return p;
        }
    }
    return nullptr;
}

// Moves every pending block into the cache (the caller has synchronized the
// device, so all their events have completed) and destroys the spare events.
// Caller holds g_alloc_mu.
void drain_pending(int dev) {
    for (auto it = g_pending.begin(); it != g_pending.end();) {
        if (dev >= 0 && it->first.first != dev) {
            ++it;
            continue;
        }
        for (const PendingBlock& b : it->second) {
            g_cached[it->first].push_back(b.ptr);
            g_cached_bytes += it->first.second;
            g_pending_bytes -= it->first.second;
            (void)hipEventDestroy(b.ev);
        }
        it = g_pending.erase(it);
    }
    for (auto it = g_spare_events.begin(); it != g_spare_events.end();) {
        if (dev >= 0 && it->first != dev) {
            ++it;
            continue;
        }
        for (hipEvent_t e : it->second) (void)hipEventDestroy(e);
        it = g_spare_events.erase(it);
    }
}

bool capturing(hipStream_t st) { return stream_capturing(st); }

// The allocation itself: a cached block of the class, a pending one that `st`
// may use (st == nullptr and same_stream_ok false: only completed ones), or
// hipMalloc (after a failure: synchronize, reclaim every cached and pending
// block of the device and retry once). Caller holds g_alloc_mu.
int alloc_locked(int dev, size_t cls, hipStream_t st, bool same_stream_ok, void** out) {
    *out = take_pending(dev, cls, st, same_stream_ok);
    if (!*out) {
        auto it = g_cached.find({dev, cls});
        if (it != g_cached.end() && !it->second.empty()) {
            *out = it->second.back();
            it->second.pop_back();
            g_cached_bytes -= cls;
        }
    }
    if (!*out) {
        hipError_t e = hipMalloc(out, cls);
        if (e == hipErrorOutOfMemory || e == hipErrorMemoryAllocation) {
            (void)hipGetLastError();  // clear the sticky allocation error
            SEERA_HIP_TRY(hipDeviceSynchronize());
            drain_pending(dev);
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
}  // namespace

void note_async_work() { g_async_pending.store(true, std::memory_order_release); }
void note_device_synchronized() { g_async_pending.store(false, std::memory_order_release); }

int device_malloc(void** out, size_t nbytes) {
    *out = nullptr;
    int dev = 0;
    SEERA_HIP_TRY(hipGetDevice(&dev));
    std::lock_guard<std::mutex> lock(g_alloc_mu);
    return alloc_locked(dev, size_class(nbytes), nullptr, false, out);
}

int device_malloc_async(void** out, size_t nbytes, hipStream_t st) {
    *out = nullptr;
    if (capturing(st))
        return fail(SEERA_ERR_INVALID_ARGUMENT,
                    "stream-ordered allocation is not supported during graph capture");
    int dev = 0;
    SEERA_HIP_TRY(hipGetDevice(&dev));
    std::lock_guard<std::mutex> lock(g_alloc_mu);
    return alloc_locked(dev, size_class(nbytes), st, true, out);
}

int device_free_async(void* ptr, hipStream_t st) {
    if (!ptr) return SEERA_OK;
    if (capturing(st))
        return fail(SEERA_ERR_INVALID_ARGUMENT,
                    "stream-ordered free is not supported during graph capture");
    std::lock_guard<std::mutex> lock(g_alloc_mu);
    auto it = g_live.find(ptr);
    if (it == g_live.end())
        return fail(SEERA_ERR_INVALID_ARGUMENT,
                    "seera_hip_free_async: %p was not allocated by seera_hip_malloc(_async)", ptr);
    const LiveBlock b = it->second;
    std::vector<hipEvent_t>& spare = g_spare_events[b.dev];
    hipEvent_t ev = nullptr;
    if (!spare.empty()) {
        ev = spare.back();
        spare.pop_back();
    } else {
        SEERA_HIP_TRY(hipEventCreateWithFlags(&ev, hipEventDisableTiming));
    }
    const hipError_t e = hipEventRecord(ev, st);
    if (e != hipSuccess) {
        spare.push_back(ev);
        return fail_hip(e, "hipEventRecord for a stream-ordered free");
    }
    g_live.erase(it);
    g_live_bytes -= b.bytes;
    g_pending[{b.dev, b.bytes}].push_back(PendingBlock{ptr, st, ev, false});
    g_pending_bytes += b.bytes;
    return SEERA_OK;
}

void streams_gone_for_pending(hipStream_t st) {
    std::lock_guard<std::mutex> lock(g_alloc_mu);
    for (auto& kv : g_pending)
        for (PendingBlock& b : kv.second)
            if (b.stream == st) b.stream_gone = true;
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
    drain_pending(-1);
    return release_cached(-1);
}

void device_memory_stats(size_t* live_bytes, size_t* cached_bytes) {
    std::lock_guard<std::mutex> lock(g_alloc_mu);
    if (live_bytes) *live_bytes = g_live_bytes;
    if (cached_bytes) *cached_bytes = g_cached_bytes + g_pending_bytes;
}

int device_cus() {
    int dev = 0, n = 0;
    if (hipGetDevice(&dev) != hipSuccess ||
        hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0)
        return 256;
    return n;
}

}  // namespace seera
