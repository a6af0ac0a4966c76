// workspace_pool.h -- bookkeeping of the library's device workspaces, written
// against an abstract backend so that the rules can be tested on a host with
// no GPU (tests/cpp/test_workspace_pool.cpp drives it with a fake backend).
//
// Rules:
//   * one workspace per (device, stream): calls on one stream run in order and
//     share it, calls on two streams never do;
//   * a workspace grows on demand (rounded up to 1 MiB) and is kept;
//   * growing frees the old buffer after synchronizing its own stream (the
//     only eager work that can still use it is queued there); while any
//     executable graph is live on that device the old buffer is retired
//     instead, with no synchronize at all, since a replay still writes to the
//     address it was captured with; the device's retired buffers are freed,
//     after a device synchronize, when its last graph is destroyed;
//   * growing while the stream is being captured is refused (kGrowUnderCapture):
//     the capture would record a buffer that a later call could free;
//   * destroying a stream (or releasing a caller-owned stream's workspace)
//     frees its workspace after synchronizing that stream (retired instead
//     while a graph is live on the device), so a new stream that gets the
//     same handle starts empty.
//
// Backend interface (all return 0 on success or a nonzero status):
//   int alloc(int dev, size_t bytes, void** out);
//   int release(int dev, void* p);
//   int sync(int dev);                              whole device
//   int sync_stream(int dev, const void* stream);   one stream's queued work
// Not thread-safe by itself; the caller holds a lock.
#pragma once

#include <stddef.h>

#include <map>
#include <unordered_map>
#include <utility>
#include <vector>

namespace seera {

template <class Backend>
class WorkspacePool {
public:
    static constexpr int kGrowUnderCapture = -1;
    static constexpr size_t kRound = (size_t)1 << 20;

    explicit WorkspacePool(Backend& b) : b_(b) {}

    // Returns a buffer of at least `bytes` for (dev, stream) in *out.
    int get(int dev, const void* stream, size_t bytes, bool capturing, void** out) {
        *out = nullptr;
        Buf& s = bufs_[{dev, stream}];
        if (bytes > s.bytes) {
            if (capturing) return kGrowUnderCapture;
            if (s.ptr) {
                if (live_graphs_[dev] > 0) {
                    retired_[dev].push_back(s.ptr);
                } else {
                    if (int e = b_.sync_stream(dev, stream)) return e;
                    if (int e = b_.release(dev, s.ptr)) return e;
                }
                s.ptr = nullptr;
                s.bytes = 0;
            }
            const size_t want = (bytes + kRound - 1) / kRound * kRound;
            if (int e = b_.alloc(dev, want, &s.ptr)) {
                s.ptr = nullptr;
                return e;
            }
            s.bytes = want;
        }
        *out = s.ptr;
        return 0;
    }

    // The stream is being destroyed (or its owner gives its workspace back):
    // the workspace is freed after the stream's queued work, or retired while
    // a graph on the device may reference it.
    int stream_destroyed(int dev, const void* stream) {
        auto it = bufs_.find({dev, stream});
        if (it == bufs_.end()) return 0;
        void* p = it->second.ptr;
        bufs_.erase(it);
        if (!p) return 0;
        if (live_graphs_[dev] > 0) {
            retired_[dev].push_back(p);
            return 0;
        }
        if (int e = b_.sync_stream(dev, stream)) {
            retired_[dev].push_back(p);  // freed with the device's graphs, or never
            return e;
        }
        return b_.release(dev, p);
    }

    void graph_created(const void* exec, int dev) {
        graph_dev_[exec] = dev;
        ++live_graphs_[dev];
    }

    // Frees the device's retired buffers once its last live graph is gone.
    int graph_destroyed(const void* exec) {
        auto it = graph_dev_.find(exec);
        if (it == graph_dev_.end()) return 0;
        const int dev = it->second;
        graph_dev_.erase(it);
        if (--live_graphs_[dev] > 0) return 0;
        std::vector<void*>& r = retired_[dev];
        if (r.empty()) return 0;
        if (int e = b_.sync(dev)) return e;  // a replay may still be running
        while (!r.empty()) {
            if (int e = b_.release(dev, r.back())) return e;
            r.pop_back();
        }
        return 0;
    }

    size_t held_bytes() const {
        size_t h = 0;
        for (auto& kv : bufs_) h += kv.second.bytes;
        return h;
    }
    size_t retired_count() const {
        size_t n = 0;
        for (auto& kv : retired_) n += kv.second.size();
        return n;
    }
    int live_graphs(int dev) const {
        auto it = live_graphs_.find(dev);
        return it == live_graphs_.end() ? 0 : it->second;
    }

private:
    struct Buf {
        void* ptr = nullptr;
        size_t bytes = 0;
    };
    Backend& b_;
    std::map<std::pair<int, const void*>, Buf> bufs_;
    std::map<int, std::vector<void*>> retired_;
    std::map<int, int> live_graphs_;
    std::unordered_map<const void*, int> graph_dev_;
};

}  // namespace seera
