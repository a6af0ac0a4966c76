// Host-only test of the workspace bookkeeping (ml_framework_amd/csrc/
// workspace_pool.h) with a fake backend: "device memory" is host memory and
// every allocation, release and synchronize is recorded. Built and run by
// tests/test_workspace_pool.py with g++; exits nonzero on the first failure.
#include <stdio.h>
#include <stdlib.h>

#include <set>
#include <vector>

#include "workspace_pool.h"

namespace {

int g_failures = 0;
#define CHECK(cond)                                                         \
    do {                                                                    \
        if (!(cond)) {                                                      \
            fprintf(stderr, "%s:%d: check failed: %s\n", __FILE__, __LINE__, #cond); \
            ++g_failures;                                                   \
        }                                                                   \
    } while (0)

struct FakeBackend {
    std::set<void*> live;
    int allocs = 0, releases = 0, syncs = 0;
    std::vector<const void*> stream_syncs;  // streams synchronized one by one
    bool fail_next_alloc = false;
    ~FakeBackend() {
        for (void* p : live) free(p);  // the pool keeps its buffers until exit
    }
    int alloc(int, size_t bytes, void** out) {
        if (fail_next_alloc) {
            fail_next_alloc = false;
            return 3;  // out of memory
        }
        *out = malloc(bytes);
        live.insert(*out);
        ++allocs;
        return 0;
    }
    int release(int, void* p) {
        if (!live.count(p)) return 7;  // double free / unknown pointer
        live.erase(p);
        free(p);
        ++releases;
        return 0;
    }
    int sync(int) {
        ++syncs;
        return 0;
    }
    int sync_stream(int, const void* stream) {
        stream_syncs.push_back(stream);
        return 0;
    }
};

using Pool = seera::WorkspacePool<FakeBackend>;
const void* const kS1 = (const void*)0x10;
const void* const kS2 = (const void*)0x20;
const void* const kG1 = (const void*)0x100;
const void* const kG2 = (const void*)0x200;
constexpr size_t MiB = (size_t)1 << 20;

void per_stream_buffers() {
    FakeBackend b;
    Pool pool(b);
    void *p1 = nullptr, *p2 = nullptr, *p1b = nullptr;
    CHECK(pool.get(0, kS1, 100, false, &p1) == 0);
    CHECK(pool.get(0, kS2, 100, false, &p2) == 0);
    CHECK(p1 && p2 && p1 != p2);              // two streams never share
    CHECK(pool.get(0, kS1, MiB, false, &p1b) == 0);
    CHECK(p1b == p1);                          // rounded up to 1 MiB: no regrowth
    CHECK(pool.held_bytes() == 2 * MiB);
    void* p3 = nullptr;
    CHECK(pool.get(1, kS1, 100, false, &p3) == 0);
    CHECK(p3 != p1);                           // per device too
}

void growth_without_graphs_frees() {
    FakeBackend b;
    Pool pool(b);
    void *p = nullptr, *q = nullptr;
    CHECK(pool.get(0, kS1, 10, false, &p) == 0);
    CHECK(pool.get(0, kS1, 3 * MiB, false, &q) == 0);
    CHECK(q != nullptr);
    CHECK(!b.live.count(p));                   // old buffer released
    CHECK(b.stream_syncs.size() == 1 && b.stream_syncs[0] == kS1);  // after its stream's work
    CHECK(b.syncs == 0);                       // no device-wide synchronize
    CHECK(pool.retired_count() == 0);
    CHECK(pool.held_bytes() == 3 * MiB);
}

void growth_with_live_graph_retires() {
    FakeBackend b;
    Pool pool(b);
    void *p = nullptr, *q = nullptr, *r = nullptr;
    CHECK(pool.get(0, kS1, 10, false, &p) == 0);
    pool.graph_created(kG1, 0);                // captured with p
    pool.graph_created(kG2, 0);
    CHECK(pool.get(0, kS1, 2 * MiB + 1, false, &q) == 0);
    CHECK(b.live.count(p));                    // a replay still writes to p
    CHECK(b.syncs == 0 && b.stream_syncs.empty());  // retiring waits for nothing
    CHECK(pool.retired_count() == 1);
    CHECK(pool.get(0, kS1, 5 * MiB, false, &r) == 0);
    CHECK(b.live.count(q) && pool.retired_count() == 2);
    CHECK(pool.graph_destroyed(kG1) == 0);
    CHECK(b.live.count(p) && b.live.count(q)); // kG2 still live
    const int syncs = b.syncs;
    CHECK(pool.graph_destroyed(kG2) == 0);
    CHECK(!b.live.count(p) && !b.live.count(q));
    CHECK(b.syncs == syncs + 1);               // synchronized before the frees
    CHECK(b.live.count(r));                    // the current buffer stays
    CHECK(pool.retired_count() == 0);
    CHECK(pool.graph_destroyed(kG2) == 0);     // unknown graph: no-op
    CHECK(pool.live_graphs(0) == 0);
}

void graph_on_other_device_does_not_pin() {
    FakeBackend b;
    Pool pool(b);
    void *p = nullptr, *q = nullptr;
    pool.graph_created(kG1, 1);
    CHECK(pool.get(0, kS1, 10, false, &p) == 0);
    CHECK(pool.get(0, kS1, 2 * MiB, false, &q) == 0);
    CHECK(!b.live.count(p) && pool.retired_count() == 0);
}

void capture_refuses_growth() {
    FakeBackend b;
    Pool pool(b);
    void *p = nullptr, *q = nullptr;
    CHECK(pool.get(0, kS1, MiB, false, &p) == 0);
    const int allocs = b.allocs;
    CHECK(pool.get(0, kS1, MiB, true, &q) == 0 && q == p);   // fits: fine under capture
    CHECK(pool.get(0, kS1, MiB + 1, true, &q) == Pool::kGrowUnderCapture);
    CHECK(q == nullptr && b.allocs == allocs && b.live.count(p));
    CHECK(pool.get(0, kS2, 1, true, &q) == Pool::kGrowUnderCapture);  // first use too
}

void failed_alloc_leaves_clean_state() {
    FakeBackend b;
    Pool pool(b);
    void *p = nullptr, *q = nullptr;
    CHECK(pool.get(0, kS1, 10, false, &p) == 0);
    b.fail_next_alloc = true;
    CHECK(pool.get(0, kS1, 4 * MiB, false, &q) == 3);
    CHECK(q == nullptr && pool.held_bytes() == 0 && b.live.empty());
    CHECK(pool.get(0, kS1, 4 * MiB, false, &q) == 0 && q != nullptr);
    CHECK(pool.held_bytes() == 4 * MiB);
}

void stream_destroy_frees_or_retires() {
    FakeBackend b;
    Pool pool(b);
    void *p = nullptr, *q = nullptr, *r = nullptr;
    CHECK(pool.get(0, kS1, 3 * MiB, false, &p) == 0);
    CHECK(pool.stream_destroyed(0, kS1) == 0);
    CHECK(!b.live.count(p) && pool.held_bytes() == 0);
    CHECK(b.syncs == 0 && b.stream_syncs.size() == 1 && b.stream_syncs[0] == kS1);
    CHECK(pool.get(0, kS1, 10, false, &q) == 0);   // a new stream, same handle: fresh
    CHECK(pool.held_bytes() == MiB);
    pool.graph_created(kG1, 0);
    CHECK(pool.stream_destroyed(0, kS1) == 0);
    CHECK(b.live.count(q) && pool.retired_count() == 1);  // the graph may use it
    CHECK(pool.stream_destroyed(0, kS2) == 0);            // never used: no-op
    CHECK(pool.graph_destroyed(kG1) == 0);
    CHECK(!b.live.count(q) && pool.retired_count() == 0);
    CHECK(pool.get(0, kS2, 10, false, &r) == 0 && r != nullptr);
}

void growth_syncs_only_its_stream() {
    FakeBackend b;
    Pool pool(b);
    void *p1 = nullptr, *p2 = nullptr, *q = nullptr;
    CHECK(pool.get(0, kS1, 10, false, &p1) == 0);
    CHECK(pool.get(0, kS2, 10, false, &p2) == 0);
    CHECK(pool.get(0, kS2, 4 * MiB, false, &q) == 0);    // S2 grows
    CHECK(b.live.count(p1) && !b.live.count(p2));       // S1's buffer untouched
    CHECK(b.stream_syncs.size() == 1 && b.stream_syncs[0] == kS2);
    CHECK(b.syncs == 0);
}

}  // namespace

int main() {
    per_stream_buffers();
    growth_without_graphs_frees();
    growth_with_live_graph_retires();
    graph_on_other_device_does_not_pin();
    capture_refuses_growth();
    failed_alloc_leaves_clean_state();
    stream_destroy_frees_or_retires();
    growth_syncs_only_its_stream();
    if (g_failures) {
        fprintf(stderr, "%d check(s) failed\n", g_failures);
        return 1;
    }
    printf("workspace pool: all checks passed\n");
    return 0;
}
