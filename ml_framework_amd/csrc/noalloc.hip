// noalloc.hip -- seera_hip_matmul_noalloc: the GEMM forward for callers that
// cannot allocate device memory (code under HIP graph capture, serving
// loops, harnesses that forbid hipMalloc).
//
// The only device memory the GEMM needs beyond its inputs and output is the
// split-K partial sums (plan.h run_plan). Here they go to `scratch`, a fixed
// array of kNoAllocScratchBytes that the code object carries: the runtime
// places one copy on each GPU the library runs on, kept until the process
// ends. Its device address is taken once per device with hipGetSymbolAddress
// (the array's name in host code is not a device address) and handed to the
// kernels through a FixedWorkspace, exactly as the allocating entry point
// hands them its workspace. Nothing is allocated or freed per call.
//
// The split-K partials of a call are written in full before they are read,
// so the array needs no clearing. Every call on a GPU shares that GPU's
// array: calls that overlap on one GPU (queued on two streams, or from two
// host threads) race on it.
#include <mutex>

#include "kernels.h"
#include "runtime.h"

namespace seera {

// The planner (plan.h) splits K only for the 64x64 tile and only when there
// are fewer than 128 tiles, each split over at most ceil(256 / tiles) parts
// (and more than kMaxGroupSplits: fewer run as wave groups in the block):
// at most 382 partial tiles of 64 x 64 fp32, 6.3 MB. 8 MiB covers every shape;
// a request above it (a future plan) fails cleanly in workspace().
constexpr size_t kNoAllocScratchBytes = (size_t)8 << 20;

static __device__ __align__(256) float scratch[kNoAllocScratchBytes / sizeof(float)];

namespace {
constexpr int kMaxDevices = 64;
std::mutex g_mu;
void* g_scratch_ptr[kMaxDevices] = {};

// The device address of the current device's copy of `scratch`.
int scratch_address(void** out) {
    int dev = 0;
    SEERA_HIP_TRY(hipGetDevice(&dev));
    if (dev < 0 || dev >= kMaxDevices)
        return fail(SEERA_ERR_HIP, "device id %d out of range", dev);
    std::lock_guard<std::mutex> lock(g_mu);
    if (!g_scratch_ptr[dev]) {
        void* p = nullptr;
        SEERA_HIP_TRY(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)));
        if (!p) return fail(SEERA_ERR_HIP, "hipGetSymbolAddress returned no address");
        g_scratch_ptr[dev] = p;
    }
    *out = g_scratch_ptr[dev];
    return SEERA_OK;
}
}  // namespace

}  // namespace seera

extern "C" int seera_hip_matmul_noalloc(const float* A, const float* B, float* C, int M, int N,
                                        int K, int Nbatch, void* stream) {
    using namespace seera;
    clear_error();
    if (M < 0 || N < 0 || K < 0 || Nbatch < 0)
        return fail(SEERA_ERR_INVALID_ARGUMENT,
                    "matmul dims must be >= 0 (M=%d N=%d K=%d Nbatch=%d)", M, N, K, Nbatch);
    const bool work = (int64_t)M * N * Nbatch > 0;
    if (work && (!C || (K > 0 && (!A || !B))))
        return fail(SEERA_ERR_INVALID_ARGUMENT, "null device pointer");
    void* p = nullptr;
    SEERA_TRY(scratch_address(&p));
    FixedWorkspace fixed(p, kNoAllocScratchBytes, "seera_hip_matmul_noalloc");
    const int st = gemm_fwd(A, B, C, M, N, K, Nbatch, reinterpret_cast<hipStream_t>(stream));
    if (st == SEERA_OK) note_async_work();
    return st;
}
