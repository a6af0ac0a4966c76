// memory.hip -- device fill for the allocate-and-fill entry points
// (cuda_ones_f / cuda_zeros_f, engine_cuda/src/cuda_bindings.cpp:467-477).
#include "kernels.h"
#include "runtime.h"

namespace seera {
namespace {

// Grid-stride fill; 16-byte stores over the aligned body, scalar stores for
// the head and tail.
__global__ __launch_bounds__(256) void fill_f32_kernel(float* __restrict__ p, float v, size_t n,
                                                       size_t head) {
    const size_t stride = (size_t)gridDim.x * blockDim.x;
    const size_t t = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (t < head) p[t] = v;
    const size_t body = (n - head) / 4;
    float4* q = reinterpret_cast<float4*>(p + head);
    const float4 v4 = make_float4(v, v, v, v);
    for (size_t i = t; i < body; i += stride) q[i] = v4;
    const size_t tail0 = head + body * 4;
    if (t < n - tail0) p[tail0 + t] = v;
}

}  // namespace

int fill_f32(float* p, float v, size_t n, hipStream_t st) {
    if (n == 0) return SEERA_OK;
    const size_t mis = (reinterpret_cast<uintptr_t>(p) >> 2) & 3;  // floats to the next 16 B
    const size_t head = mis == 0 ? 0 : (n < 4 - mis ? n : 4 - mis);
    const size_t body = (n - head) / 4;
    size_t blocks = (body + 255) / 256;
    if (blocks < 1) blocks = 1;
    if (blocks > 4096) blocks = 4096;
    hipLaunchKernelGGL(fill_f32_kernel, dim3((unsigned)blocks), dim3(256), 0, st, p, v, n, head);
    SEERA_HIP_TRY(hipGetLastError());
    return SEERA_OK;
}

}  // namespace seera
