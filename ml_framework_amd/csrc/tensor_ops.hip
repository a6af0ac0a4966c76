// tensor_ops.hip -- the reference GPU engine's element-wise, activation,
// softmax, broadcast, unpooling and reduction functions: the seera_cuda names
// around the GEMM / convolution path that cuTen.py and Seera_Engine.py call
// on every layer (bias add, activation, softmax head, bias gradient).
//
// Semantics follow the reference kernels operation for operation:
//   activations.cu:9-85     x -> (out, local grad) pairs
//   activations.cu:87-161   softmax over rows [N, C] and its VJP
//   elemops.cu:14-40        C = A op B
//   cuTen_essentails.cu:8-58 in-place scalar multiply / add / power
//   broadcast.cu:12-153     4-D broadcast add / multiply
//   unpooling.cu:7-50       nearest-neighbour upsample and its backward
//   reductionKernels.cu     sum / mean / max / min / argmax / argmin along
//                           one axis and the backward of the first four
// Bit-level notes. Everything except the transcendental functions (exp, log,
// tanh, pow: device math library) and the softmax sums is exact IEEE fp32 in
// the reference's order: reductions add along the reduced axis in index order
// from +0, unpooling's backward adds its window row by row, division and
// square root are correctly rounded. The softmax row max / sum use a fixed
// butterfly order (deterministic, not the reference's shared-memory tree).
//
// Layout: element-wise kernels are grid-stride with 16-byte accesses when every
// pointer is 16-byte aligned (cuTen hands out offsets into concatenated
// buffers, cuTen.py:675-686, so alignment is checked per call); a reduction
// runs one thread per output, consecutive threads on consecutive inner
// positions so that the loads along the reduced axis coalesce.
#include <math.h>

#include <algorithm>

#include "kernels.h"
#include "runtime.h"

namespace seera {
namespace {

constexpr int kThreads = 256;

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

unsigned grid_for(int64_t work) {
    const int64_t b = (work + kThreads - 1) / kThreads;
    return (unsigned)std::max<int64_t>(1, std::min<int64_t>(b, 8192));
}

// ---- activations: out = f(x), grad = f'(x) (activations.cu:9-85) ----
struct ReluOp {
    __device__ void operator()(float v, float& o, float& g) const {
        o = v > 0.f ? v : 0.f;
        g = v > 0.f ? 1.f : 0.f;
    }
};
struct SigmoidOp {
    __device__ void operator()(float v, float& o, float& g) const {
        const float s = 1.f / (1.f + expf(-v));
        o = s;
        g = s * (1.f - s);
    }
};
struct TanhOp {
    __device__ void operator()(float v, float& o, float& g) const {
        const float t = tanhf(v);
        o = t;
        g = 1.f - t * t;
    }
};
struct LogOp {
    __device__ void operator()(float v, float& o, float& g) const {
        o = logf(v);
        g = 1.f / v;
    }
};
struct ExpOp {
    __device__ void operator()(float v, float& o, float& g) const {
        const float e = expf(v);
        o = e;
        g = e;
    }
};
struct AbsOp {
    __device__ void operator()(float v, float& o, float& g) const {
        o = fabsf(v);
        g = v > 0.f ? 1.f : (v < 0.f ? -1.f : 0.f);
    }
};
struct SqrtOp {
    __device__ void operator()(float v, float& o, float& g) const {
        const float s = sqrtf(v);
        o = s;
        g = 0.5f / (s + 1e-12f);
    }
};
struct PowOp {
    float e;
    __device__ void operator()(float v, float& o, float& g) const {
        o = powf(v, e);
        g = e * powf(v, e - 1.f);
    }
};
struct ClipOp {
    float lo, hi;
    __device__ void operator()(float v, float& o, float& g) const {
        o = fminf(fmaxf(v, lo), hi);
        g = (v >= lo && v <= hi) ? 1.f : 0.f;
    }
};

template <bool V4, class Op>
__global__ __launch_bounds__(kThreads) void act_kernel(const float* __restrict__ x,
                                                       float* __restrict__ out,
                                                       float* __restrict__ grad, int64_t n,
                                                       Op op) {
    const int64_t stride = (int64_t)gridDim.x * kThreads;
    const int64_t t = (int64_t)blockIdx.x * kThreads + threadIdx.x;
    int64_t done = 0;
    if constexpr (V4) {
        const int64_t n4 = n / 4;
        for (int64_t i = t; i < n4; i += stride) {
            const float4 v = reinterpret_cast<const float4*>(x)[i];
            float4 o, g;
            op(v.x, o.x, g.x);
            op(v.y, o.y, g.y);
            op(v.z, o.z, g.z);
            op(v.w, o.w, g.w);
            reinterpret_cast<float4*>(out)[i] = o;
            reinterpret_cast<float4*>(grad)[i] = g;
        }
        done = n4 * 4;
    }
    for (int64_t i = done + t; i < n; i += stride) op(x[i], out[i], grad[i]);
}

// ---- element-wise binary: C = A op B (elemops.cu:14-40) ----
struct AddOp {
    __device__ float operator()(float a, float b) const { return a + b; }
};
struct SubOp {
    __device__ float operator()(float a, float b) const { return a - b; }
};
struct MulOp {
    __device__ float operator()(float a, float b) const { return a * b; }
};
struct DivOp {
    __device__ float operator()(float a, float b) const { return a / b; }
};

template <bool V4, class Op>
__global__ __launch_bounds__(kThreads) void binary_kernel(const float* __restrict__ A,
                                                          const float* __restrict__ B,
                                                          float* __restrict__ C, int64_t n,
                                                          Op op) {
    const int64_t stride = (int64_t)gridDim.x * kThreads;
    const int64_t t = (int64_t)blockIdx.x * kThreads + threadIdx.x;
    int64_t done = 0;
    if constexpr (V4) {
        const int64_t n4 = n / 4;
        for (int64_t i = t; i < n4; i += stride) {
            const float4 a = reinterpret_cast<const float4*>(A)[i];
            const float4 b = reinterpret_cast<const float4*>(B)[i];
            reinterpret_cast<float4*>(C)[i] =
                make_float4(op(a.x, b.x), op(a.y, b.y), op(a.z, b.z), op(a.w, b.w));
        }
        done = n4 * 4;
    }
    for (int64_t i = done + t; i < n; i += stride) C[i] = op(A[i], B[i]);
}

// ---- in place with a scalar (cuTen_essentails.cu:8-58) ----
struct ScaleOp {
    float k;
    __device__ float operator()(float a) const { return a * k; }
};
struct ShiftOp {
    float k;
    __device__ float operator()(float a) const { return a + k; }
};
struct PowerOp {
    float k;
    __device__ float operator()(float a) const { return powf(a, k); }
};

template <bool V4, class Op>
__global__ __launch_bounds__(kThreads) void scalar_kernel(float* __restrict__ p, int64_t n,
                                                          Op op) {
    const int64_t stride = (int64_t)gridDim.x * kThreads;
    const int64_t t = (int64_t)blockIdx.x * kThreads + threadIdx.x;
    int64_t done = 0;
    if constexpr (V4) {
        const int64_t n4 = n / 4;
        for (int64_t i = t; i < n4; i += stride) {
            float4 a = reinterpret_cast<float4*>(p)[i];
            reinterpret_cast<float4*>(p)[i] = make_float4(op(a.x), op(a.y), op(a.z), op(a.w));
        }
        done = n4 * 4;
    }
    for (int64_t i = done + t; i < n; i += stride) p[i] = op(p[i]);
}

// ---- 4-D broadcast (broadcast.cu:12-64): output extent per axis is the
// non-1 extent of A or B; an operand's extent-1 axes are read at index 0 ----
struct Bcast {
    int oN, oC, oH, oW;
    int64_t as[4], bs[4];  // operand strides per output axis (0 on broadcast axes)
};

template <bool MUL>
__global__ __launch_bounds__(kThreads) void broadcast_kernel(const float* __restrict__ A,
                                                             const float* __restrict__ B,
                                                             float* __restrict__ C, Bcast g,
                                                             int64_t total) {
    const int64_t stride = (int64_t)gridDim.x * kThreads;
    for (int64_t t = (int64_t)blockIdx.x * kThreads + threadIdx.x; t < total; t += stride) {
        int64_t r = t;
        const int w = (int)(r % g.oW);
        r /= g.oW;
        const int h = (int)(r % g.oH);
        r /= g.oH;
        const int c = (int)(r % g.oC);
        const int n = (int)(r / g.oC);
        const float a = A[n * g.as[0] + c * g.as[1] + h * g.as[2] + w * g.as[3]];
        const float b = B[n * g.bs[0] + c * g.bs[1] + h * g.bs[2] + w * g.bs[3]];
        C[t] = MUL ? a * b : a + b;
    }
}

// ---- nearest-neighbour unpooling (unpooling.cu:7-50) ----
__global__ __launch_bounds__(kThreads) void unpool_fwd_kernel(const float* __restrict__ in,
                                                              float* __restrict__ out,
                                                              int64_t planes, int H, int W,
                                                              int sh, int sw) {
    const int Ho = H * sh, Wo = W * sw;
    const int64_t total = planes * Ho * Wo;
    const int64_t stride = (int64_t)gridDim.x * kThreads;
    for (int64_t t = (int64_t)blockIdx.x * kThreads + threadIdx.x; t < total; t += stride) {
        const int wo = (int)(t % Wo);
        const int64_t r = t / Wo;
        const int ho = (int)(r % Ho);
        const int64_t p = r / Ho;
        out[t] = in[(p * H + ho / sh) * W + wo / sw];
    }
}

// dx[h, w] = sum over the sh x sw block it was copied to, row by row from +0.
__global__ __launch_bounds__(kThreads) void unpool_bwd_kernel(const float* __restrict__ dout,
                                                              float* __restrict__ dx,
                                                              int64_t planes, int H, int W,
                                                              int sh, int sw) {
    const int Wo = W * sw;
    const int64_t total = planes * H * W;
    const int64_t stride = (int64_t)gridDim.x * kThreads;
    for (int64_t t = (int64_t)blockIdx.x * kThreads + threadIdx.x; t < total; t += stride) {
        const int w = (int)(t % W);
        const int64_t r = t / W;
        const int h = (int)(r % H);
        const int64_t p = r / H;
        const float* src = dout + (p * H * sh + (int64_t)h * sh) * Wo + (int64_t)w * sw;
        float s = 0.f;
        for (int i = 0; i < sh; ++i)
            for (int j = 0; j < sw; ++j) s += src[(int64_t)i * Wo + j];
        dx[t] = s;
    }
}

// ---- softmax over rows (activations.cu:87-161): one wave per row ----
__device__ float wave_max(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
    return v;
}
__device__ float wave_sum(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
    return v;
}

constexpr int kRowsPerBlock = kThreads / 64;

__global__ __launch_bounds__(kThreads) void softmax_kernel(const float* __restrict__ x,
                                                           float* __restrict__ out, int N,
                                                           int C) {
    const int row = blockIdx.x * kRowsPerBlock + (threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    if (row >= N) return;  // whole wave
    const float* xr = x + (int64_t)row * C;
    float* orow = out + (int64_t)row * C;
    float m = -INFINITY;
    for (int i = lane; i < C; i += 64) m = fmaxf(m, xr[i]);
    m = wave_max(m);
    float s = 0.f;
    for (int i = lane; i < C; i += 64) s += expf(xr[i] - m);
    const float inv = 1.f / wave_sum(s);
    for (int i = lane; i < C; i += 64) orow[i] = expf(xr[i] - m) * inv;
}

// dx = s * (dout - <s, dout>) per row.
__global__ __launch_bounds__(kThreads) void softmax_vjp_kernel(const float* __restrict__ s,
                                                               const float* __restrict__ d,
                                                               float* __restrict__ dx, int N,
                                                               int C) {
    const int row = blockIdx.x * kRowsPerBlock + (threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    if (row >= N) return;
    const int64_t o = (int64_t)row * C;
    float dot = 0.f;
    for (int i = lane; i < C; i += 64) dot += s[o + i] * d[o + i];
    dot = wave_sum(dot);
    for (int i = lane; i < C; i += 64) dx[o + i] = s[o + i] * (d[o + i] - dot);
}

// ---- reductions along one axis (reductionKernels.cu) ----
// Output t = (outer, inner); the reduced elements sit at
// base + i * stride, base = outer * limit + inner, i < len.
struct Axis {
    int64_t outputs, stride, limit;
    int len;
};

template <int KIND>  // 0 sum (divided by div), 1 max, 2 min
__global__ __launch_bounds__(kThreads) void reduce_kernel(const float* __restrict__ A,
                                                          float* __restrict__ out, Axis a,
                                                          float div) {
    const int64_t t = (int64_t)blockIdx.x * kThreads + threadIdx.x;
    if (t >= a.outputs) return;
    const int64_t base = (t / a.stride) * a.limit + t % a.stride;
    float acc = 0.f;
    if constexpr (KIND != 0) acc = A[base];  // max / min start at the first element
    for (int i = 0; i < a.len; ++i) {
        const float v = A[base + i * a.stride];
        if constexpr (KIND == 0) acc += v;
        else if constexpr (KIND == 1) acc = fmaxf(acc, v);
        else acc = fminf(acc, v);
    }
    out[t] = KIND == 0 ? acc / div : acc;
}

// Index of the last element >= (argmax) or <= (argmin) every earlier one.
template <bool MAX>
__global__ __launch_bounds__(kThreads) void arg_kernel(const float* __restrict__ A,
                                                       int* __restrict__ out, Axis a) {
    const int64_t t = (int64_t)blockIdx.x * kThreads + threadIdx.x;
    if (t >= a.outputs) return;
    const int64_t base = (t / a.stride) * a.limit + t % a.stride;
    float best = A[base];
    int arg = 0;
    for (int i = 0; i < a.len; ++i) {
        const float v = A[base + i * a.stride];
        if (MAX ? v >= best : v <= best) {
            best = v;
            arg = i;
        }
    }
    out[t] = arg;
}

// dA along the axis = dOut / div (sum, mean).
__global__ __launch_bounds__(kThreads) void reduce_bwd_kernel(const float* __restrict__ dOut,
                                                              float* __restrict__ dA, Axis a,
                                                              float div) {
    const int64_t t = (int64_t)blockIdx.x * kThreads + threadIdx.x;
    if (t >= a.outputs) return;
    const int64_t base = (t / a.stride) * a.limit + t % a.stride;
    const float g = dOut[t] / div;
    for (int i = 0; i < a.len; ++i) dA[base + i * a.stride] = g;
}

// dA = dOut at the first element equal to the forward output, 0 elsewhere.
__global__ __launch_bounds__(kThreads) void select_bwd_kernel(const float* __restrict__ dOut,
                                                              const float* __restrict__ X,
                                                              const float* __restrict__ Y,
                                                              float* __restrict__ dA, Axis a) {
    const int64_t t = (int64_t)blockIdx.x * kThreads + threadIdx.x;
    if (t >= a.outputs) return;
    const int64_t base = (t / a.stride) * a.limit + t % a.stride;
    const float y = Y[t], g = dOut[t];
    bool found = false;
    for (int i = 0; i < a.len; ++i) {
        const int64_t k = base + i * a.stride;
        const bool hit = !found && X[k] == y;
        dA[k] = hit ? g : 0.f;
        found = found || hit;
    }
}

// Launches the 16-byte (k4) or the scalar (k1) variant of a grid-stride
// element-wise kernel over n elements.
template <class... P, class... A>
int launch_map(int64_t n, bool v4, hipStream_t st, void (*k4)(P...), void (*k1)(P...),
               A... args) {
    if (n == 0) return SEERA_OK;
    const unsigned g = grid_for(v4 ? (n + 3) / 4 : n);
    hipLaunchKernelGGL(v4 ? k4 : k1, dim3(g), dim3(kThreads), 0, st, args...);
    SEERA_HIP_TRY(hipGetLastError());
    return SEERA_OK;
}
#define SEERA_MAP(K, OP, ...) launch_map(n, v4, st, K<true, OP>, K<false, OP>, __VA_ARGS__)

}  // namespace

int activation_fwd(int kind, const float* x, float* out, float* grad, int64_t n, float p0,
                   float p1, hipStream_t st) {
    const bool v4 = aligned16(x) && aligned16(out) && aligned16(grad);
    switch (kind) {
        case kActFwdRelu: return SEERA_MAP(act_kernel, ReluOp, x, out, grad, n, ReluOp{});
        case kActFwdSigmoid:
            return SEERA_MAP(act_kernel, SigmoidOp, x, out, grad, n, SigmoidOp{});
        case kActFwdTanh: return SEERA_MAP(act_kernel, TanhOp, x, out, grad, n, TanhOp{});
        case kActFwdLog: return SEERA_MAP(act_kernel, LogOp, x, out, grad, n, LogOp{});
        case kActFwdExp: return SEERA_MAP(act_kernel, ExpOp, x, out, grad, n, ExpOp{});
        case kActFwdAbs: return SEERA_MAP(act_kernel, AbsOp, x, out, grad, n, AbsOp{});
        case kActFwdSqrt: return SEERA_MAP(act_kernel, SqrtOp, x, out, grad, n, SqrtOp{});
        case kActFwdPow:
            return SEERA_MAP(act_kernel, PowOp, x, out, grad, n, PowOp{p0});
        case kActFwdClip:
            return SEERA_MAP(act_kernel, ClipOp, x, out, grad, n, ClipOp{p0, p1});
        default: return fail(SEERA_ERR_INVALID_ARGUMENT, "unknown activation kind %d", kind);
    }
}

int elementwise(int op, const float* A, const float* B, float* C, int64_t n, hipStream_t st) {
    const bool v4 = aligned16(A) && aligned16(B) && aligned16(C);
    switch (op) {
        case kElemAdd: return SEERA_MAP(binary_kernel, AddOp, A, B, C, n, AddOp{});
        case kElemSub: return SEERA_MAP(binary_kernel, SubOp, A, B, C, n, SubOp{});
        case kElemMul: return SEERA_MAP(binary_kernel, MulOp, A, B, C, n, MulOp{});
        case kElemDiv: return SEERA_MAP(binary_kernel, DivOp, A, B, C, n, DivOp{});
        default: return fail(SEERA_ERR_INVALID_ARGUMENT, "unknown element-wise op %d", op);
    }
}

int scalar_inplace(int op, float* p, float k, int64_t n, hipStream_t st) {
    const bool v4 = aligned16(p);
    switch (op) {
        case kScalarMul: return SEERA_MAP(scalar_kernel, ScaleOp, p, n, ScaleOp{k});
        case kScalarAdd: return SEERA_MAP(scalar_kernel, ShiftOp, p, n, ShiftOp{k});
        case kScalarPow: return SEERA_MAP(scalar_kernel, PowerOp, p, n, PowerOp{k});
        default: return fail(SEERA_ERR_INVALID_ARGUMENT, "unknown scalar op %d", op);
    }
}

int broadcast_4d(bool mul, const float* A, const float* B, float* C, const int a[4],
                 const int b[4], hipStream_t st) {
    int o[4];
    for (int i = 0; i < 4; ++i) {
        if (a[i] < 0 || b[i] < 0)
            return fail(SEERA_ERR_INVALID_ARGUMENT, "broadcast: negative extent");
        if (a[i] == b[i] || b[i] == 1) o[i] = a[i];
        else if (a[i] == 1) o[i] = b[i];
        else
            return fail(SEERA_ERR_INVALID_ARGUMENT,
                        "broadcast: shapes (%d,%d,%d,%d) and (%d,%d,%d,%d) do not broadcast",
                        a[0], a[1], a[2], a[3], b[0], b[1], b[2], b[3]);
    }
    const int64_t total = (int64_t)o[0] * o[1] * o[2] * o[3];
    if (total == 0) return SEERA_OK;
    if (!A || !B || !C) return fail(SEERA_ERR_INVALID_ARGUMENT, "null device pointer");
    Bcast g;
    g.oN = o[0]; g.oC = o[1]; g.oH = o[2]; g.oW = o[3];
    const int64_t ast[4] = {(int64_t)a[1] * a[2] * a[3], (int64_t)a[2] * a[3], a[3], 1};
    const int64_t bst[4] = {(int64_t)b[1] * b[2] * b[3], (int64_t)b[2] * b[3], b[3], 1};
    for (int i = 0; i < 4; ++i) {
        g.as[i] = a[i] == 1 ? 0 : ast[i];
        g.bs[i] = b[i] == 1 ? 0 : bst[i];
    }
    if (mul)
        hipLaunchKernelGGL(broadcast_kernel<true>, dim3(grid_for(total)), dim3(kThreads), 0, st,
                           A, B, C, g, total);
    else
        hipLaunchKernelGGL(broadcast_kernel<false>, dim3(grid_for(total)), dim3(kThreads), 0, st,
                           A, B, C, g, total);
    SEERA_HIP_TRY(hipGetLastError());
    return SEERA_OK;
}

int unpool(bool backward, const float* src, float* dst, int B, int C, int H, int W, int sh,
           int sw, hipStream_t st) {
    const int64_t planes = (int64_t)B * C;
    const int64_t total = backward ? planes * H * W : planes * H * sh * W * sw;
    if (total == 0) return SEERA_OK;
    if (backward)
        hipLaunchKernelGGL(unpool_bwd_kernel, dim3(grid_for(total)), dim3(kThreads), 0, st, src,
                           dst, planes, H, W, sh, sw);
    else
        hipLaunchKernelGGL(unpool_fwd_kernel, dim3(grid_for(total)), dim3(kThreads), 0, st, src,
                           dst, planes, H, W, sh, sw);
    SEERA_HIP_TRY(hipGetLastError());
    return SEERA_OK;
}

int softmax(bool vjp, const float* a, const float* b, float* out, int N, int C, hipStream_t st) {
    if (N == 0 || C == 0) return SEERA_OK;
    const dim3 grid((unsigned)((N + kRowsPerBlock - 1) / kRowsPerBlock));
    if (vjp)
        hipLaunchKernelGGL(softmax_vjp_kernel, grid, dim3(kThreads), 0, st, a, b, out, N, C);
    else
        hipLaunchKernelGGL(softmax_kernel, grid, dim3(kThreads), 0, st, a, out, N, C);
    SEERA_HIP_TRY(hipGetLastError());
    return SEERA_OK;
}

int reduce_axis(int kind, const float* A, const float* Y, const float* dOut, void* out, int ndims,
                int dim, const int* dims, hipStream_t st) {
    if (ndims < 1 || ndims > 64 || dim < 0 || dim >= ndims)
        return fail(SEERA_ERR_INVALID_ARGUMENT, "reduction: dim %d of %d axes", dim, ndims);
    if (!dims) return fail(SEERA_ERR_INVALID_ARGUMENT, "reduction: null extents");
    Axis a{1, 1, 1, dims[dim]};
    for (int i = 0; i < ndims; ++i) {
        if (dims[i] < 0) return fail(SEERA_ERR_INVALID_ARGUMENT, "reduction: negative extent");
        if (i != dim) a.outputs *= dims[i];
        if (i > dim) a.stride *= dims[i];
        if (a.outputs > (int64_t)1 << 40 || a.stride > (int64_t)1 << 40)
            return fail(SEERA_ERR_INVALID_ARGUMENT, "reduction: tensor too large");
    }
    a.limit = a.stride * a.len;
    if (a.outputs == 0) return SEERA_OK;
    const bool need_input = kind != kRedSumBwd && kind != kRedMeanBwd;
    if (!out || (a.len > 0 && need_input && !A) ||
        ((kind == kRedSumBwd || kind == kRedMeanBwd || kind == kRedMaxBwd || kind == kRedMinBwd) &&
         !dOut) ||
        ((kind == kRedMaxBwd || kind == kRedMinBwd) && !Y))
        return fail(SEERA_ERR_INVALID_ARGUMENT, "null device pointer");
    // The reference reads the first element of an empty axis for max / min /
    // argmax / argmin (out of bounds); refuse instead.
    if (a.len == 0 && (kind == kRedMax || kind == kRedMin || kind == kRedArgmax ||
                       kind == kRedArgmin))
        return fail(SEERA_ERR_INVALID_ARGUMENT, "reduction: max/min over an empty axis");
    const dim3 grid((unsigned)((a.outputs + kThreads - 1) / kThreads)), blk(kThreads);
    if (grid.x > 0x7fffffffu) return fail(SEERA_ERR_INVALID_ARGUMENT, "reduction: grid too large");
    const float len = (float)a.len;
    float* o = static_cast<float*>(out);
    switch (kind) {
        case kRedSum: hipLaunchKernelGGL(reduce_kernel<0>, grid, blk, 0, st, A, o, a, 1.f); break;
        case kRedMean: hipLaunchKernelGGL(reduce_kernel<0>, grid, blk, 0, st, A, o, a, len); break;
        case kRedMax: hipLaunchKernelGGL(reduce_kernel<1>, grid, blk, 0, st, A, o, a, 0.f); break;
        case kRedMin: hipLaunchKernelGGL(reduce_kernel<2>, grid, blk, 0, st, A, o, a, 0.f); break;
        case kRedArgmax:
            hipLaunchKernelGGL(arg_kernel<true>, grid, blk, 0, st, A, static_cast<int*>(out), a);
            break;
        case kRedArgmin:
            hipLaunchKernelGGL(arg_kernel<false>, grid, blk, 0, st, A, static_cast<int*>(out), a);
            break;
        case kRedSumBwd:
            hipLaunchKernelGGL(reduce_bwd_kernel, grid, blk, 0, st, dOut, o, a, 1.f);
            break;
        case kRedMeanBwd:
            hipLaunchKernelGGL(reduce_bwd_kernel, grid, blk, 0, st, dOut, o, a, len);
            break;
        case kRedMaxBwd:
        case kRedMinBwd:
            hipLaunchKernelGGL(select_bwd_kernel, grid, blk, 0, st, dOut, A, Y, o, a);
            break;
        default: return fail(SEERA_ERR_INVALID_ARGUMENT, "unknown reduction kind %d", kind);
    }
    SEERA_HIP_TRY(hipGetLastError());
    return SEERA_OK;
}

}  // namespace seera
