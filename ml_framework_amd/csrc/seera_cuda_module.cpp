// seera_cuda_module.cpp -- the `seera_cuda` Python module: the reference's
// function names and signatures (engine_cuda/src/cuda_bindings.cpp:14-533)
// over the C ABI of include/seera_hip.h. Device pointers cross as Python ints
// (uintptr_t), dims as C ints, exactly as cuTen.py and Seera_Engine.py pass
// them. A failing call raises RuntimeError (the reference ignores errors).
//
// Host-only translation unit: no HIP headers, no GPU code.
#include <pybind11/numpy.h>
#include <pybind11/pybind11.h>
#include <pybind11/stl.h>
#include <stdint.h>

#include <algorithm>
#include <stdexcept>
#include <string>
#include <vector>

#include "seera_hip.h"

namespace py = pybind11;

using arr_f = py::array_t<float, py::array::c_style | py::array::forcecast>;
using arr_i = py::array_t<int32_t, py::array::c_style | py::array::forcecast>;
using arr_s = py::array_t<int16_t, py::array::c_style | py::array::forcecast>;

namespace {

void check(int status) {
    if (status != SEERA_OK)
        throw std::runtime_error(std::string("seera_cuda: ") + seera_hip_last_error());
}

template <class T>
T* dev(uintptr_t p) {
    return reinterpret_cast<T*>(p);
}

uintptr_t alloc_bytes(size_t n) {
    void* p = nullptr;
    check(seera_hip_malloc(&p, n));
    return reinterpret_cast<uintptr_t>(p);
}

std::vector<ssize_t> dims_of(const py::tuple& shape, size_t* count) {
    std::vector<ssize_t> dims;
    size_t n = 1;
    for (auto s : shape) {
        const ssize_t d = s.cast<ssize_t>();
        if (d < 0) throw std::invalid_argument("seera_cuda: negative extent in shape");
        dims.push_back(d);
        n *= (size_t)d;
    }
    *count = n;
    return dims;
}

template <class T, class Arr>
uintptr_t upload(const Arr& a) {
    const size_t bytes = (size_t)a.size() * sizeof(T);
    const uintptr_t p = alloc_bytes(bytes);
    check(seera_hip_memcpy_h2d(dev<void>(p), a.data(), bytes));
    return p;
}

template <class T>
py::array_t<T> download(uintptr_t ptr, const py::tuple& shape) {
    size_t n = 0;
    std::vector<ssize_t> dims = dims_of(shape, &n);
    py::array_t<T> out(dims);
    check(seera_hip_memcpy_d2h(out.mutable_data(), dev<const void>(ptr), n * sizeof(T)));
    return out;
}

}  // namespace

PYBIND11_MODULE(seera_cuda, m) {
    m.doc() = "Seera GEMM/conv hot path on MI355X (gfx950): fp16 MFMA, fp32 accumulate";

    // ---- memory management (cuda_bindings.cpp:23-66) ----
    m.def("cuda_malloc", [](size_t n_bytes) { return alloc_bytes(n_bytes); },
          "Allocate n bytes on the GPU, returns the device address");
    m.def("cuda_malloc_f16", [](int n) { return alloc_bytes((size_t)n * sizeof(float)); },
          "Allocate n float elements (the reference stores fp32 here too)");
    m.def("cuda_malloc_f32", [](int n) { return alloc_bytes((size_t)n * sizeof(float)); },
          "Allocate n float32 elements on the GPU");
    m.def("cuda_malloc_i32", [](int n) { return alloc_bytes((size_t)n * sizeof(int32_t)); },
          "Allocate n int32 elements on the GPU");
    m.def("cuda_malloc_i16", [](int n) { return alloc_bytes((size_t)n * sizeof(int16_t)); },
          "Allocate n int16 elements on the GPU");
    m.def("cuda_free", [](uintptr_t p) { check(seera_hip_free(dev<void>(p))); },
          "Free GPU memory");
    m.def("cuda_memcopy_devicetodevice",
          [](uintptr_t dst, uintptr_t src, int num_elem) {
              check(seera_hip_memcpy_d2d(dev<void>(dst), dev<const void>(src),
                                         (size_t)num_elem * sizeof(float)));
          },
          "Copy num_elem floats from ptr2 to ptr1 on the GPU");
    m.def("cuda_memset",
          [](uintptr_t p, int value, size_t n_bytes) {
              check(seera_hip_memset(dev<void>(p), value, n_bytes));
          },
          "Memset GPU memory");
    // cuda_bindings.cpp:467-477: allocate total_elements floats and fill them.
    m.def("cuda_ones_f",
          [](int total_elements) {
              const uintptr_t p = alloc_bytes((size_t)std::max(total_elements, 0) * sizeof(float));
              check(seera_hip_fill_f32(dev<float>(p), 1.f, (size_t)std::max(total_elements, 0)));
              return p;
          },
          "Allocate total_elements floats filled with 1 (GPU ptr)");
    m.def("cuda_zeros_f",
          [](int total_elements) {
              const uintptr_t p = alloc_bytes((size_t)std::max(total_elements, 0) * sizeof(float));
              check(seera_hip_fill_f32(dev<float>(p), 0.f, (size_t)std::max(total_elements, 0)));
              return p;
          },
          "Allocate total_elements floats filled with 0 (GPU ptr)");
    // cuda_bindings.cpp:338-351 (mask: int32 [batchN, C, H, W], as cuTen.py:592 allocates it).
    m.def("cuda_maxpool_fwd",
          [](uintptr_t image, uintptr_t out, uintptr_t mask, int batchN, int C, int H, int W,
             int R, int S, int pad_h, int pad_w, int stride_h, int stride_w) {
              check(seera_hip_maxpool_fwd(dev<const float>(image), dev<float>(out), dev<int>(mask),
                                          batchN, C, H, W, R, S, pad_h, pad_w, stride_h, stride_w));
          },
          "MaxPool2D forward (GPU ptrs, mask int32 [N, C, H, W])");
    m.def("cuda_maxpool_bwd",
          [](uintptr_t dout, uintptr_t mask, uintptr_t dX, int batchN, int C, int H, int W, int R,
             int S, int pad_h, int pad_w, int stride_h, int stride_w) {
              check(seera_hip_maxpool_bwd(dev<const float>(dout), dev<const int>(mask),
                                          dev<float>(dX), batchN, C, H, W, R, S, pad_h, pad_w,
                                          stride_h, stride_w));
          },
          "MaxPool2D backward (GPU ptrs)");
    // Not in the reference: the fused layer entry points of the C ABI (bias,
    // ReLU and its mask in the GEMM / convolution store; the ReLU backward in
    // the dA store; fixed-order bias gradients). Pointers as above; mask and
    // bias may be 0 (none). act: 0 none, 1 ReLU.
    m.def("cuda_matmul_bias_act",
          [](uintptr_t A, uintptr_t B, uintptr_t bias, uintptr_t C, uintptr_t mask, int M, int N,
             int K, int Nbatch, int act) {
              check(seera_hip_matmul_bias_act(dev<const float>(A), dev<const float>(B),
                                              dev<const float>(bias), dev<float>(C),
                                              dev<float>(mask), M, N, K, Nbatch, act));
          },
          "C = act(A @ B + bias); ReLU mask into mask (GPU ptrs)");
    m.def("cuda_matmul_bwd_relu",
          [](uintptr_t A, uintptr_t B, uintptr_t dC, uintptr_t mask, uintptr_t dA, uintptr_t dB,
             int M, int N, int K, int Nbatch) {
              check(seera_hip_matmul_bwd_relu(dev<const float>(A), dev<const float>(B),
                                              dev<const float>(dC), dev<const float>(mask),
                                              dev<float>(dA), dev<float>(dB), M, N, K, Nbatch));
          },
          "dA = (dC @ B^T) * mask, dB = A^T @ dC (GPU ptrs)");
    m.def("cuda_matmul_bwd_bias",
          [](uintptr_t A, uintptr_t B, uintptr_t dC, uintptr_t dA, uintptr_t dB, uintptr_t db, int M,
             int N, int K, int Nbatch) {
              check(seera_hip_matmul_bwd_bias(dev<const float>(A), dev<const float>(B),
                                              dev<const float>(dC), dev<float>(dA), dev<float>(dB),
                                              dev<float>(db), M, N, K, Nbatch));
          },
          "dA = dC @ B^T, dB = A^T @ dC and db = column sums of dC from the dB GEMM (GPU ptrs)");
    m.def("cuda_matmul_bwd_relu_bias",
          [](uintptr_t A, uintptr_t B, uintptr_t dC, uintptr_t mask, uintptr_t dA, uintptr_t dB,
             uintptr_t db, int M, int N, int K, int Nbatch) {
              check(seera_hip_matmul_bwd_relu_bias(dev<const float>(A), dev<const float>(B),
                                                   dev<const float>(dC), dev<const float>(mask),
                                                   dev<float>(dA), dev<float>(dB), dev<float>(db), M,
                                                   N, K, Nbatch));
          },
          "cuda_matmul_bwd_relu and db = column sums of dC from the dB GEMM (GPU ptrs)");
    m.def("cuda_bias_grad",
          [](uintptr_t dY, uintptr_t db, int rows, int N) {
              check(seera_hip_bias_grad(dev<const float>(dY), dev<float>(db), rows, N));
          },
          "db[n] = sum over rows of dY[rows, N] (GPU ptrs)");
    m.def("cuda_conv2d_fwd_bias_act",
          [](uintptr_t image, uintptr_t kernel, uintptr_t bias, uintptr_t conv, uintptr_t mask,
             int batchN, int C, int H, int W, int N, int R, int S, int pad_h, int pad_w,
             int stride_h, int stride_w, int act) {
              check(seera_hip_conv2d_fwd_bias_act(
                  dev<const float>(image), dev<const float>(kernel), dev<const float>(bias),
                  dev<float>(conv), dev<float>(mask), batchN, C, H, W, N, R, S, pad_h, pad_w,
                  stride_h, stride_w, act));
          },
          "conv = act(conv2d(image, kernel) + bias[n]) (GPU ptrs, pad before stride)");
    m.def("cuda_conv2d_bwd_bias",
          [](uintptr_t W, uintptr_t X, uintptr_t dY, uintptr_t dX, uintptr_t dW, uintptr_t db,
             int batch, int C, int H, int W_in, int N, int R, int S, int strideh, int stridew,
             int padh, int padw) {
              check(seera_hip_conv2d_bwd_bias(dev<const float>(W), dev<const float>(X),
                                              dev<const float>(dY), dev<float>(dX),
                                              dev<float>(dW), dev<float>(db), batch, C, H, W_in,
                                              N, R, S, strideh, stridew, padh, padw));
          },
          "cuda_conv2d_bwd plus db = sum of dY per channel from the same pass (GPU ptrs)");
    m.def("cuda_conv_bias_grad",
          [](uintptr_t dY, uintptr_t db, int batchN, int N, int HW) {
              check(seera_hip_conv_bias_grad(dev<const float>(dY), dev<float>(db), batchN, N, HW));
          },
          "db[n] = sum over images and pixels of dY[batchN, N, HW] (GPU ptrs)");
    // Not in the reference: the caching allocator behind cuda_malloc / cuda_free.
    m.def("cuda_empty_cache", []() { check(seera_hip_empty_cache()); },
          "Return the allocator's cached blocks to HIP");
    m.def("cuda_memory_stats",
          []() {
              size_t live = 0, cached = 0;
              check(seera_hip_memory_stats(&live, &cached));
              return py::make_tuple(live, cached);
          },
          "(bytes in live allocations, bytes cached for reuse)");

    // ---- activations (cuda_bindings.cpp:176-239): x -> out, grad ----
#define SEERA_ACT(name, fn, doc)                                                          \
    m.def(name,                                                                           \
          [](uintptr_t x, uintptr_t out, uintptr_t grad, int size) {                     \
              check(fn(dev<const float>(x), dev<float>(out), dev<float>(grad), size));   \
          },                                                                              \
          doc)
    SEERA_ACT("cuda_relu_fwd", seera_hip_relu_fwd, "ReLU forward: x -> out, grad (GPU ptrs)");
    SEERA_ACT("cuda_sigmoid_fwd", seera_hip_sigmoid_fwd, "Sigmoid forward (GPU ptrs)");
    SEERA_ACT("cuda_tanh_fwd", seera_hip_tanh_fwd, "Tanh forward (GPU ptrs)");
    SEERA_ACT("cuda_log_fwd", seera_hip_log_fwd, "Log forward (GPU ptrs)");
    SEERA_ACT("cuda_exp_fwd", seera_hip_exp_fwd, "Exp forward (GPU ptrs)");
    SEERA_ACT("cuda_abs_fwd", seera_hip_abs_fwd, "Abs forward (GPU ptrs)");
    SEERA_ACT("cuda_sqrt_fwd", seera_hip_sqrt_fwd, "Sqrt forward (GPU ptrs)");
#undef SEERA_ACT
    m.def("cuda_pow_fwd",
          [](uintptr_t x, float exponent, uintptr_t out, uintptr_t grad, int size) {
              check(seera_hip_pow_fwd(dev<const float>(x), exponent, dev<float>(out),
                                      dev<float>(grad), size));
          },
          "Pow forward (GPU ptrs)");
    m.def("cuda_clip_fwd",
          [](uintptr_t x, float lo, float hi, uintptr_t out, uintptr_t grad, int size) {
              check(seera_hip_clip_fwd(dev<const float>(x), lo, hi, dev<float>(out),
                                       dev<float>(grad), size));
          },
          "Clip forward (GPU ptrs)");

    // ---- softmax (cuda_bindings.cpp:243-253) ----
    m.def("cuda_softmax_fwd",
          [](uintptr_t x, uintptr_t out, int N, int C) {
              check(seera_hip_softmax_fwd(dev<const float>(x), dev<float>(out), N, C));
          },
          "Softmax forward: x[N,C] -> out[N,C] (GPU ptrs)");
    m.def("cuda_softmax_vjp",
          [](uintptr_t s, uintptr_t dout, uintptr_t dx, int N, int C) {
              check(seera_hip_softmax_vjp(dev<const float>(s), dev<const float>(dout),
                                          dev<float>(dx), N, C));
          },
          "Softmax VJP backward (GPU ptrs)");

    // ---- unpooling (cuda_bindings.cpp:358-370) ----
    m.def("cuda_unpooling_fwd",
          [](uintptr_t inp, uintptr_t out, int batchN, int C, int H, int W, int sh, int sw) {
              check(seera_hip_unpooling_fwd(dev<const float>(inp), dev<float>(out), batchN, C, H,
                                            W, sh, sw));
          },
          "Unpooling (nearest upsample) forward (GPU ptrs)");
    m.def("cuda_unpooling_bwd",
          [](uintptr_t dout, uintptr_t dx, int batchN, int C, int H, int W, int sh, int sw) {
              check(seera_hip_unpooling_bwd(dev<const float>(dout), dev<float>(dx), batchN, C, H,
                                            W, sh, sw));
          },
          "Unpooling backward (GPU ptrs)");

    // ---- reductions (cuda_bindings.cpp:376-457); dimarr is a host int32
    // array with ndims entries ----
    auto dims_ok = [](const arr_i& d, int ndims) {
        if (ndims < 0 || d.size() < ndims)
            throw std::invalid_argument("seera_cuda: dimarr holds fewer than ndims extents");
        return d.data();
    };
#define SEERA_RED(name, fn, T, doc)                                                        \
    m.def(name,                                                                            \
          [dims_ok](uintptr_t A, uintptr_t out, int ndims, int dim, arr_i dimarr) {        \
              check(fn(dev<const float>(A), dev<T>(out), ndims, dim, dims_ok(dimarr, ndims))); \
          },                                                                               \
          doc)
    SEERA_RED("cuda_sum_fwd", seera_hip_sum_fwd, float,
              "Sum reduction forward (A, out: GPU ptrs; dimarr: numpy)");
    SEERA_RED("cuda_mean_fwd", seera_hip_mean_fwd, float,
              "Mean reduction forward (A, out: GPU ptrs; dimarr: numpy)");
    SEERA_RED("cuda_max_fwd", seera_hip_max_fwd, float,
              "Max reduction forward (A, out: GPU ptrs; dimarr: numpy)");
    SEERA_RED("cuda_min_fwd", seera_hip_min_fwd, float,
              "Min reduction forward (A, out: GPU ptrs; dimarr: numpy)");
    SEERA_RED("cuda_argmax_fwd", seera_hip_argmax_fwd, int,
              "Argmax reduction forward (A: float GPU, out: int GPU; dimarr: numpy)");
    SEERA_RED("cuda_argmin_fwd", seera_hip_argmin_fwd, int,
              "Argmin reduction forward (A: float GPU, out: int GPU; dimarr: numpy)");
    SEERA_RED("cuda_sum_bwd", seera_hip_sum_bwd, float,
              "Sum reduction backward (GPU ptrs; dimarr: numpy)");
    SEERA_RED("cuda_mean_bwd", seera_hip_mean_bwd, float,
              "Mean reduction backward (GPU ptrs; dimarr: numpy)");
#undef SEERA_RED
    m.def("cuda_max_bwd",
          [dims_ok](uintptr_t dOut, uintptr_t fwdInput, uintptr_t fwdOutput, uintptr_t dA,
                    int ndims, int dim, arr_i dimarr) {
              check(seera_hip_max_bwd(dev<const float>(dOut), dev<const float>(fwdInput),
                                      dev<const float>(fwdOutput), dev<float>(dA), ndims, dim,
                                      dims_ok(dimarr, ndims)));
          },
          "Max reduction backward (GPU ptrs; dimarr: numpy)");
    m.def("cuda_min_bwd",
          [dims_ok](uintptr_t dOut, uintptr_t fwdInput, uintptr_t fwdOutput, uintptr_t dA,
                    int ndims, int dim, arr_i dimarr) {
              check(seera_hip_min_bwd(dev<const float>(dOut), dev<const float>(fwdInput),
                                      dev<const float>(fwdOutput), dev<float>(dA), ndims, dim,
                                      dims_ok(dimarr, ndims)));
          },
          "Min reduction backward (GPU ptrs; dimarr: numpy)");

    // ---- scalar ops (cuda_bindings.cpp:461-465, 479-481), in place ----
    m.def("cuda_scaler_multiply_f",
          [](uintptr_t arr, float k, int total_elements) {
              check(seera_hip_scaler_multiply_f(dev<float>(arr), k, total_elements));
          },
          "Scalar multiply float (GPU ptr)");
    m.def("cuda_scaler_add_f",
          [](uintptr_t arr, float k, int total_elements) {
              check(seera_hip_scaler_add_f(dev<float>(arr), k, total_elements));
          },
          "Scalar add float (GPU ptr)");
    m.def("cuda_power_of",
          [](uintptr_t arr, float k, int total_elements) {
              check(seera_hip_power_of(dev<float>(arr), k, total_elements));
          },
          "Element-wise power arr = arr ** k (GPU ptr)");

    // ---- element-wise (cuda_bindings.cpp:486-512) ----
#define SEERA_ELEM(name, fn, doc)                                                     \
    m.def(name,                                                                       \
          [](uintptr_t A, uintptr_t B, uintptr_t C, int size) {                      \
              check(fn(dev<const float>(A), dev<const float>(B), dev<float>(C), size)); \
          },                                                                          \
          doc)
    SEERA_ELEM("cuda_elemadd", seera_hip_elemadd, "Elementwise add (float)");
    SEERA_ELEM("cuda_elemsub", seera_hip_elemsub, "Elementwise sub (float)");
    SEERA_ELEM("cuda_elemdiv", seera_hip_elemdiv, "Elementwise div (float)");
    SEERA_ELEM("cuda_elemmult", seera_hip_elemmult, "Elementwise mul (float)");
#undef SEERA_ELEM

    // ---- 4-D broadcast (cuda_bindings.cpp:518-532) ----
    m.def("broadcast_add_4d",
          [](uintptr_t A, uintptr_t B, uintptr_t C, int aN, int aC, int aH, int aW, int bN,
             int bC, int bH, int bW) {
              check(seera_hip_broadcast_add_4d(dev<const float>(A), dev<const float>(B),
                                               dev<float>(C), aN, aC, aH, aW, bN, bC, bH, bW));
          },
          "Broadcast add 4D (GPU ptrs)");
    m.def("broadcast_mul_4d",
          [](uintptr_t A, uintptr_t B, uintptr_t C, int aN, int aC, int aH, int aW, int bN,
             int bC, int bH, int bW) {
              check(seera_hip_broadcast_mul_4d(dev<const float>(A), dev<const float>(B),
                                               dev<float>(C), aN, aC, aH, aW, bN, bC, bH, bW));
          },
          "Broadcast mul 4D (GPU ptrs)");

    // ---- transfers (cuda_bindings.cpp:73-170) ----
    m.def("to_device_f16", [](arr_f a) { return upload<float>(a); },
          "Upload float32 numpy -> float32 GPU buffer (reference name)");
    m.def("to_host_f16", [](uintptr_t p, py::tuple s) { return download<float>(p, s); },
          "Download float32 GPU buffer -> numpy with shape (reference name)");
    m.def("to_device_f32", [](arr_f a) { return upload<float>(a); },
          "Upload float32 numpy -> float32 GPU buffer");
    m.def("to_host_f32", [](uintptr_t p, py::tuple s) { return download<float>(p, s); },
          "Download float32 GPU buffer -> numpy with shape");
    m.def("to_host_i32", [](uintptr_t p, py::tuple s) { return download<int32_t>(p, s); },
          "Download int32 GPU buffer -> numpy with shape");
    m.def("to_host_i16", [](uintptr_t p, py::tuple s) { return download<int16_t>(p, s); },
          "Download int16 GPU buffer -> numpy with shape");
    m.def("to_device_i16", [](arr_s a) { return upload<int16_t>(a); },
          "Upload int16 numpy -> GPU buffer");
    m.def("to_device_i32", [](arr_i a) { return upload<int32_t>(a); },
          "Upload int32 numpy -> GPU buffer");

    // ---- matmul (cuda_bindings.cpp:260-287) ----
    m.def("cuda_matmul",
          [](uintptr_t A, uintptr_t B, uintptr_t C, int M, int N, int K, int Nbatch) {
              check(seera_hip_matmul(dev<const float>(A), dev<const float>(B), dev<float>(C), M,
                                     N, K, Nbatch));
          },
          "Matmul: C[Nbatch,M,N] = A[Nbatch,M,K] @ B[K,N] (GPU ptrs)");
    m.def("cuda_matmul_bwd",
          [](uintptr_t A, uintptr_t B, uintptr_t dC, uintptr_t dA, uintptr_t dB, int M, int N,
             int K, int Nbatch) {
              check(seera_hip_matmul_bwd(dev<const float>(A), dev<const float>(B),
                                         dev<const float>(dC), dev<float>(dA), dev<float>(dB), M,
                                         N, K, Nbatch));
          },
          "Matmul backward: dA = dC @ B^T, dB = sum_b A_b^T @ dC_b (GPU ptrs)");
    m.def("cuda_transpose_2d",
          [](uintptr_t in, uintptr_t out, int rows, int cols) {
              check(seera_hip_transpose_2d(dev<const float>(in), dev<float>(out), rows, cols));
          },
          "Transpose 2D: in[rows,cols] -> out[cols,rows] (GPU ptrs)");
    m.def("cuda_transpose_3d",
          [](uintptr_t in, uintptr_t out, int Nbatch, int M, int K) {
              check(seera_hip_transpose_3d(dev<const float>(in), dev<float>(out), Nbatch, M, K));
          },
          "Transpose 3D batched: in[Nbatch,M,K] -> out[Nbatch,K,M] (GPU ptrs)");

    // ---- Conv2D (cuda_bindings.cpp:294-309) ----
    m.def("cuda_conv2d_fwd",
          [](uintptr_t image, uintptr_t kernel, uintptr_t conv, int batchN, int C, int H, int W,
             int N, int R, int S, int pad_h, int pad_w, int stride_h, int stride_w) {
              check(seera_hip_conv2d_fwd(dev<const float>(image), dev<const float>(kernel),
                                         dev<float>(conv), batchN, C, H, W, N, R, S, pad_h, pad_w,
                                         stride_h, stride_w));
          },
          "Conv2D forward (GPU ptrs); note pad before stride");
    m.def("cuda_conv2d_bwd",
          [](uintptr_t W, uintptr_t X, uintptr_t dY, uintptr_t dX, uintptr_t dW, int batch, int C,
             int H, int W_in, int N, int R, int S, int strideh, int stridew, int padh, int padw) {
              check(seera_hip_conv2d_bwd(dev<const float>(W), dev<const float>(X),
                                         dev<const float>(dY), dev<float>(dX), dev<float>(dW),
                                         batch, C, H, W_in, N, R, S, strideh, stridew, padh,
                                         padw));
          },
          "Conv2D backward (GPU ptrs); note stride before pad");

    // ---- ConvTranspose2D (cuda_bindings.cpp:316-331) ----
    m.def("cuda_conv2DTranpose_fwd",
          [](uintptr_t X, uintptr_t W, uintptr_t out, int batch, int Cin, int Hin, int Win,
             int Cout, int KH, int KW, int strideh, int stridew, int padh, int padw) {
              check(seera_hip_conv2DTranpose_fwd(dev<const float>(X), dev<const float>(W),
                                                 dev<float>(out), batch, Cin, Hin, Win, Cout, KH,
                                                 KW, strideh, stridew, padh, padw));
          },
          "ConvTranspose2D forward (GPU ptrs)");
    m.def("cuda_conv2DTranspose_bwd",
          [](uintptr_t W, uintptr_t X, uintptr_t dY, uintptr_t dX, uintptr_t dW, int batch,
             int Cin, int Hin, int Win, int Cout, int KH, int KW, int strideh, int stridew,
             int padh, int padw) {
              check(seera_hip_conv2DTranspose_bwd(dev<const float>(W), dev<const float>(X),
                                                  dev<const float>(dY), dev<float>(dX),
                                                  dev<float>(dW), batch, Cin, Hin, Win, Cout, KH,
                                                  KW, strideh, stridew, padh, padw));
          },
          "ConvTranspose2D backward (GPU ptrs)");
}
