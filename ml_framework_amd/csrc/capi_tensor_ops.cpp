// capi_tensor_ops.cpp -- the extern "C" entry points of include/seera_hip.h
// for the reference's element-wise, activation, softmax, broadcast,
// unpooling and reduction functions (tensor_ops.hip). Each validates its
// arguments, enqueues on the null stream and synchronizes before returning,
// so the result is ready when the call returns, as in the reference
// wrappers.
#include <limits.h>

#include "kernels.h"
#include "runtime.h"

using namespace seera;

namespace {

// Returned by a call that found nothing to do: no work was queued, so there
// is nothing to wait for.
constexpr int kNoWork = -1;

int done(int status) {
    if (status == kNoWork) return SEERA_OK;
    if (status != SEERA_OK) return status;
    SEERA_HIP_TRY(hipDeviceSynchronize());
    note_device_synchronized();
    return SEERA_OK;
}

template <class F>
int guarded(F&& f) {
    clear_error();
    return done(f());
}

int need(bool cond, const char* what) {
    return cond ? (int)SEERA_OK : fail(SEERA_ERR_INVALID_ARGUMENT, "%s", what);
}

int act(int kind, const float* x, float* out, float* grad, int size, float p0 = 0.f,
        float p1 = 0.f) {
    return guarded([&] {
        SEERA_TRY(need(size >= 0, "activation: size must be >= 0"));
        if (size == 0) return kNoWork;
        SEERA_TRY(need(x && out && grad, "activation: null device pointer"));
        return activation_fwd(kind, x, out, grad, size, p0, p1, nullptr);
    });
}

int elem(int op, const float* A, const float* B, float* C, int size) {
    return guarded([&] {
        SEERA_TRY(need(size >= 0, "element-wise: size must be >= 0"));
        if (size == 0) return kNoWork;
        SEERA_TRY(need(A && B && C, "element-wise: null device pointer"));
        return elementwise(op, A, B, C, size, nullptr);
    });
}

int scal(int op, float* p, float k, int n) {
    return guarded([&] {
        SEERA_TRY(need(n >= 0, "scalar op: total_elements must be >= 0"));
        if (n == 0) return kNoWork;
        SEERA_TRY(need(p != nullptr, "scalar op: null device pointer"));
        return scalar_inplace(op, p, k, n, nullptr);
    });
}

int unpool_call(bool bwd, const float* src, float* dst, int B, int C, int H, int W, int sh,
                int sw) {
    return guarded([&] {
        SEERA_TRY(need(B >= 0 && C >= 0 && H >= 0 && W >= 0, "unpooling: negative extent"));
        SEERA_TRY(need(sh >= 1 && sw >= 1, "unpooling: scale factors must be >= 1"));
        SEERA_TRY(need((int64_t)H * sh <= INT_MAX && (int64_t)W * sw <= INT_MAX,
                       "unpooling: output extent exceeds int range"));
        if ((int64_t)B * C * H * W == 0) return kNoWork;
        SEERA_TRY(need(src && dst, "unpooling: null device pointer"));
        return unpool(bwd, src, dst, B, C, H, W, sh, sw, nullptr);
    });
}

int softmax_call(bool vjp, const float* a, const float* b, float* out, int N, int C) {
    return guarded([&] {
        SEERA_TRY(need(N >= 0 && C >= 0, "softmax: N and C must be >= 0"));
        if ((int64_t)N * C == 0) return kNoWork;
        SEERA_TRY(need(a && out && (!vjp || b), "softmax: null device pointer"));
        return softmax(vjp, a, b, out, N, C, nullptr);
    });
}

int red(int kind, const float* A, const float* Y, const float* dOut, void* out, int ndims,
        int dim, const int* dims) {
    return guarded([&] { return reduce_axis(kind, A, Y, dOut, out, ndims, dim, dims, nullptr); });
}

int bcast(bool mul, const float* A, const float* B, float* C, int aN, int aC, int aH, int aW,
          int bN, int bC, int bH, int bW) {
    return guarded([&] {
        const int a[4] = {aN, aC, aH, aW}, b[4] = {bN, bC, bH, bW};
        return broadcast_4d(mul, A, B, C, a, b, nullptr);
    });
}

}  // namespace

extern "C" {

int seera_hip_relu_fwd(const float* x, float* out, float* grad, int size) {
    return act(kActFwdRelu, x, out, grad, size);
}
int seera_hip_sigmoid_fwd(const float* x, float* out, float* grad, int size) {
    return act(kActFwdSigmoid, x, out, grad, size);
}
int seera_hip_tanh_fwd(const float* x, float* out, float* grad, int size) {
    return act(kActFwdTanh, x, out, grad, size);
}
int seera_hip_log_fwd(const float* x, float* out, float* grad, int size) {
    return act(kActFwdLog, x, out, grad, size);
}
int seera_hip_exp_fwd(const float* x, float* out, float* grad, int size) {
    return act(kActFwdExp, x, out, grad, size);
}
int seera_hip_abs_fwd(const float* x, float* out, float* grad, int size) {
    return act(kActFwdAbs, x, out, grad, size);
}
int seera_hip_sqrt_fwd(const float* x, float* out, float* grad, int size) {
    return act(kActFwdSqrt, x, out, grad, size);
}
int seera_hip_pow_fwd(const float* x, float exponent, float* out, float* grad, int size) {
    return act(kActFwdPow, x, out, grad, size, exponent);
}
int seera_hip_clip_fwd(const float* x, float lo, float hi, float* out, float* grad, int size) {
    return act(kActFwdClip, x, out, grad, size, lo, hi);
}

int seera_hip_softmax_fwd(const float* x, float* out, int N, int C) {
    return softmax_call(false, x, nullptr, out, N, C);
}
int seera_hip_softmax_vjp(const float* s, const float* dout, float* dx, int N, int C) {
    return softmax_call(true, s, dout, dx, N, C);
}

int seera_hip_unpooling_fwd(const float* inp, float* out, int batchN, int C, int H, int W, int sh,
                            int sw) {
    return unpool_call(false, inp, out, batchN, C, H, W, sh, sw);
}
int seera_hip_unpooling_bwd(const float* dout, float* dx, int batchN, int C, int H, int W, int sh,
                            int sw) {
    return unpool_call(true, dout, dx, batchN, C, H, W, sh, sw);
}

int seera_hip_sum_fwd(const float* A, float* out, int ndims, int dim, const int* dimarr) {
    return red(kRedSum, A, nullptr, nullptr, out, ndims, dim, dimarr);
}
int seera_hip_mean_fwd(const float* A, float* out, int ndims, int dim, const int* dimarr) {
    return red(kRedMean, A, nullptr, nullptr, out, ndims, dim, dimarr);
}
int seera_hip_max_fwd(const float* A, float* out, int ndims, int dim, const int* dimarr) {
    return red(kRedMax, A, nullptr, nullptr, out, ndims, dim, dimarr);
}
int seera_hip_min_fwd(const float* A, float* out, int ndims, int dim, const int* dimarr) {
    return red(kRedMin, A, nullptr, nullptr, out, ndims, dim, dimarr);
}
int seera_hip_argmax_fwd(const float* A, int* out, int ndims, int dim, const int* dimarr) {
    return red(kRedArgmax, A, nullptr, nullptr, out, ndims, dim, dimarr);
}
int seera_hip_argmin_fwd(const float* A, int* out, int ndims, int dim, const int* dimarr) {
    return red(kRedArgmin, A, nullptr, nullptr, out, ndims, dim, dimarr);
}
int seera_hip_sum_bwd(const float* dOut, float* dA, int ndims, int dim, const int* dimarr) {
    return red(kRedSumBwd, nullptr, nullptr, dOut, dA, ndims, dim, dimarr);
}
int seera_hip_mean_bwd(const float* dOut, float* dA, int ndims, int dim, const int* dimarr) {
    return red(kRedMeanBwd, nullptr, nullptr, dOut, dA, ndims, dim, dimarr);
}
int seera_hip_max_bwd(const float* dOut, const float* fwdInput, const float* fwdOutput, float* dA,
                      int ndims, int dim, const int* dimarr) {
    return red(kRedMaxBwd, fwdInput, fwdOutput, dOut, dA, ndims, dim, dimarr);
}
int seera_hip_min_bwd(const float* dOut, const float* fwdInput, const float* fwdOutput, float* dA,
                      int ndims, int dim, const int* dimarr) {
    return red(kRedMinBwd, fwdInput, fwdOutput, dOut, dA, ndims, dim, dimarr);
}

int seera_hip_scaler_multiply_f(float* arr, float k, int total_elements) {
    return scal(kScalarMul, arr, k, total_elements);
}
int seera_hip_scaler_add_f(float* arr, float k, int total_elements) {
    return scal(kScalarAdd, arr, k, total_elements);
}
int seera_hip_power_of(float* arr, float k, int total_elements) {
    return scal(kScalarPow, arr, k, total_elements);
}

int seera_hip_elemadd(const float* A, const float* B, float* C, int size) {
    return elem(kElemAdd, A, B, C, size);
}
int seera_hip_elemsub(const float* A, const float* B, float* C, int size) {
    return elem(kElemSub, A, B, C, size);
}
int seera_hip_elemdiv(const float* A, const float* B, float* C, int size) {
    return elem(kElemDiv, A, B, C, size);
}
int seera_hip_elemmult(const float* A, const float* B, float* C, int size) {
    return elem(kElemMul, A, B, C, size);
}

int seera_hip_broadcast_add_4d(const float* A, const float* B, float* C, int aN, int aC, int aH,
                               int aW, int bN, int bC, int bH, int bW) {
    return bcast(false, A, B, C, aN, aC, aH, aW, bN, bC, bH, bW);
}
int seera_hip_broadcast_mul_4d(const float* A, const float* B, float* C, int aN, int aC, int aH,
                               int aW, int bN, int bC, int bH, int bW) {
    return bcast(true, A, B, C, aN, aC, aH, aW, bN, bC, bH, bW);
}

}  // extern "C"
