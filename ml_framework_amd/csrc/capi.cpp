// capi.cpp -- the extern "C" boundary declared in include/seera_hip.h.
//
// Each hot-path entry validates its arguments (the reference validates none:
// engine_cuda/src/cuda_bindings.cpp passes everything straight through),
// enqueues the kernels and, in its synchronous form, waits for the device
// like every reference wrapper does (cudaDeviceSynchronize at GEMM.cu:102,
// convolution.cu:388, upsampling.cu:316, ...).
#include <limits.h>

#include "kernels.h"
#include "runtime.h"

namespace seera {
const char* last_error();
}

using namespace seera;

namespace {

hipStream_t as_stream(void* s) { return reinterpret_cast<hipStream_t>(s); }

int sync_after(int status) {
    if (status != SEERA_OK) return status;
    SEERA_HIP_TRY(hipDeviceSynchronize());
    note_device_synchronized();
    return SEERA_OK;
}
// *_async entry points: the enqueued work may still use its buffers after the
// call returns, so the next free synchronizes first.
int queued(int status) {
    if (status == SEERA_OK) note_async_work();
    return status;
}

bool nonneg(int a) { return a >= 0; }

int check_ptrs(bool need, const void* a, const void* b, const void* c, const void* d = (void*)1,
               const void* e = (void*)1) {
    if (need && (!a || !b || !c || !d || !e))
        return fail(SEERA_ERR_INVALID_ARGUMENT, "null device pointer");
    return SEERA_OK;
}

int64_t prod(int64_t a, int64_t b, int64_t c = 1, int64_t d = 1) { return a * b * c * d; }

// Output extent of a convolution: floor((in + 2 pad - k) / stride) + 1.
int conv_out(int in, int pad, int k, int stride) { return (in + 2 * pad - k) / stride + 1; }

int check_conv_geometry(int R, int S, int sh, int sw, int ph, int pw) {
    if (R < 1 || S < 1) return fail(SEERA_ERR_INVALID_ARGUMENT, "kernel extent must be >= 1");
    if (sh < 1 || sw < 1) return fail(SEERA_ERR_INVALID_ARGUMENT, "stride must be >= 1");
    if (ph < 0 || pw < 0) return fail(SEERA_ERR_INVALID_ARGUMENT, "padding must be >= 0");
    return SEERA_OK;
}

int matmul_impl(const float* A, const float* B, float* C, int M, int N, int K, int Nbatch,
                hipStream_t st) {
    if (!nonneg(M) || !nonneg(N) || !nonneg(K) || !nonneg(Nbatch))
        return fail(SEERA_ERR_INVALID_ARGUMENT, "matmul dims must be >= 0 (M=%d N=%d K=%d Nbatch=%d)",
                    M, N, K, Nbatch);
    const bool work = prod(M, N, Nbatch) > 0;
    SEERA_TRY(check_ptrs(work, C, work && K > 0 ? A : C, work && K > 0 ? B : C));
    return gemm_fwd(A, B, C, M, N, K, Nbatch, st);
}

int matmul_bias_act_impl(const float* A, const float* B, const float* bias, float* C, float* mask,
                         int M, int N, int K, int Nbatch, int act, hipStream_t st) {
    if (!nonneg(M) || !nonneg(N) || !nonneg(K) || !nonneg(Nbatch))
        return fail(SEERA_ERR_INVALID_ARGUMENT, "matmul dims must be >= 0 (M=%d N=%d K=%d Nbatch=%d)",
                    M, N, K, Nbatch);
    if (act != SEERA_ACT_NONE && act != SEERA_ACT_RELU)
        return fail(SEERA_ERR_INVALID_ARGUMENT, "unknown activation %d", act);
    const bool work = prod(M, N, Nbatch) > 0;
    SEERA_TRY(check_ptrs(work, C, work && K > 0 ? A : C, work && K > 0 ? B : C));
    return gemm_fwd_bias_act(A, B, bias, C, act == SEERA_ACT_RELU ? mask : nullptr, M, N, K,
                             Nbatch, act, st);
}
int bias_grad_impl(const float* dY, float* db, int rows, int N, hipStream_t st) {
    if (rows < 0 || N < 0) return fail(SEERA_ERR_INVALID_ARGUMENT, "bias_grad dims must be >= 0");
    SEERA_TRY(check_ptrs(N > 0, db, rows > 0 ? dY : db, db));
    return bias_grad(dY, db, rows, N, st);
}
int pool_dims(int B, int C, int H, int W, int R, int S, int ph, int pw, int sh, int sw) {
    SEERA_TRY(check_conv_geometry(R, S, sh, sw, ph, pw));
    if (B < 0 || C < 1 || H < 1 || W < 1)
        return fail(SEERA_ERR_INVALID_ARGUMENT, "maxpool: bad tensor dims");
    // Keeps h * sh + R and H + 2 * ph (and the W counterparts) inside int.
    constexpr int kMaxExtent = 1 << 20;
    if (H > kMaxExtent || W > kMaxExtent || R > kMaxExtent || S > kMaxExtent ||
        ph > kMaxExtent || pw > kMaxExtent || sh > kMaxExtent || sw > kMaxExtent)
        return fail(SEERA_ERR_INVALID_ARGUMENT, "maxpool: extent, pad or stride above 2^20");
    if (H + 2 * ph < R || W + 2 * pw < S)
        return fail(SEERA_ERR_INVALID_ARGUMENT, "maxpool: window larger than padded input");
    const int Ho = (H + 2 * ph - R) / sh + 1, Wo = (W + 2 * pw - S) / sw + 1;
    if (prod(B, C, H, W) > INT_MAX || prod(B, C, Ho, Wo) > INT_MAX)
        return fail(SEERA_ERR_INVALID_ARGUMENT, "maxpool: tensor exceeds int range");
    return SEERA_OK;
}
int maxpool_fwd_impl(const float* x, float* out, int* mask, int B, int C, int H, int W, int R,
                     int S, int ph, int pw, int sh, int sw, hipStream_t st) {
    SEERA_TRY(pool_dims(B, C, H, W, R, S, ph, pw, sh, sw));
    SEERA_TRY(check_ptrs(B > 0, x, out, mask));
    return maxpool_fwd(x, out, mask, B, C, H, W, R, S, ph, pw, sh, sw, st);
}
int maxpool_bwd_impl(const float* dout, const int* mask, float* dx, int B, int C, int H, int W,
                     int R, int S, int ph, int pw, int sh, int sw, hipStream_t st) {
    SEERA_TRY(pool_dims(B, C, H, W, R, S, ph, pw, sh, sw));
    SEERA_TRY(check_ptrs(B > 0, dout, mask, dx));
    return maxpool_bwd(dout, mask, dx, B, C, H, W, R, S, ph, pw, sh, sw, st);
}
int matmul_bwd_impl(const float* A, const float* B, const float* dC, float* dA, float* dB, int M,
                    int N, int K, int Nbatch, hipStream_t st) {
    if (!nonneg(M) || !nonneg(N) || !nonneg(K) || !nonneg(Nbatch))
        return fail(SEERA_ERR_INVALID_ARGUMENT, "matmul_bwd dims must be >= 0");
    if (prod(M, N, K, Nbatch) > 0 || prod(K, N) > 0)
        SEERA_TRY(check_ptrs(true, A, B, dC, dA, dB));
    return gemm_bwd(A, B, dC, dA, dB, M, N, K, Nbatch, st);
}
// mask: nullptr for seera_hip_matmul_bwd_bias (checked non-null by the ReLU entry).
int matmul_bwd_bias_impl(const float* A, const float* B, const float* dC, const float* mask,
                         float* dA, float* dB, float* db, int M, int N, int K, int Nbatch,
                         hipStream_t st) {
    if (!nonneg(M) || !nonneg(N) || !nonneg(K) || !nonneg(Nbatch))
        return fail(SEERA_ERR_INVALID_ARGUMENT, "matmul_bwd dims must be >= 0");
    if (prod(M, N, K, Nbatch) > 0 || prod(K, N) > 0)
        SEERA_TRY(check_ptrs(true, A, B, dC, dA, dB));
    if (N > 0) SEERA_TRY(check_ptrs(true, db, db, prod(M, Nbatch, N) > 0 ? dC : db));
    return gemm_bwd_bias(A, B, dC, mask, dA, dB, db, M, N, K, Nbatch, st);
}
int matmul_bwd_relu_bias_impl(const float* A, const float* B, const float* dC, const float* mask,
                              float* dA, float* dB, float* db, int M, int N, int K, int Nbatch,
                              hipStream_t st) {
    if (prod(M, K, Nbatch) > 0) SEERA_TRY(check_ptrs(true, mask, mask, mask));
    return matmul_bwd_bias_impl(A, B, dC, prod(M, K, Nbatch) > 0 ? mask : nullptr, dA, dB, db, M, N,
                                K, Nbatch, st);
}
int matmul_bwd_relu_impl(const float* A, const float* B, const float* dC, const float* mask,
                         float* dA, float* dB, int M, int N, int K, int Nbatch, hipStream_t st) {
    if (!nonneg(M) || !nonneg(N) || !nonneg(K) || !nonneg(Nbatch))
        return fail(SEERA_ERR_INVALID_ARGUMENT, "matmul_bwd dims must be >= 0");
    if (prod(M, N, K, Nbatch) > 0 || prod(K, N) > 0)
        SEERA_TRY(check_ptrs(true, A, B, dC, dA, dB));
    if (prod(M, K, Nbatch) > 0) SEERA_TRY(check_ptrs(true, mask, mask, mask));
    return gemm_bwd_relu(A, B, dC, mask, dA, dB, M, N, K, Nbatch, st);
}

int conv2d_fwd_impl(const float* image, const float* kernel, float* conv, int batchN, int C, int H,
                    int W, int N, int R, int S, int pad_h, int pad_w, int stride_h, int stride_w,
                    hipStream_t st) {
    SEERA_TRY(check_conv_geometry(R, S, stride_h, stride_w, pad_h, pad_w));
    if (batchN < 0 || C < 1 || H < 1 || W < 1 || N < 1)
        return fail(SEERA_ERR_INVALID_ARGUMENT, "conv2d_fwd: bad tensor dims");
    if (H + 2 * pad_h < R || W + 2 * pad_w < S)
        return fail(SEERA_ERR_INVALID_ARGUMENT, "conv2d_fwd: kernel larger than padded input");
    SEERA_TRY(check_ptrs(batchN > 0, image, kernel, conv));
    return conv_fwd(image, kernel, conv, batchN, C, H, W, N, R, S, stride_h, stride_w, pad_h, pad_w,
                    st);
}
int conv2d_fwd_bias_act_impl(const float* image, const float* kernel, const float* bias,
                             float* conv, float* mask, int batchN, int C, int H, int W, int N,
                             int R, int S, int pad_h, int pad_w, int stride_h, int stride_w,
                             int act, hipStream_t st) {
    SEERA_TRY(check_conv_geometry(R, S, stride_h, stride_w, pad_h, pad_w));
    if (batchN < 0 || C < 1 || H < 1 || W < 1 || N < 1)
        return fail(SEERA_ERR_INVALID_ARGUMENT, "conv2d_fwd: bad tensor dims");
    if (H + 2 * pad_h < R || W + 2 * pad_w < S)
        return fail(SEERA_ERR_INVALID_ARGUMENT, "conv2d_fwd: kernel larger than padded input");
    if (act != SEERA_ACT_NONE && act != SEERA_ACT_RELU)
        return fail(SEERA_ERR_INVALID_ARGUMENT, "unknown activation %d", act);
    SEERA_TRY(check_ptrs(batchN > 0, image, kernel, conv));
    return conv_fwd_bias_act(image, kernel, bias, conv, act == SEERA_ACT_RELU ? mask : nullptr,
                             batchN, C, H, W, N, R, S, stride_h, stride_w, pad_h, pad_w, act, st);
}
int conv_bias_grad_impl(const float* dY, float* db, int batchN, int N, int HW, hipStream_t st) {
    if (batchN < 0 || N < 0 || HW < 0)
        return fail(SEERA_ERR_INVALID_ARGUMENT, "conv_bias_grad dims must be >= 0");
    if (prod(batchN, N, HW) > INT64_C(1) << 40)
        return fail(SEERA_ERR_INVALID_ARGUMENT, "conv_bias_grad: tensor too large");
    SEERA_TRY(check_ptrs(N > 0, db, prod(batchN, N, HW) > 0 ? dY : db, db));
    return conv_bias_grad(dY, db, batchN, N, HW, st);
}

int conv2d_bwd_impl(const float* Wt, const float* X, const float* dY, float* dX, float* dW,
                    int batch, int C, int H, int W_in, int N, int R, int S, int strideh,
                    int stridew, int padh, int padw, hipStream_t st) {
    SEERA_TRY(check_conv_geometry(R, S, strideh, stridew, padh, padw));
    if (batch < 0 || C < 1 || H < 1 || W_in < 1 || N < 1)
        return fail(SEERA_ERR_INVALID_ARGUMENT, "conv2d_bwd: bad tensor dims");
    if (H + 2 * padh < R || W_in + 2 * padw < S)
        return fail(SEERA_ERR_INVALID_ARGUMENT, "conv2d_bwd: kernel larger than padded input");
    SEERA_TRY(check_ptrs(true, Wt, dW, batch > 0 ? X : dW, batch > 0 ? dY : dW,
                         batch > 0 ? dX : dW));
    return conv_bwd(dY, Wt, X, dX, dW, nullptr, batch, C, H, W_in, N, R, S, strideh, stridew, padh,
                    padw, st);
}

int conv2d_bwd_bias_impl(const float* Wt, const float* X, const float* dY, float* dX, float* dW,
                         float* db, int batch, int C, int H, int W_in, int N, int R, int S,
                         int strideh, int stridew, int padh, int padw, hipStream_t st) {
    if (!db) return fail(SEERA_ERR_INVALID_ARGUMENT, "null device pointer (db)");
    SEERA_TRY(check_conv_geometry(R, S, strideh, stridew, padh, padw));
    if (batch < 0 || C < 1 || H < 1 || W_in < 1 || N < 1)
        return fail(SEERA_ERR_INVALID_ARGUMENT, "conv2d_bwd: bad tensor dims");
    if (H + 2 * padh < R || W_in + 2 * padw < S)
        return fail(SEERA_ERR_INVALID_ARGUMENT, "conv2d_bwd: kernel larger than padded input");
    SEERA_TRY(check_ptrs(true, Wt, dW, batch > 0 ? X : dW, batch > 0 ? dY : dW,
                         batch > 0 ? dX : dW));
    return conv_bwd(dY, Wt, X, dX, dW, db, batch, C, H, W_in, N, R, S, strideh, stridew, padh, padw,
                    st);
}

int convT_dims(int Hin, int Win, int KH, int KW, int sh, int sw, int ph, int pw, int* Hout,
               int* Wout) {
    SEERA_TRY(check_conv_geometry(KH, KW, sh, sw, ph, pw));
    const int64_t ho = (int64_t)(Hin - 1) * sh - 2 * (int64_t)ph + KH;
    const int64_t wo = (int64_t)(Win - 1) * sw - 2 * (int64_t)pw + KW;
    if (ho < 1 || wo < 1 || ho > INT_MAX || wo > INT_MAX)
        return fail(SEERA_ERR_INVALID_ARGUMENT, "conv_transpose: output extent %lld x %lld",
                    (long long)ho, (long long)wo);
    *Hout = (int)ho;
    *Wout = (int)wo;
    return SEERA_OK;
}

int convT_fwd_impl(const float* X, const float* Wt, float* out, int batch, int Cin, int Hin,
                   int Win, int Cout, int KH, int KW, int sh, int sw, int ph, int pw,
                   hipStream_t st) {
    if (batch < 0 || Cin < 1 || Hin < 1 || Win < 1 || Cout < 1)
        return fail(SEERA_ERR_INVALID_ARGUMENT, "conv2DTranpose_fwd: bad tensor dims");
    int Hout, Wout;
    SEERA_TRY(convT_dims(Hin, Win, KH, KW, sh, sw, ph, pw, &Hout, &Wout));
    SEERA_TRY(check_ptrs(batch > 0, X, Wt, out));
    return conv_dgrad(X, Wt, out, batch, Cin, Hin, Win, Cout, Hout, Wout, KH, KW, sh, sw, ph, pw,
                      st);
}

int convT_bwd_impl(const float* Wt, const float* X, const float* dY, float* dX, float* dW,
                   int batch, int Cin, int Hin, int Win, int Cout, int KH, int KW, int sh, int sw,
                   int ph, int pw, hipStream_t st) {
    if (batch < 0 || Cin < 1 || Hin < 1 || Win < 1 || Cout < 1)
        return fail(SEERA_ERR_INVALID_ARGUMENT, "conv2DTranspose_bwd: bad tensor dims");
    int Hout, Wout;
    SEERA_TRY(convT_dims(Hin, Win, KH, KW, sh, sw, ph, pw, &Hout, &Wout));
    SEERA_TRY(check_ptrs(true, Wt, dW, batch > 0 ? X : dW, batch > 0 ? dY : dW,
                         batch > 0 ? dX : dW));
    // dX = conv2d(dY, W viewed as [F = Cin, C = Cout, KH, KW]); its output
    // extent (Hout + 2ph - KH)/sh + 1 equals Hin exactly.
    SEERA_TRY(conv_fwd(dY, Wt, dX, batch, Cout, Hout, Wout, Cin, KH, KW, sh, sw, ph, pw, st));
    // dW[ci, co, kh, kw] = sum X[b, ci, hi, wi] dY[b, co, hi*sh-ph+kh, wi*sw-pw+kw]:
    // the conv weight gradient with X in the role of dY and dY in that of X.
    return conv_wgrad(X, dY, dW, nullptr, batch, Cout, Hout, Wout, Cin, KH, KW, sh, sw, ph, pw, st);
}

template <class F>
int guarded(F&& f) {
    clear_error();
    return f();
}

}  // namespace

extern "C" {

const char* seera_hip_last_error(void) { return seera::last_error(); }

const char* seera_hip_version(void) { return "seera-hip 0.1 (gfx950)"; }

int seera_hip_device_count(void) {
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess) return -1;
    return n;
}

int seera_hip_malloc(void** out, size_t nbytes) {
    return guarded([&] {
        if (!out) return fail(SEERA_ERR_INVALID_ARGUMENT, "null out pointer");
        return device_malloc(out, nbytes);
    });
}

int seera_hip_free(void* ptr) {
    return guarded([&] { return device_free(ptr); });
}

int seera_hip_malloc_async(void** out, size_t nbytes, void* stream) {
    return guarded([&] {
        if (!out) return fail(SEERA_ERR_INVALID_ARGUMENT, "null out pointer");
        return device_malloc_async(out, nbytes, as_stream(stream));
    });
}

int seera_hip_free_async(void* ptr, void* stream) {
    return guarded([&] { return device_free_async(ptr, as_stream(stream)); });
}

int seera_hip_empty_cache(void) {
    return guarded([&] { return device_empty_cache(); });
}

int seera_hip_memory_stats(size_t* live_bytes, size_t* cached_bytes) {
    return guarded([&] {
        device_memory_stats(live_bytes, cached_bytes);
        return (int)SEERA_OK;
    });
}

int seera_hip_memset(void* ptr, int value, size_t nbytes) {
    return guarded([&] {
        if (nbytes == 0) return (int)SEERA_OK;
        if (!ptr) return fail(SEERA_ERR_INVALID_ARGUMENT, "null device pointer");
        SEERA_HIP_TRY(hipMemset(ptr, value, nbytes));
        return queued(SEERA_OK);
    });
}

int seera_hip_fill_f32(float* ptr, float value, size_t count) {
    return guarded([&] {
        if (count == 0) return (int)SEERA_OK;
        if (!ptr) return fail(SEERA_ERR_INVALID_ARGUMENT, "null device pointer");
        return sync_after(fill_f32(ptr, value, count, nullptr));
    });
}

static int copy(void* dst, const void* src, size_t nbytes, hipMemcpyKind kind) {
    return guarded([&] {
        if (nbytes == 0) return (int)SEERA_OK;
        if (!dst || !src) return fail(SEERA_ERR_INVALID_ARGUMENT, "null pointer in copy");
        SEERA_HIP_TRY(hipMemcpy(dst, src, nbytes, kind));
        return (int)SEERA_OK;
    });
}

int seera_hip_memcpy_d2d(void* dst, const void* src, size_t n) {
    // A device-to-device hipMemcpy may return before the copy has run.
    return queued(copy(dst, src, n, hipMemcpyDeviceToDevice));
}
int seera_hip_memcpy_h2d(void* dst, const void* src, size_t n) {
    return copy(dst, src, n, hipMemcpyHostToDevice);
}
int seera_hip_memcpy_d2h(void* dst, const void* src, size_t n) {
    return copy(dst, src, n, hipMemcpyDeviceToHost);
}

int seera_hip_synchronize(void) {
    return guarded([&] {
        SEERA_HIP_TRY(hipDeviceSynchronize());
        note_device_synchronized();
        return (int)SEERA_OK;
    });
}

int seera_hip_matmul_async(const float* A, const float* B, float* C, int M, int N, int K,
                           int Nbatch, void* stream) {
    return guarded([&] { return queued(matmul_impl(A, B, C, M, N, K, Nbatch, as_stream(stream))); });
}
int seera_hip_matmul(const float* A, const float* B, float* C, int M, int N, int K, int Nbatch) {
    return guarded([&] { return sync_after(matmul_impl(A, B, C, M, N, K, Nbatch, nullptr)); });
}

int seera_hip_matmul_bwd_bias(const float* A, const float* B, const float* dC, float* dA, float* dB,
                              float* db, int M, int N, int K, int Nbatch) {
    return guarded([&] {
        return sync_after(
            matmul_bwd_bias_impl(A, B, dC, nullptr, dA, dB, db, M, N, K, Nbatch, nullptr));
    });
}

int seera_hip_matmul_bwd_bias_async(const float* A, const float* B, const float* dC, float* dA,
                                    float* dB, float* db, int M, int N, int K, int Nbatch,
                                    void* stream) {
    return guarded([&] {
        return queued(matmul_bwd_bias_impl(A, B, dC, nullptr, dA, dB, db, M, N, K, Nbatch,
                                           as_stream(stream)));
    });
}

int seera_hip_matmul_bwd_relu_bias(const float* A, const float* B, const float* dC,
                                   const float* mask, float* dA, float* dB, float* db, int M,
                                   int N, int K, int Nbatch) {
    return guarded([&] {
        return sync_after(
            matmul_bwd_relu_bias_impl(A, B, dC, mask, dA, dB, db, M, N, K, Nbatch, nullptr));
    });
}

int seera_hip_matmul_bwd_relu_bias_async(const float* A, const float* B, const float* dC,
                                         const float* mask, float* dA, float* dB, float* db,
                                         int M, int N, int K, int Nbatch, void* stream) {
    return guarded([&] {
        return queued(matmul_bwd_relu_bias_impl(A, B, dC, mask, dA, dB, db, M, N, K, Nbatch,
                                                as_stream(stream)));
    });
}

int seera_hip_matmul_bwd_relu(const float* A, const float* B, const float* dC, const float* mask,
                              float* dA, float* dB, int M, int N, int K, int Nbatch) {
    return guarded([&] {
        return sync_after(matmul_bwd_relu_impl(A, B, dC, mask, dA, dB, M, N, K, Nbatch, nullptr));
    });
}
int seera_hip_matmul_bwd_relu_async(const float* A, const float* B, const float* dC,
                                    const float* mask, float* dA, float* dB, int M, int N, int K,
                                    int Nbatch, void* stream) {
    return guarded([&] {
        return queued(
            matmul_bwd_relu_impl(A, B, dC, mask, dA, dB, M, N, K, Nbatch, as_stream(stream)));
    });
}
int seera_hip_matmul_bwd_async(const float* A, const float* B, const float* dC, float* dA,
                               float* dB, int M, int N, int K, int Nbatch, void* stream) {
    return guarded(
        [&] { return queued(matmul_bwd_impl(A, B, dC, dA, dB, M, N, K, Nbatch, as_stream(stream))); });
}
int seera_hip_matmul_bwd(const float* A, const float* B, const float* dC, float* dA, float* dB,
                         int M, int N, int K, int Nbatch) {
    return guarded([&] {
        return sync_after(matmul_bwd_impl(A, B, dC, dA, dB, M, N, K, Nbatch, nullptr));
    });
}

int seera_hip_matmul_bias_act_async(const float* A, const float* B, const float* bias, float* C,
                                    float* mask, int M, int N, int K, int Nbatch, int act,
                                    void* stream) {
    return guarded([&] {
        return queued(matmul_bias_act_impl(A, B, bias, C, mask, M, N, K, Nbatch, act,
                                           as_stream(stream)));
    });
}
int seera_hip_matmul_bias_act(const float* A, const float* B, const float* bias, float* C,
                              float* mask, int M, int N, int K, int Nbatch, int act) {
    return guarded([&] {
        return sync_after(matmul_bias_act_impl(A, B, bias, C, mask, M, N, K, Nbatch, act, nullptr));
    });
}

int seera_hip_bias_grad_async(const float* dY, float* db, int rows, int N, void* stream) {
    return guarded([&] { return queued(bias_grad_impl(dY, db, rows, N, as_stream(stream))); });
}
int seera_hip_bias_grad(const float* dY, float* db, int rows, int N) {
    return guarded([&] { return sync_after(bias_grad_impl(dY, db, rows, N, nullptr)); });
}

int seera_hip_maxpool_fwd(const float* image, float* out, int* mask, int batchN, int C, int H,
                          int W, int R, int S, int pad_h, int pad_w, int stride_h, int stride_w) {
    return guarded([&] {
        return sync_after(maxpool_fwd_impl(image, out, mask, batchN, C, H, W, R, S, pad_h, pad_w,
                                           stride_h, stride_w, nullptr));
    });
}
int seera_hip_maxpool_bwd(const float* dout, const int* mask, float* dX, int batchN, int C, int H,
                          int W, int R, int S, int pad_h, int pad_w, int stride_h, int stride_w) {
    return guarded([&] {
        return sync_after(maxpool_bwd_impl(dout, mask, dX, batchN, C, H, W, R, S, pad_h, pad_w,
                                           stride_h, stride_w, nullptr));
    });
}
int seera_hip_maxpool_fwd_async(const float* image, float* out, int* mask, int batchN, int C,
                                int H, int W, int R, int S, int pad_h, int pad_w, int stride_h,
                                int stride_w, void* stream) {
    return guarded([&] {
        return queued(maxpool_fwd_impl(image, out, mask, batchN, C, H, W, R, S, pad_h, pad_w,
                                       stride_h, stride_w, as_stream(stream)));
    });
}
int seera_hip_maxpool_bwd_async(const float* dout, const int* mask, float* dX, int batchN, int C,
                                int H, int W, int R, int S, int pad_h, int pad_w, int stride_h,
                                int stride_w, void* stream) {
    return guarded([&] {
        return queued(maxpool_bwd_impl(dout, mask, dX, batchN, C, H, W, R, S, pad_h, pad_w,
                                       stride_h, stride_w, as_stream(stream)));
    });
}

int seera_hip_transpose_2d(const float* in, float* out, int rows, int cols) {
    return guarded([&] {
        if (rows < 0 || cols < 0) return fail(SEERA_ERR_INVALID_ARGUMENT, "negative extent");
        SEERA_TRY(check_ptrs(prod(rows, cols) > 0, in, out, out));
        return sync_after(transpose(in, out, 1, rows, cols, nullptr));
    });
}

int seera_hip_transpose_3d(const float* in, float* out, int Nbatch, int M, int K) {
    return guarded([&] {
        if (Nbatch < 0 || M < 0 || K < 0) return fail(SEERA_ERR_INVALID_ARGUMENT, "negative extent");
        SEERA_TRY(check_ptrs(prod(Nbatch, M, K) > 0, in, out, out));
        return sync_after(transpose(in, out, Nbatch, M, K, nullptr));
    });
}

int seera_hip_conv2d_fwd_async(const float* image, const float* kernel, float* conv, int batchN,
                               int C, int H, int W, int N, int R, int S, int pad_h, int pad_w,
                               int stride_h, int stride_w, void* stream) {
    return guarded([&] {
        return queued(conv2d_fwd_impl(image, kernel, conv, batchN, C, H, W, N, R, S, pad_h,
                                      pad_w, stride_h, stride_w, as_stream(stream)));
    });
}
int seera_hip_conv2d_fwd_bias_act(const float* image, const float* kernel, const float* bias,
                                  float* conv, float* mask, int batchN, int C, int H, int W, int N,
                                  int R, int S, int pad_h, int pad_w, int stride_h, int stride_w,
                                  int act) {
    return guarded([&] {
        return sync_after(conv2d_fwd_bias_act_impl(image, kernel, bias, conv, mask, batchN, C, H,
                                                   W, N, R, S, pad_h, pad_w, stride_h, stride_w,
                                                   act, nullptr));
    });
}
int seera_hip_conv2d_fwd_bias_act_async(const float* image, const float* kernel,
                                        const float* bias, float* conv, float* mask, int batchN,
                                        int C, int H, int W, int N, int R, int S, int pad_h,
                                        int pad_w, int stride_h, int stride_w, int act,
                                        void* stream) {
    return guarded([&] {
        return queued(conv2d_fwd_bias_act_impl(image, kernel, bias, conv, mask, batchN, C, H, W,
                                               N, R, S, pad_h, pad_w, stride_h, stride_w, act,
                                               as_stream(stream)));
    });
}
int seera_hip_conv_bias_grad(const float* dY, float* db, int batchN, int N, int HW) {
    return guarded([&] { return sync_after(conv_bias_grad_impl(dY, db, batchN, N, HW, nullptr)); });
}
int seera_hip_conv_bias_grad_async(const float* dY, float* db, int batchN, int N, int HW,
                                   void* stream) {
    return guarded([&] {
        return queued(conv_bias_grad_impl(dY, db, batchN, N, HW, as_stream(stream)));
    });
}
int seera_hip_conv2d_fwd(const float* image, const float* kernel, float* conv, int batchN, int C,
                         int H, int W, int N, int R, int S, int pad_h, int pad_w, int stride_h,
                         int stride_w) {
    return guarded([&] {
        return sync_after(conv2d_fwd_impl(image, kernel, conv, batchN, C, H, W, N, R, S, pad_h,
                                          pad_w, stride_h, stride_w, nullptr));
    });
}

int seera_hip_conv2d_bwd_async(const float* W, const float* X, const float* dY, float* dX,
                               float* dW, int batch, int C, int H, int W_in, int N, int R, int S,
                               int strideh, int stridew, int padh, int padw, void* stream) {
    return guarded([&] {
        return queued(conv2d_bwd_impl(W, X, dY, dX, dW, batch, C, H, W_in, N, R, S, strideh,
                                      stridew, padh, padw, as_stream(stream)));
    });
}
int seera_hip_conv2d_bwd(const float* W, const float* X, const float* dY, float* dX, float* dW,
                         int batch, int C, int H, int W_in, int N, int R, int S, int strideh,
                         int stridew, int padh, int padw) {
    return guarded([&] {
        return sync_after(conv2d_bwd_impl(W, X, dY, dX, dW, batch, C, H, W_in, N, R, S, strideh,
                                          stridew, padh, padw, nullptr));
    });
}

int seera_hip_conv2d_bwd_bias(const float* W, const float* X, const float* dY, float* dX,
                              float* dW, float* db, int batch, int C, int H, int W_in, int N,
                              int R, int S, int strideh, int stridew, int padh, int padw) {
    return guarded([&] {
        return sync_after(conv2d_bwd_bias_impl(W, X, dY, dX, dW, db, batch, C, H, W_in, N, R, S,
                                               strideh, stridew, padh, padw, nullptr));
    });
}
int seera_hip_conv2d_bwd_bias_async(const float* W, const float* X, const float* dY, float* dX,
                                    float* dW, float* db, int batch, int C, int H, int W_in,
                                    int N, int R, int S, int strideh, int stridew, int padh,
                                    int padw, void* stream) {
    return guarded([&] {
        return queued(conv2d_bwd_bias_impl(W, X, dY, dX, dW, db, batch, C, H, W_in, N, R, S,
                                           strideh, stridew, padh, padw, as_stream(stream)));
    });
}

int seera_hip_conv2DTranpose_fwd_async(const float* X, const float* W, float* out, int batch,
                                       int Cin, int Hin, int Win, int Cout, int KH, int KW,
                                       int strideh, int stridew, int padh, int padw,
                                       void* stream) {
    return guarded([&] {
        return queued(convT_fwd_impl(X, W, out, batch, Cin, Hin, Win, Cout, KH, KW, strideh,
                                     stridew, padh, padw, as_stream(stream)));
    });
}
int seera_hip_conv2DTranpose_fwd(const float* X, const float* W, float* out, int batch, int Cin,
                                 int Hin, int Win, int Cout, int KH, int KW, int strideh,
                                 int stridew, int padh, int padw) {
    return guarded([&] {
        return sync_after(convT_fwd_impl(X, W, out, batch, Cin, Hin, Win, Cout, KH, KW, strideh,
                                         stridew, padh, padw, nullptr));
    });
}

int seera_hip_conv2DTranspose_bwd_async(const float* W, const float* X, const float* dY,
                                        float* dX, float* dW, int batch, int Cin, int Hin,
                                        int Win, int Cout, int KH, int KW, int strideh,
                                        int stridew, int padh, int padw, void* stream) {
    return guarded([&] {
        return queued(convT_bwd_impl(W, X, dY, dX, dW, batch, Cin, Hin, Win, Cout, KH, KW,
                                     strideh, stridew, padh, padw, as_stream(stream)));
    });
}
int seera_hip_conv2DTranspose_bwd(const float* W, const float* X, const float* dY, float* dX,
                                  float* dW, int batch, int Cin, int Hin, int Win, int Cout,
                                  int KH, int KW, int strideh, int stridew, int padh, int padw) {
    return guarded([&] {
        return sync_after(convT_bwd_impl(W, X, dY, dX, dW, batch, Cin, Hin, Win, Cout, KH, KW,
                                         strideh, stridew, padh, padw, nullptr));
    });
}

int seera_hip_event_create(void** event) {
    return guarded([&] {
        if (!event) return fail(SEERA_ERR_INVALID_ARGUMENT, "null out pointer");
        SEERA_HIP_TRY(hipEventCreate(reinterpret_cast<hipEvent_t*>(event)));
        return (int)SEERA_OK;
    });
}
int seera_hip_event_record(void* event, void* stream) {
    return guarded([&] {
        SEERA_HIP_TRY(hipEventRecord(reinterpret_cast<hipEvent_t>(event), as_stream(stream)));
        return (int)SEERA_OK;
    });
}
int seera_hip_event_elapsed_ms(void* start, void* stop, float* ms) {
    return guarded([&] {
        SEERA_HIP_TRY(hipEventSynchronize(reinterpret_cast<hipEvent_t>(stop)));
        SEERA_HIP_TRY(hipEventElapsedTime(ms, reinterpret_cast<hipEvent_t>(start),
                                          reinterpret_cast<hipEvent_t>(stop)));
        return (int)SEERA_OK;
    });
}
int seera_hip_event_destroy(void* event) {
    return guarded([&] {
        if (event) SEERA_HIP_TRY(hipEventDestroy(reinterpret_cast<hipEvent_t>(event)));
        return (int)SEERA_OK;
    });
}
int seera_hip_stream_create(void** stream) {
    return guarded([&] {
        if (!stream) return fail(SEERA_ERR_INVALID_ARGUMENT, "null out pointer");
        SEERA_HIP_TRY(hipStreamCreate(reinterpret_cast<hipStream_t*>(stream)));
        return (int)SEERA_OK;
    });
}
int seera_hip_stream_destroy(void* stream) {
    return guarded([&] {
        if (!stream) return (int)SEERA_OK;
        SEERA_TRY(stream_destroyed(as_stream(stream)));  // its workspace goes with it
        SEERA_HIP_TRY(hipStreamDestroy(as_stream(stream)));
        return (int)SEERA_OK;
    });
}
int seera_hip_stream_release_workspace(void* stream) {
    return guarded([&] {
        SEERA_TRY(stream_destroyed(as_stream(stream)));  // null stream: kept
        return (int)SEERA_OK;
    });
}
int seera_hip_graph_capture_begin(void* stream) {
    return guarded([&] {
        if (!stream) return fail(SEERA_ERR_INVALID_ARGUMENT, "capture needs a created stream");
        SEERA_HIP_TRY(hipStreamBeginCapture(as_stream(stream), hipStreamCaptureModeThreadLocal));
        return (int)SEERA_OK;
    });
}
int seera_hip_graph_capture_end(void* stream, void** graph_exec) {
    return guarded([&] {
        if (!stream || !graph_exec) return fail(SEERA_ERR_INVALID_ARGUMENT, "null argument");
        *graph_exec = nullptr;
        hipGraph_t graph = nullptr;
        SEERA_HIP_TRY(hipStreamEndCapture(as_stream(stream), &graph));
        hipGraphExec_t exec = nullptr;
        const hipError_t e = hipGraphInstantiate(&exec, graph, nullptr, nullptr, 0);
        (void)hipGraphDestroy(graph);
        if (e != hipSuccess) return fail_hip(e, "hipGraphInstantiate");
        // The graph holds the workspace addresses it was captured with: from
        // now on a grown workspace keeps its old buffer until this graph (and
        // every other live one on the device) is destroyed.
        const int st = graph_created(exec);
        if (st != SEERA_OK) {
            (void)hipGraphExecDestroy(exec);
            return st;
        }
        *graph_exec = exec;
        return (int)SEERA_OK;
    });
}
int seera_hip_graph_launch(void* graph_exec, void* stream) {
    return guarded([&] {
        if (!graph_exec) return fail(SEERA_ERR_INVALID_ARGUMENT, "null graph");
        SEERA_HIP_TRY(hipGraphLaunch(static_cast<hipGraphExec_t>(graph_exec), as_stream(stream)));
        return queued(SEERA_OK);
    });
}
int seera_hip_graph_destroy(void* graph_exec) {
    return guarded([&] {
        if (!graph_exec) return (int)SEERA_OK;
        SEERA_HIP_TRY(hipGraphExecDestroy(static_cast<hipGraphExec_t>(graph_exec)));
        return graph_destroyed(graph_exec);
    });
}
int seera_hip_workspace_stats(size_t* held_bytes, size_t* retired_buffers) {
    return guarded([&] {
        workspace_stats(held_bytes, retired_buffers);
        return (int)SEERA_OK;
    });
}
int seera_hip_stream_synchronize(void* stream) {
    return guarded([&] {
        SEERA_HIP_TRY(hipStreamSynchronize(as_stream(stream)));
        return (int)SEERA_OK;
    });
}

}  // extern "C"
