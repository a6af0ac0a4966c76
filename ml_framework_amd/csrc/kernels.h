// kernels.h -- internal (C++) entry points of the HIP kernels. All enqueue on
// `st` without synchronizing and return a SEERA_* status.
#pragma once

#include <hip/hip_runtime.h>

namespace seera {

// C[Mb, N] = A[Mb, K] . B[K, N] with Mb = M * Nbatch.
int gemm_fwd(const float* A, const float* B, float* C, int M, int N, int K, int Nbatch,
             hipStream_t st);
// C = act(A . B + bias[n]) (bias may be null; act: 0 none, 1 ReLU, which also
// writes mask = pre-activation > 0 when mask is non-null).
int gemm_fwd_bias_act(const float* A, const float* B, const float* bias, float* C, float* mask,
                      int M, int N, int K, int Nbatch, int act, hipStream_t st);
// db[n] = sum_r dY[r, n] for dY [rows, N].
int bias_grad(const float* dY, float* db, int rows, int N, hipStream_t st);
// dA = dC . B^T, dB = A^T . dC over the folded batch.
int gemm_bwd(const float* A, const float* B, const float* dC, float* dA, float* dB, int M, int N,
             int K, int Nbatch, hipStream_t st);
// gemm_bwd plus db[n] = sum over the Nbatch*M rows of dC[., n], taken from the
// dB GEMM's own loads of dC (fp32, before rounding); with a mask, dA as in
// gemm_bwd_relu.
int gemm_bwd_bias(const float* A, const float* B, const float* dC, const float* mask, float* dA,
                  float* dB, float* db, int M, int N, int K, int Nbatch, hipStream_t st);
// gemm_bwd with dA = (dC . B^T) * mask (the ReLU backward of A's layer).
int gemm_bwd_relu(const float* A, const float* B, const float* dC, const float* mask, float* dA,
                  float* dB, int M, int N, int K, int Nbatch, hipStream_t st);
// out[b, c, r] = in[b, r, c] for b < batch.
int transpose(const float* in, float* out, int batch, int rows, int cols, hipStream_t st);

// MaxPool2D with the reference GPU engine's semantics (pool.hip): out
// [B, C, Ho, Wo], mask [B, C, H, W] int32 0/1; dX = mask * sum of covering dout.
int maxpool_fwd(const float* x, float* out, int* mask, int B, int C, int H, int W, int R, int S,
                int ph, int pw, int sh, int sw, hipStream_t st);
int maxpool_bwd(const float* dout, const int* mask, float* dx, int B, int C, int H, int W, int R,
                int S, int ph, int pw, int sh, int sw, hipStream_t st);

// p[0, n) = v.
int fill_f32(float* p, float v, size_t n, hipStream_t st);

// Y[B, F, Ho, Wo] = conv(X[B, C, H, W], Wt[F, C, R, S]).
int conv_fwd(const float* X, const float* Wt, float* Y, int B, int C, int H, int W, int F, int R,
             int S, int sh, int sw, int ph, int pw, hipStream_t st);
// Y = act(conv(X, Wt) + bias[f]) in the convolution's store; bias [F] or
// nullptr, act 0 (none) or 1 (ReLU, mask [B, F, Ho, Wo] = Y > 0 if not null).
int conv_fwd_bias_act(const float* X, const float* Wt, const float* bias, float* Y, float* mask,
                      int B, int C, int H, int W, int F, int R, int S, int sh, int sw, int ph,
                      int pw, int act, hipStream_t st);
// db[F] = sum over images and pixels of dY[B, F, HW], fixed order.
int conv_bias_grad(const float* dY, float* db, int B, int F, int HW, hipStream_t st);
// out[B, C, H, W] = transposed conv of Y[B, F, Hi, Wi] with W[F, C, R, S].
int conv_dgrad(const float* Yin, const float* Wconv, float* out, int B, int F, int Hi, int Wi,
               int C, int H, int W, int R, int S, int sh, int sw, int ph, int pw, hipStream_t st);
// dW[F, C, R, S] = sum over (b, ho, wo) of Y[B, F, Ho, Wo] x im2col(X[B, C, H, W]);
// with db non-null also db[F] = sum over (b, ho, wo) of Y (fused into the
// stride-1 row-streaming pass, a separate fixed-order pass otherwise).
int conv_wgrad(const float* Y, const float* X, float* dW, float* db, int B, int C, int H, int W,
               int F, int R, int S, int sh, int sw, int ph, int pw, hipStream_t st);

// Conv2D backward: dX = conv_dgrad(dY, Wconv), dW (and db when not nullptr) =
// conv_wgrad(dY, X); one fused pass over dY where it applies (3x3, stride 1,
// pad 1, 64 -> 64 channels), the two passes otherwise.
int conv_bwd(const float* dY, const float* Wconv, const float* X, float* dX, float* dW,
             float* db, int B, int C, int H, int W, int F, int R, int S, int sh, int sw, int ph,
             int pw, hipStream_t st);

// ---- tensor_ops.hip: the reference's element-wise, activation, softmax,
// broadcast, unpooling and reduction functions ----
enum {
    kActFwdRelu, kActFwdSigmoid, kActFwdTanh, kActFwdLog, kActFwdExp, kActFwdAbs, kActFwdSqrt,
    kActFwdPow, kActFwdClip
};
// out = f(x), grad = f'(x) over n elements; p0 = exponent (pow) or lo (clip),
// p1 = hi (clip).
int activation_fwd(int kind, const float* x, float* out, float* grad, int64_t n, float p0,
                   float p1, hipStream_t st);
enum { kElemAdd, kElemSub, kElemMul, kElemDiv };
// C = A op B over n elements.
int elementwise(int op, const float* A, const float* B, float* C, int64_t n, hipStream_t st);
enum { kScalarMul, kScalarAdd, kScalarPow };
// p = p op k in place.
int scalar_inplace(int op, float* p, float k, int64_t n, hipStream_t st);
// C = A + B (or A * B) with 4-D broadcasting of extent-1 axes.
int broadcast_4d(bool mul, const float* A, const float* B, float* C, const int a[4],
                 const int b[4], hipStream_t st);
// Nearest-neighbour upsample of [B, C, H, W] by (sh, sw), or its backward
// (dst [B, C, H, W] = block sums of src [B, C, H*sh, W*sw]).
int unpool(bool backward, const float* src, float* dst, int B, int C, int H, int W, int sh,
           int sw, hipStream_t st);
// Row softmax of a [N, C] into out, or (vjp) out = a * (b - <a, b>) per row
// with a = softmax output, b = dout.
int softmax(bool vjp, const float* a, const float* b, float* out, int N, int C, hipStream_t st);
enum {
    kRedSum, kRedMean, kRedMax, kRedMin, kRedArgmax, kRedArgmin, kRedSumBwd, kRedMeanBwd,
    kRedMaxBwd, kRedMinBwd
};
// Reduction of axis `dim` of a row-major tensor with host extents dims[ndims]:
//   forward kinds: A -> out (float, or int for argmax / argmin)
//   kRedSumBwd / kRedMeanBwd: dOut -> out (= dA)
//   kRedMaxBwd / kRedMinBwd: dOut, A (forward input), Y (forward output) -> out
int reduce_axis(int kind, const float* A, const float* Y, const float* dOut, void* out, int ndims,
                int dim, const int* dims, hipStream_t st);

}  // namespace seera
