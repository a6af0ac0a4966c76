/*
 * seera_hip.h -- C ABI of the MI355X (gfx950) Seera matmul/conv hot path.
 *
 * Every entry point takes plain device pointers (fp32, row-major / NCHW, as
 * the reference's cuTen buffers hold them) and C ints, and returns a status
 * code (0 = success). On failure, seera_hip_last_error() gives a message for
 * the calling thread. Operands are rounded to fp16 (round-to-nearest-even) on
 * their way into the matrix cores and accumulated in fp32; outputs are fp32
 * and are overwritten, never accumulated into.
 *
 * The plain entry points keep the reference's "result ready on return"
 * contract (they synchronize the device before returning, like every wrapper
 * in engine_cuda/src). The *_async forms enqueue on `stream` (a hipStream_t;
 * NULL = the null stream) and return without synchronizing.
 */
#ifndef SEERA_HIP_H
#define SEERA_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum {
    SEERA_OK = 0,
    SEERA_ERR_INVALID_ARGUMENT = 1, /* bad dims, null pointer, int overflow */
    SEERA_ERR_HIP = 2,              /* a HIP runtime call or launch failed */
    SEERA_ERR_OUT_OF_MEMORY = 3,    /* device allocation failed */
};

/* Message describing the last failure on this thread ("" if none). */
const char *seera_hip_last_error(void);
/* Library version string. */
const char *seera_hip_version(void);
/* Number of visible devices, or -1 when no HIP device is present. */
int seera_hip_device_count(void);

/* ---- memory and transfer: engine_cuda/src/cuda_bindings.cpp:23-170 ---- */

/* cuda_malloc / cuda_malloc_f32 / _i32 / _i16 / _f16 (cuda_bindings.cpp:23-56). */
int seera_hip_malloc(void **out, size_t nbytes);
/* cuda_free (cuda_bindings.cpp:58-59). NULL is a no-op. Blocks from
 * seera_hip_malloc go back to a per-device cache of their size class and are
 * handed out again; if an *_async entry point (or a memset / device copy) may
 * still have work queued, the device is synchronized first, as cudaFree does. */
int seera_hip_free(void *ptr);
/* No counterpart in the reference (its cuda_malloc / cuda_free synchronize):
 * stream-ordered allocation, for callers that queue work on streams.
 * seera_hip_malloc_async returns a block that work queued on `stream` after
 * the call may use. seera_hip_free_async(ptr, stream) returns a block from
 * either malloc without synchronizing: work queued on `stream` before the
 * free may still use it; a later seera_hip_malloc_async on the same stream
 * may get it back at once (stream order), any other request only once that
 * work has completed (an event recorded at the free). Both fail with
 * SEERA_ERR_INVALID_ARGUMENT while `stream` is being captured into a graph;
 * free_async fails for pointers this allocator did not hand out. */
int seera_hip_malloc_async(void **out, size_t nbytes, void *stream);
int seera_hip_free_async(void *ptr, void *stream);
/* No counterpart in the reference: hands every cached block back to HIP
 * (after a device synchronize), for callers that need the memory elsewhere. */
int seera_hip_empty_cache(void);
/* No counterpart in the reference: bytes held by live allocations and by the
 * cache (size classes: 512 B, powers of two up to 1 MiB, multiples of 2 MiB). */
int seera_hip_memory_stats(size_t *live_bytes, size_t *cached_bytes);
/* cuda_ones_f / cuda_zeros_f (cuda_bindings.cpp:467-477) fill what they
 * allocate: ptr[0, count) = value. Synchronous. */
int seera_hip_fill_f32(float *ptr, float value, size_t count);
/* cuda_memset (cuda_bindings.cpp:65-66). */
int seera_hip_memset(void *ptr, int value, size_t nbytes);
/* cuda_memcopy_devicetodevice (cuda_bindings.cpp:61-62): dst <- src. */
int seera_hip_memcpy_d2d(void *dst, const void *src, size_t nbytes);
/* to_device_* (cuda_bindings.cpp:73-80, 98-105, 155-170): host -> device. */
int seera_hip_memcpy_h2d(void *dst, const void *src, size_t nbytes);
/* to_host_* (cuda_bindings.cpp:82-96, 107-153): device -> host. */
int seera_hip_memcpy_d2h(void *dst, const void *src, size_t nbytes);
/* cudaDeviceSynchronize as closed every reference wrapper. */
int seera_hip_synchronize(void);

/* ---- GEMM: engine_cuda/src/GEMM.cu ---- */

/* cuda_matmul (GEMM.cu:95-103; binding cuda_bindings.cpp:260-264).
 * C[b] = A[b] . B for b < Nbatch: A [Nbatch,M,K], B [K,N] (shared across the
 * batch), C [Nbatch,M,N]. */
int seera_hip_matmul(const float *A, const float *B, float *C, int M, int N,
                     int K, int Nbatch);
int seera_hip_matmul_async(const float *A, const float *B, float *C, int M,
                           int N, int K, int Nbatch, void *stream);

/* No counterpart in the reference: seera_hip_matmul_async for callers that
 * cannot allocate device memory (code under HIP graph capture, serving
 * loops, harnesses that forbid hipMalloc). It calls no hipMalloc / hipFree:
 * its split-K partial sums go to a fixed 8 MiB device array that the
 * library keeps on each GPU it runs on until the process ends (no shape needs
 * more than 6.3 MB of partials today; a call that would exceed 8 MiB fails
 * with SEERA_ERR_INVALID_ARGUMENT). The first call on each device looks up
 * the array's device address (hipGetSymbolAddress): make it outside graph
 * capture; later calls need no warm-up. Every
 * call on one GPU shares that array, so calls that overlap on one GPU (on two
 * streams, or from two host threads) race: queue them on one stream. */
int seera_hip_matmul_noalloc(const float *A, const float *B, float *C, int M,
                             int N, int K, int Nbatch, void *stream);

/* cuda_matmul_bwd (GEMM.cu:164-225; binding cuda_bindings.cpp:267-273).
 * dA[b] = dC[b] . B^T  and  dB = sum_b A[b]^T . dC[b]; both overwritten. */
int seera_hip_matmul_bwd(const float *A, const float *B, const float *dC,
                         float *dA, float *dB, int M, int N, int K,
                         int Nbatch);
int seera_hip_matmul_bwd_async(const float *A, const float *B, const float *dC,
                               float *dA, float *dB, int M, int N, int K,
                               int Nbatch, void *stream);

/* No single counterpart in the reference: the backward of a Dense layer with
 * its bias gradient, which the reference runs as cuda_matmul_bwd (GEMM.cu:
 * 164-225) and a separate sum of dY over the batch rows (Reductionsum,
 * reductionKernels.cu:12-29, called from Seera_Engine.py:43-65). Here
 * db[n] = sum over the Nbatch*M rows of dC[., n] (db [N]) is taken in fp32
 * from the dB GEMM's own loads of dC, in a fixed order (bit-reproducible);
 * dA and dB are bit-identical to seera_hip_matmul_bwd. */
int seera_hip_matmul_bwd_bias(const float *A, const float *B, const float *dC,
                              float *dA, float *dB, float *db, int M, int N,
                              int K, int Nbatch);
int seera_hip_matmul_bwd_bias_async(const float *A, const float *B,
                                    const float *dC, float *dA, float *dB,
                                    float *db, int M, int N, int K, int Nbatch,
                                    void *stream);
/* The two above together for a Dense layer whose input came out of a ReLU:
 * dA = (dC . B^T) * mask as in seera_hip_matmul_bwd_relu, dB and db as in
 * seera_hip_matmul_bwd_bias (no single counterpart in the reference). */
int seera_hip_matmul_bwd_relu_bias(const float *A, const float *B,
                                   const float *dC, const float *mask,
                                   float *dA, float *dB, float *db, int M,
                                   int N, int K, int Nbatch);
int seera_hip_matmul_bwd_relu_bias_async(const float *A, const float *B,
                                         const float *dC, const float *mask,
                                         float *dA, float *dB, float *db, int M,
                                         int N, int K, int Nbatch,
                                         void *stream);

/* No single counterpart in the reference: the backward of a Dense layer whose
 * input A came out of a ReLU. The reference runs cuda_matmul_bwd, then the
 * ReLU's chain rule on dA -- local_grad * cp with local_grad the ReLU's 0/1
 * grad buffer (Seera_Engine.py:575-583; activations.cu:9-15). Here
 * dA = (dC . B^T) * mask is applied in the dA GEMM's store (mask
 * [Nbatch*M, K], as written by seera_hip_matmul_bias_act with ReLU, read
 * only); dB = A^T . dC as in seera_hip_matmul_bwd. Bit-identical to the two
 * calls. */
int seera_hip_matmul_bwd_relu(const float *A, const float *B, const float *dC,
                              const float *mask, float *dA, float *dB, int M,
                              int N, int K, int Nbatch);
int seera_hip_matmul_bwd_relu_async(const float *A, const float *B,
                                    const float *dC, const float *mask,
                                    float *dA, float *dB, int M, int N, int K,
                                    int Nbatch, void *stream);

/* No single counterpart in the reference: the Dense-layer forward it runs as
 * three calls -- cuda_matmul (GEMM.cu:95-103), broadcast_add_4d of the bias
 * (broadcast.cu:12-64, 140-146) and cuda_relu_fwd (activations.cu:9-15) --
 * fused into the GEMM's store: C = act(A . B + bias[n]), with bias [N] (NULL:
 * none) added in fp32 and act SEERA_ACT_NONE or SEERA_ACT_RELU. ReLU gives
 * C = v > 0 ? v : 0 and, when mask is non-NULL, mask = v > 0 ? 1 : 0 (the
 * reference's relu grad buffer), [Nbatch*M, N] like C. Bit-identical to the
 * three calls. */
enum { SEERA_ACT_NONE = 0, SEERA_ACT_RELU = 1 };
int seera_hip_matmul_bias_act(const float *A, const float *B, const float *bias,
                              float *C, float *mask, int M, int N, int K,
                              int Nbatch, int act);
int seera_hip_matmul_bias_act_async(const float *A, const float *B,
                                    const float *bias, float *C, float *mask,
                                    int M, int N, int K, int Nbatch, int act,
                                    void *stream);

/* The bias gradient the reference takes with Reductionsum over the batch
 * (reductionKernels.cu:12-29 via Seera_Engine.py:43-65): db[n] = sum over
 * rows of dY [rows, N], in a fixed order. */
int seera_hip_bias_grad(const float *dY, float *db, int rows, int N);
int seera_hip_bias_grad_async(const float *dY, float *db, int rows, int N,
                              void *stream);

/* cuda_maxpool_fwd (maxPool.cu:9-53, 79-103; binding cuda_bindings.cpp:338-343):
 * out [batchN, C, Ho, Wo] with Ho = (H + 2 pad_h - R) / stride_h + 1; mask
 * [batchN, C, H, W] int32, 1 at each window's argmax and 0 elsewhere. The max
 * starts at the window origin (0 if the origin is padding) and ties go to the
 * later element, as in the reference; where windows overlap, an element that
 * is any window's argmax is 1 (the reference leaves that to thread order). */
int seera_hip_maxpool_fwd(const float *image, float *out, int *mask, int batchN,
                          int C, int H, int W, int R, int S, int pad_h,
                          int pad_w, int stride_h, int stride_w);
/* cuda_maxpool_bwd (maxPool.cu:56-77, 105-129; binding cuda_bindings.cpp:346-351):
 * dX [batchN, C, H, W] = sum over the windows covering each element of
 * dout * mask (overwritten). */
int seera_hip_maxpool_bwd(const float *dout, const int *mask, float *dX,
                          int batchN, int C, int H, int W, int R, int S,
                          int pad_h, int pad_w, int stride_h, int stride_w);
/* The same two on `stream`, returning once queued (as the other _async
 * entry points). */
int seera_hip_maxpool_fwd_async(const float *image, float *out, int *mask,
                                int batchN, int C, int H, int W, int R, int S,
                                int pad_h, int pad_w, int stride_h,
                                int stride_w, void *stream);
int seera_hip_maxpool_bwd_async(const float *dout, const int *mask, float *dX,
                                int batchN, int C, int H, int W, int R, int S,
                                int pad_h, int pad_w, int stride_h,
                                int stride_w, void *stream);

/* cuda_transpose_2d (GEMM.cu:229-235; binding cuda_bindings.cpp:276-280).
 * out[c,r] = in[r,c], bit-exact. */
int seera_hip_transpose_2d(const float *in, float *out, int rows, int cols);

/* cuda_transpose_3d (GEMM.cu:143-150; binding cuda_bindings.cpp:283-287).
 * out[b,k,m] = in[b,m,k], bit-exact. */
int seera_hip_transpose_3d(const float *in, float *out, int Nbatch, int M,
                           int K);

/* ---- Conv2D: engine_cuda/src/convolution.cu ---- */

/* cuda_conv2d_fwd (convolution.cu:367-389; binding cuda_bindings.cpp:294-299).
 * NOTE the argument order: pad before stride.
 * conv[b,n,ho,wo] = sum_{c,r,s} kernel[n,c,r,s] *
 *                   image[b,c,ho*stride_h-pad_h+r, wo*stride_w-pad_w+s]
 * image [batchN,C,H,W], kernel [N,C,R,S], conv [batchN,N,Hout,Wout],
 * Hout = (H + 2 pad_h - R)/stride_h + 1. */
int seera_hip_conv2d_fwd(const float *image, const float *kernel, float *conv,
                         int batchN, int C, int H, int W, int N, int R, int S,
                         int pad_h, int pad_w, int stride_h, int stride_w);
int seera_hip_conv2d_fwd_async(const float *image, const float *kernel,
                               float *conv, int batchN, int C, int H, int W,
                               int N, int R, int S, int pad_h, int pad_w,
                               int stride_h, int stride_w, void *stream);

/* No single counterpart in the reference: a Conv2D layer's forward
 * (Seera.py:254-257) runs cuda_conv2d_fwd (convolution.cu:367-389), then
 * broadcast_add_4d of the bias [1, N, 1, 1] (broadcast.cu:12-64, 140-146),
 * then cuda_relu_fwd (activations.cu:9-15). Here the bias (NULL: none) and
 * act (SEERA_ACT_NONE or SEERA_ACT_RELU) are applied in the convolution's
 * store: conv = act(conv2d(image, kernel) + bias[n]), and with ReLU and a
 * non-NULL mask, mask = v > 0 ? 1 : 0, [batchN, N, Hout, Wout] like conv.
 * Bit-identical to the three calls. Argument order as seera_hip_conv2d_fwd. */
int seera_hip_conv2d_fwd_bias_act(const float *image, const float *kernel,
                                  const float *bias, float *conv, float *mask,
                                  int batchN, int C, int H, int W, int N, int R,
                                  int S, int pad_h, int pad_w, int stride_h,
                                  int stride_w, int act);
int seera_hip_conv2d_fwd_bias_act_async(const float *image, const float *kernel,
                                        const float *bias, float *conv,
                                        float *mask, int batchN, int C, int H,
                                        int W, int N, int R, int S, int pad_h,
                                        int pad_w, int stride_h, int stride_w,
                                        int act, void *stream);

/* The Conv2D bias gradient: the reference reduces dY [batchN, N, H, W] to the
 * bias shape [1, N, 1, 1] with three sums (Seera_Engine.py:42-65, cuTen sum
 * over axes 3, 2, 0; reductionKernels.cu:12-29). Here db[n] = sum over images
 * and the HW pixels of dY in one fixed order (deterministic; fp32 sums in
 * another order than the reference's). */
int seera_hip_conv_bias_grad(const float *dY, float *db, int batchN, int N,
                             int HW);
int seera_hip_conv_bias_grad_async(const float *dY, float *db, int batchN,
                                   int N, int HW, void *stream);

/* cuda_conv2d_bwd (convolution.cu:393-453; binding cuda_bindings.cpp:302-309).
 * NOTE the argument order: stride before pad.
 * dX = adjoint of conv2d_fwd in the image, dW = adjoint in the kernel. */
int seera_hip_conv2d_bwd(const float *W, const float *X, const float *dY,
                         float *dX, float *dW, int batch, int C, int H,
                         int W_in, int N, int R, int S, int strideh,
                         int stridew, int padh, int padw);
int seera_hip_conv2d_bwd_async(const float *W, const float *X, const float *dY,
                               float *dX, float *dW, int batch, int C, int H,
                               int W_in, int N, int R, int S, int strideh,
                               int stridew, int padh, int padw, void *stream);

/* No single counterpart in the reference: a Conv2D layer's backward with its
 * bias. The reference runs cuda_conv2d_bwd (convolution.cu:393-453) and, for
 * the bias, reduces dY to [1, N, 1, 1] with three cuten.sum calls
 * (Seera_Engine.py:42-65; reductionKernels.cu:12-29). Here dX and dW are
 * those of seera_hip_conv2d_bwd (same kernels, same bits) and db[n] = sum of
 * dY over images and pixels is taken from the fp32 dY values as the
 * weight-gradient pass loads them (stride-1 convolutions whose rows fit its
 * tiles; other shapes take a separate fixed-order pass), so dY is not read a
 * second time. db sums in a fixed order (deterministic; another order than
 * the reference's). Argument order as seera_hip_conv2d_bwd, db after dW. */
int seera_hip_conv2d_bwd_bias(const float *W, const float *X, const float *dY,
                              float *dX, float *dW, float *db, int batch,
                              int C, int H, int W_in, int N, int R, int S,
                              int strideh, int stridew, int padh, int padw);
int seera_hip_conv2d_bwd_bias_async(const float *W, const float *X,
                                    const float *dY, float *dX, float *dW,
                                    float *db, int batch, int C, int H,
                                    int W_in, int N, int R, int S,
                                    int strideh, int stridew, int padh,
                                    int padw, void *stream);

/* ---- ConvTranspose2D: engine_cuda/src/upsampling.cu ---- */

/* cuda_conv2DTranpose_fwd [sic] (upsampling.cu:376-401; binding
 * cuda_bindings.cpp:316-321). X [batch,Cin,Hin,Win], W [Cin,Cout,KH,KW],
 * out [batch,Cout,Hout,Wout], Hout = (Hin-1)*strideh - 2 padh + KH. */
int seera_hip_conv2DTranpose_fwd(const float *X, const float *W, float *out,
                                 int batch, int Cin, int Hin, int Win,
                                 int Cout, int KH, int KW, int strideh,
                                 int stridew, int padh, int padw);
int seera_hip_conv2DTranpose_fwd_async(const float *X, const float *W,
                                       float *out, int batch, int Cin, int Hin,
                                       int Win, int Cout, int KH, int KW,
                                       int strideh, int stridew, int padh,
                                       int padw, void *stream);

/* cuda_conv2DTranspose_bwd (upsampling.cu:322-375; binding
 * cuda_bindings.cpp:324-331). dX [batch,Cin,Hin,Win], dW [Cin,Cout,KH,KW]. */
int seera_hip_conv2DTranspose_bwd(const float *W, const float *X,
                                  const float *dY, float *dX, float *dW,
                                  int batch, int Cin, int Hin, int Win,
                                  int Cout, int KH, int KW, int strideh,
                                  int stridew, int padh, int padw);
int seera_hip_conv2DTranspose_bwd_async(const float *W, const float *X,
                                        const float *dY, float *dX, float *dW,
                                        int batch, int Cin, int Hin, int Win,
                                        int Cout, int KH, int KW, int strideh,
                                        int stridew, int padh, int padw,
                                        void *stream);

/* ---- the functions around the path: activations, softmax, element-wise,
 * scalar, broadcast, unpooling and reductions. cuTen.py and Seera_Engine.py
 * call them on every layer (bias add cuTen.py:160, activation cuTen.py:329,
 * softmax head cuTen.py:401, bias gradient cuTen.py:490). All are
 * synchronous: the result is ready on return. Sizes are element counts.
 * Exact fp32 in the reference's order except where noted: the transcendental
 * functions (exp, log, tanh, pow) come from the device math library and the
 * softmax sums run in a fixed butterfly order. ---- */

/* Activations: out = f(x) and grad = f'(x), the local gradient the autograd
 * multiplies in later (activations.cu:9-85, 164-198; bindings
 * cuda_bindings.cpp:176-239):
 *   relu    out = x > 0 ? x : 0,         grad = x > 0 ? 1 : 0
 *   sigmoid out = s = 1/(1 + exp(-x)),   grad = s (1 - s)
 *   tanh    out = t = tanh(x),           grad = 1 - t t
 *   log     out = log(x),                grad = 1 / x
 *   exp     out = e = exp(x),            grad = e
 *   abs     out = |x|,                   grad = sign(x) (0 at 0)
 *   sqrt    out = s = sqrt(x),           grad = 0.5 / (s + 1e-12)
 *   pow     out = x^p,                   grad = p x^(p-1)
 *   clip    out = min(max(x, lo), hi),   grad = lo <= x <= hi ? 1 : 0 */
int seera_hip_relu_fwd(const float *x, float *out, float *grad, int size);
int seera_hip_sigmoid_fwd(const float *x, float *out, float *grad, int size);
int seera_hip_tanh_fwd(const float *x, float *out, float *grad, int size);
int seera_hip_log_fwd(const float *x, float *out, float *grad, int size);
int seera_hip_exp_fwd(const float *x, float *out, float *grad, int size);
int seera_hip_abs_fwd(const float *x, float *out, float *grad, int size);
int seera_hip_sqrt_fwd(const float *x, float *out, float *grad, int size);
int seera_hip_pow_fwd(const float *x, float exponent, float *out, float *grad,
                      int size);
int seera_hip_clip_fwd(const float *x, float lo, float hi, float *out,
                       float *grad, int size);

/* cuda_softmax_fwd (activations.cu:87-127, 201-204; binding
 * cuda_bindings.cpp:243-247): out[n] = exp(x[n] - max) / sum over each row
 * of x [N, C]. */
int seera_hip_softmax_fwd(const float *x, float *out, int N, int C);
/* cuda_softmax_vjp (activations.cu:129-161, 206-209; binding
 * cuda_bindings.cpp:249-253): dx = s * (dout - <s, dout>) per row, with s
 * the softmax output. */
int seera_hip_softmax_vjp(const float *s, const float *dout, float *dx, int N,
                          int C);

/* cuda_unpooling_fwd (unpooling.cu:7-26, 55-76; binding cuda_bindings.cpp:
 * 358-363): out [batchN, C, H*sh, W*sw], out[.., h, w] = inp[.., h/sh, w/sw]. */
int seera_hip_unpooling_fwd(const float *inp, float *out, int batchN, int C,
                            int H, int W, int sh, int sw);
/* cuda_unpooling_bwd (unpooling.cu:28-50, 78-98; binding cuda_bindings.cpp:
 * 365-370): dx [batchN, C, H, W] = sum of dout over each sh x sw block, row
 * by row. */
int seera_hip_unpooling_bwd(const float *dout, float *dx, int batchN, int C,
                            int H, int W, int sh, int sw);

/* Reductions along axis `dim` of a row-major tensor whose ndims extents are
 * in the HOST array dimarr (reductionKernels.cu:12-207; bindings
 * cuda_bindings.cpp:376-421). out holds the product of the other extents:
 *   sum   in index order from +0;   mean = that sum / extent
 *   max / min   fmax / fmin from the first element
 *   argmax / argmin   index (int32) of the last element >= / <= all before */
int seera_hip_sum_fwd(const float *A, float *out, int ndims, int dim,
                      const int *dimarr);
int seera_hip_mean_fwd(const float *A, float *out, int ndims, int dim,
                       const int *dimarr);
int seera_hip_max_fwd(const float *A, float *out, int ndims, int dim,
                      const int *dimarr);
int seera_hip_min_fwd(const float *A, float *out, int ndims, int dim,
                      const int *dimarr);
int seera_hip_argmax_fwd(const float *A, int *out, int ndims, int dim,
                         const int *dimarr);
int seera_hip_argmin_fwd(const float *A, int *out, int ndims, int dim,
                         const int *dimarr);
/* Their backward (reductionKernels.cu:209-380; bindings cuda_bindings.cpp:
 * 426-457), dA with the forward input's shape, every element written:
 *   sum / mean   dA = dOut (/ extent for mean) along the axis
 *   max / min    dA = dOut at the first element equal to the forward output
 *                fwdOutput, 0 elsewhere */
int seera_hip_sum_bwd(const float *dOut, float *dA, int ndims, int dim,
                      const int *dimarr);
int seera_hip_mean_bwd(const float *dOut, float *dA, int ndims, int dim,
                       const int *dimarr);
int seera_hip_max_bwd(const float *dOut, const float *fwdInput,
                      const float *fwdOutput, float *dA, int ndims, int dim,
                      const int *dimarr);
int seera_hip_min_bwd(const float *dOut, const float *fwdInput,
                      const float *fwdOutput, float *dA, int ndims, int dim,
                      const int *dimarr);

/* In place: arr *= k, arr += k, arr = pow(arr, k) (cuTen_essentails.cu:44-51,
 * 17-24, 53-60, wrappers 88-146; bindings cuda_bindings.cpp:461-465, 479-481). */
int seera_hip_scaler_multiply_f(float *arr, float k, int total_elements);
int seera_hip_scaler_add_f(float *arr, float k, int total_elements);
int seera_hip_power_of(float *arr, float k, int total_elements);

/* C = A op B element by element (elemops.cu:14-40, 46-81; bindings
 * cuda_bindings.cpp:486-512). */
int seera_hip_elemadd(const float *A, const float *B, float *C, int size);
int seera_hip_elemsub(const float *A, const float *B, float *C, int size);
int seera_hip_elemdiv(const float *A, const float *B, float *C, int size);
int seera_hip_elemmult(const float *A, const float *B, float *C, int size);

/* 4-D broadcast (broadcast.cu:12-153; bindings cuda_bindings.cpp:518-532):
 * C = A + B or A * B, where each axis of C has the extent of A or B that is
 * not 1 and an operand's extent-1 axes are read at index 0; C must hold the
 * broadcast shape. Shapes that do not broadcast fail with
 * SEERA_ERR_INVALID_ARGUMENT (the reference prints a message and writes
 * nothing). */
int seera_hip_broadcast_add_4d(const float *A, const float *B, float *C,
                               int aN, int aC, int aH, int aW, int bN, int bC,
                               int bH, int bW);
int seera_hip_broadcast_mul_4d(const float *A, const float *B, float *C,
                               int aN, int aC, int aH, int aW, int bN, int bC,
                               int bH, int bW);

/* ---- timing (no reference counterpart; used by bench.py) ---- */

/* Events on `stream`: create / record / elapsed milliseconds / destroy. */
int seera_hip_event_create(void **event);
int seera_hip_event_record(void *event, void *stream);
int seera_hip_event_elapsed_ms(void *start, void *stop, float *ms);
int seera_hip_event_destroy(void *event);
/* Create / destroy a default-priority stream. */
int seera_hip_stream_create(void **stream);
int seera_hip_stream_destroy(void *stream);
int seera_hip_stream_synchronize(void *stream);
/* Give back the library workspace of a stream the caller created itself
 * (a framework's stream passed to the _async entry points, not one made by
 * seera_hip_stream_create): the workspace is freed once the stream's queued
 * work is done, or kept while a graph is live on the device (freed with the
 * device's last graph). Call it before destroying such a stream: HIP may hand
 * the same handle to a new stream, which would otherwise inherit the old
 * buffer; until then the workspace is held to the end of the process. A
 * later call on the stream simply starts a new workspace. Streams made by
 * seera_hip_stream_create release theirs in seera_hip_stream_destroy; the
 * null stream's workspace is kept (no-op). No counterpart in the reference,
 * which has no streams. */
int seera_hip_stream_release_workspace(void *stream);

/* HIP graphs of the _async entry points (no counterpart in the reference,
 * which launches every kernel from Python and synchronizes after each). Begin
 * capture on a created stream, queue _async calls on it, end capture to get
 * an executable graph, then replay it with seera_hip_graph_launch: one launch
 * for the whole sequence, with the pointers and sizes captured.
 *
 * Workspace rule. Temporaries (split-K partials, re-laid-out weights, dW
 * partials) live in a library workspace, one per (device, stream): _async
 * calls on two streams never share one. A graph keeps the workspace address
 * of its capture stream, so:
 *   - make one eager call of each captured call (same sizes, same stream)
 *     before capturing; a call that would have to grow the workspace during
 *     capture fails with SEERA_ERR_INVALID_ARGUMENT;
 *   - while a graph is live on a device, a workspace that grows keeps its old
 *     buffer (replays keep writing there) until the device's last graph is
 *     destroyed, so eager calls of any size may run between replays;
 *   - a replay and an eager call queued on the capture stream itself are
 *     ordered; a replay on another stream must not overlap eager calls on the
 *     capture stream (they share that stream's workspace);
 *   - seera_hip_stream_destroy frees the stream's workspace (or keeps it
 *     while a graph is live on the device); a stream the caller created
 *     itself gives its workspace back with seera_hip_stream_release_workspace
 *     before the caller destroys it.
 * The _async entry points clear memory with kernels, not memset nodes. */
int seera_hip_graph_capture_begin(void *stream);
int seera_hip_graph_capture_end(void *stream, void **graph_exec);
int seera_hip_graph_launch(void *graph_exec, void *stream);
int seera_hip_graph_destroy(void *graph_exec);
/* Bytes held by the library's workspaces (all devices and streams) and the
 * number of old workspace buffers kept alive for live graphs. */
int seera_hip_workspace_stats(size_t *held_bytes, size_t *retired_buffers);

#ifdef __cplusplus
}
#endif

#endif /* SEERA_HIP_H */
