/*
 * seera_cpp_oracle.c -- TEST INFRASTRUCTURE ONLY (parity checker and CPU
 * baseline). Nothing in the product links, loads or calls this file; only
 * tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg do.
 *
 * A C restatement of the reference's CPU engine `seera_cpp` for the GEMM /
 * Conv2D / ConvTranspose2D path (OpenBLAS sgemm + im2col/col2im + OpenMP):
 *
 *   oracle_matmul                 engine/src/tensor_ops.cpp:9-15
 *   oracle_matmul_bwd             Seera_Engine.py:557-564 (dA = dC.B^T,
 *                                 dB = A^T.dC; composed from seera_cpp.matmul)
 *   oracle_im2col_batch           engine/src/conv_ops.cpp:10-49
 *   oracle_col2im_batch           engine/src/conv_ops.cpp:52-91
 *   oracle_conv2d_forward         engine/src/conv_ops.cpp:95-122
 *   oracle_conv2d_backward        engine/src/conv_ops.cpp:127-185
 *   oracle_conv_transpose2d_fwd   engine/src/conv_ops.cpp:197-228
 *   oracle_conv_transpose2d_bwd   engine/src/conv_ops.cpp:233-287
 *
 * The reference's sgemm is OpenBLAS `cblas_sgemm` (system package, version
 * unpinned, build_engine.py:51-52). This restatement calls the OpenBLAS that
 * numpy bundles (0.3.29, ILP64 symbol `scipy_cblas_sgemm64_`), located by the
 * Python side and handed to oracle_init(). If that library cannot be opened,
 * a plain C sgemm (definition of C = op(A).op(B), fp32 accumulate) is used and
 * oracle_backend() reports 0.
 *
 * Layout conventions follow the reference: row-major / NCHW fp32, im2col row
 * index = c*KH*KW + kh*KW + kw, column index = oh*OW + ow; col2im is a
 * zero-fill followed by a scatter-add; per-sample dW partials are summed
 * serially in sample order.
 */
#include <dlfcn.h>
#include <stddef.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>
#include <omp.h>

enum { ORC_ROW_MAJOR = 101, ORC_NO_TRANS = 111, ORC_TRANS = 112 };

typedef void (*sgemm64_fn)(int order, int ta, int tb, int64_t m, int64_t n,
                           int64_t k, float alpha, const float *a, int64_t lda,
                           const float *b, int64_t ldb, float beta, float *c,
                           int64_t ldc);
typedef void (*set_threads_fn)(int64_t);

static sgemm64_fn g_blas_sgemm = NULL;
static set_threads_fn g_blas_threads = NULL;

/* Plain row-major sgemm: C = alpha*op(A).op(B) + beta*C, fp32 accumulate.
 * Used only when no OpenBLAS can be opened. i-k-j order for unit stride. */
static void plain_sgemm(int ta, int tb, int64_t m, int64_t n, int64_t k,
                        float alpha, const float *a, int64_t lda,
                        const float *b, int64_t ldb, float beta, float *c,
                        int64_t ldc)
{
    for (int64_t i = 0; i < m; i++) {
        float *ci = c + i * ldc;
        if (beta == 0.0f)
            for (int64_t j = 0; j < n; j++) ci[j] = 0.0f;
        else if (beta != 1.0f)
            for (int64_t j = 0; j < n; j++) ci[j] *= beta;
        for (int64_t p = 0; p < k; p++) {
            float av = ta == ORC_TRANS ? a[p * lda + i] : a[i * lda + p];
            av *= alpha;
            if (tb == ORC_TRANS) {
                for (int64_t j = 0; j < n; j++) ci[j] += av * b[j * ldb + p];
            } else {
                const float *bp = b + p * ldb;
                for (int64_t j = 0; j < n; j++) ci[j] += av * bp[j];
            }
        }
    }
}

static void sgemm_rm(int ta, int tb, int64_t m, int64_t n, int64_t k,
                     const float *a, int64_t lda, const float *b, int64_t ldb,
                     float beta, float *c, int64_t ldc)
{
    if (g_blas_sgemm)
        g_blas_sgemm(ORC_ROW_MAJOR, ta, tb, m, n, k, 1.0f, a, lda, b, ldb, beta,
                     c, ldc);
    else
        plain_sgemm(ta, tb, m, n, k, 1.0f, a, lda, b, ldb, beta, c, ldc);
}

/* Open OpenBLAS at `blas_path` (may be NULL). Returns 1 when the OpenBLAS
 * sgemm is in use, 0 for the plain C fallback. nthreads <= 0 keeps defaults. */
int oracle_init(const char *blas_path, int nthreads)
{
    g_blas_sgemm = NULL;
    g_blas_threads = NULL;
    if (blas_path && blas_path[0]) {
        void *h = dlopen(blas_path, RTLD_NOW | RTLD_LOCAL);
        if (h) {
            g_blas_sgemm = (sgemm64_fn)dlsym(h, "scipy_cblas_sgemm64_");
            g_blas_threads =
                (set_threads_fn)dlsym(h, "scipy_openblas_set_num_threads64_");
        }
    }
    if (nthreads > 0) {
        omp_set_num_threads(nthreads);
        if (g_blas_threads) g_blas_threads((int64_t)nthreads);
    }
    return g_blas_sgemm != NULL;
}

int oracle_backend(void) { return g_blas_sgemm != NULL; }

/* tensor_ops.cpp:9-15 -- C(M,N) = A(M,K).B(K,N). */
void oracle_matmul(const float *A, const float *B, float *C, int M, int K,
                   int N)
{
    sgemm_rm(ORC_NO_TRANS, ORC_NO_TRANS, M, N, K, A, K, B, N, 0.0f, C, N);
}

/* Batched-A forward as the GPU entry defines it (GEMM.cu:13-103): A is
 * [Nbatch,M,K], B [K,N] shared, C [Nbatch,M,N]; one 2-D product per slice. */
void oracle_matmul_batched(const float *A, const float *B, float *C, int M,
                           int N, int K, int Nbatch)
{
    for (int b = 0; b < Nbatch; b++)
        oracle_matmul(A + (size_t)b * M * K, B, C + (size_t)b * M * N, M, K, N);
}

/* Seera_Engine.py:557-564 composed per slice: dA_b = dC_b.B^T and
 * dB = sum_b A_b^T.dC_b (accumulated in slice order). Outputs overwritten. */
void oracle_matmul_bwd(const float *A, const float *B, const float *dC,
                       float *dA, float *dB, int M, int N, int K, int Nbatch)
{
    for (int b = 0; b < Nbatch; b++)
        sgemm_rm(ORC_NO_TRANS, ORC_TRANS, M, K, N, dC + (size_t)b * M * N, N,
                 B, N, 0.0f, dA + (size_t)b * M * K, K);
    for (int b = 0; b < Nbatch; b++)
        sgemm_rm(ORC_TRANS, ORC_NO_TRANS, K, N, M, A + (size_t)b * M * K, K,
                 dC + (size_t)b * M * N, N, b == 0 ? 0.0f : 1.0f, dB, N);
    if (Nbatch <= 0) memset(dB, 0, sizeof(float) * (size_t)K * N);
}

static inline int out_extent(int in, int pad, int k, int stride)
{
    return (in + 2 * pad - k) / stride + 1;
}

/* conv_ops.cpp:10-49 -- col[n][c*KH*KW + kh*KW + kw][oh*OW + ow]. */
void oracle_im2col_batch(const float *X, float *col, int N, int C, int H,
                         int W, int KH, int KW, int sh, int sw, int ph, int pw)
{
    const int OH = out_extent(H, ph, KH, sh), OW = out_extent(W, pw, KW, sw);
    const size_t rows = (size_t)C * KH * KW, cols = (size_t)OH * OW;
#pragma omp parallel for schedule(static)
    for (int n = 0; n < N; n++) {
        const float *img = X + (size_t)n * C * H * W;
        float *dst = col + (size_t)n * rows * cols;
        for (int c = 0; c < C; c++)
            for (int kh = 0; kh < KH; kh++)
                for (int kw = 0; kw < KW; kw++) {
                    float *row = dst + ((size_t)(c * KH + kh) * KW + kw) * cols;
                    for (int oh = 0; oh < OH; oh++) {
                        const int h = oh * sh + kh - ph;
                        for (int ow = 0; ow < OW; ow++) {
                            const int w = ow * sw + kw - pw;
                            row[(size_t)oh * OW + ow] =
                                (h >= 0 && h < H && w >= 0 && w < W)
                                    ? img[((size_t)c * H + h) * W + w]
                                    : 0.0f;
                        }
                    }
                }
    }
}

/* conv_ops.cpp:52-91 -- zero X, then scatter-add every col entry back. */
void oracle_col2im_batch(const float *col, float *X, int N, int C, int H,
                         int W, int KH, int KW, int sh, int sw, int ph, int pw)
{
    const int OH = out_extent(H, ph, KH, sh), OW = out_extent(W, pw, KW, sw);
    const size_t rows = (size_t)C * KH * KW, cols = (size_t)OH * OW;
    memset(X, 0, sizeof(float) * (size_t)N * C * H * W);
#pragma omp parallel for schedule(static)
    for (int n = 0; n < N; n++) {
        const float *src = col + (size_t)n * rows * cols;
        float *img = X + (size_t)n * C * H * W;
        for (int c = 0; c < C; c++)
            for (int kh = 0; kh < KH; kh++)
                for (int kw = 0; kw < KW; kw++) {
                    const float *row =
                        src + ((size_t)(c * KH + kh) * KW + kw) * cols;
                    for (int oh = 0; oh < OH; oh++) {
                        const int h = oh * sh + kh - ph;
                        if (h < 0 || h >= H) continue;
                        for (int ow = 0; ow < OW; ow++) {
                            const int w = ow * sw + kw - pw;
                            if (w >= 0 && w < W)
                                img[((size_t)c * H + h) * W + w] +=
                                    row[(size_t)oh * OW + ow];
                        }
                    }
                }
    }
}

/* conv_ops.cpp:95-122 -- out_n(F, OH*OW) = W(F, CKK) . col_n(CKK, OH*OW). */
void oracle_conv2d_forward(const float *X, const float *Wt, float *out, int N,
                           int C, int H, int W, int F, int KH, int KW, int sh,
                           int sw, int ph, int pw)
{
    const int OH = out_extent(H, ph, KH, sh), OW = out_extent(W, pw, KW, sw);
    const size_t rows = (size_t)C * KH * KW, cols = (size_t)OH * OW;
    float *col = (float *)malloc(sizeof(float) * (size_t)N * rows * cols);
    oracle_im2col_batch(X, col, N, C, H, W, KH, KW, sh, sw, ph, pw);
#pragma omp parallel for schedule(static)
    for (int n = 0; n < N; n++)
        sgemm_rm(ORC_NO_TRANS, ORC_NO_TRANS, F, cols, rows, Wt, rows,
                 col + (size_t)n * rows * cols, cols, 0.0f,
                 out + (size_t)n * F * cols, cols);
    free(col);
}

/* conv_ops.cpp:127-185 -- dW = sum_n dout_n.col_n^T (serial sum in n order);
 * dX = col2im(W^T.dout_n). */
void oracle_conv2d_backward(const float *dout, const float *X, const float *Wt,
                            float *dX, float *dW, int N, int C, int H, int W,
                            int F, int KH, int KW, int sh, int sw, int ph,
                            int pw)
{
    const int OH = out_extent(H, ph, KH, sh), OW = out_extent(W, pw, KW, sw);
    const size_t rows = (size_t)C * KH * KW, cols = (size_t)OH * OW;
    const size_t wsz = (size_t)F * rows;
    float *col = (float *)malloc(sizeof(float) * (size_t)N * rows * cols);
    oracle_im2col_batch(X, col, N, C, H, W, KH, KW, sh, sw, ph, pw);

    float *part = (float *)malloc(sizeof(float) * (size_t)N * wsz);
#pragma omp parallel for schedule(static)
    for (int n = 0; n < N; n++)
        sgemm_rm(ORC_NO_TRANS, ORC_TRANS, F, rows, cols,
                 dout + (size_t)n * F * cols, cols,
                 col + (size_t)n * rows * cols, cols, 0.0f, part + n * wsz,
                 rows);
    memset(dW, 0, sizeof(float) * wsz);
    for (int n = 0; n < N; n++)
        for (size_t i = 0; i < wsz; i++) dW[i] += part[(size_t)n * wsz + i];
    free(part);

    /* Reuse the im2col buffer for dX_col (same shape). */
#pragma omp parallel for schedule(static)
    for (int n = 0; n < N; n++)
        sgemm_rm(ORC_TRANS, ORC_NO_TRANS, rows, cols, F, Wt, rows,
                 dout + (size_t)n * F * cols, cols, 0.0f,
                 col + (size_t)n * rows * cols, cols);
    oracle_col2im_batch(col, dX, N, C, H, W, KH, KW, sh, sw, ph, pw);
    free(col);
}

/* conv_ops.cpp:197-228 -- col_n = W_flat^T.X_n, then col2im with the conv
 * geometry of the (Hout, Wout) output. */
void oracle_conv_transpose2d_fwd(const float *X, const float *Wt, float *out,
                                 int N, int Cin, int H, int W, int Cout,
                                 int KH, int KW, int sh, int sw, int ph,
                                 int pw)
{
    const int Hout = (H - 1) * sh - 2 * ph + KH;
    const int Wout = (W - 1) * sw - 2 * pw + KW;
    const size_t rows = (size_t)Cout * KH * KW, sp = (size_t)H * W;
    float *col = (float *)malloc(sizeof(float) * (size_t)N * rows * sp);
#pragma omp parallel for schedule(static)
    for (int n = 0; n < N; n++)
        sgemm_rm(ORC_TRANS, ORC_NO_TRANS, rows, sp, Cin, Wt, rows,
                 X + (size_t)n * Cin * sp, sp, 0.0f, col + (size_t)n * rows * sp,
                 sp);
    oracle_col2im_batch(col, out, N, Cout, Hout, Wout, KH, KW, sh, sw, ph, pw);
    free(col);
}

/* conv_ops.cpp:233-287 -- col = im2col(dout); dW = sum_n X_n.col_n^T (serial
 * sum); dX_n = W_flat.col_n. */
void oracle_conv_transpose2d_bwd(const float *dout, const float *X,
                                 const float *Wt, float *dX, float *dW, int N,
                                 int Cin, int H, int W, int Cout, int KH,
                                 int KW, int sh, int sw, int ph, int pw)
{
    const int Hout = (H - 1) * sh - 2 * ph + KH;
    const int Wout = (W - 1) * sw - 2 * pw + KW;
    const size_t rows = (size_t)Cout * KH * KW, sp = (size_t)H * W;
    const size_t wsz = (size_t)Cin * rows;
    float *col = (float *)malloc(sizeof(float) * (size_t)N * rows * sp);
    oracle_im2col_batch(dout, col, N, Cout, Hout, Wout, KH, KW, sh, sw, ph, pw);

    float *part = (float *)malloc(sizeof(float) * (size_t)N * wsz);
#pragma omp parallel for schedule(static)
    for (int n = 0; n < N; n++)
        sgemm_rm(ORC_NO_TRANS, ORC_TRANS, Cin, rows, sp,
                 X + (size_t)n * Cin * sp, sp, col + (size_t)n * rows * sp, sp,
                 0.0f, part + n * wsz, rows);
    memset(dW, 0, sizeof(float) * wsz);
    for (int n = 0; n < N; n++)
        for (size_t i = 0; i < wsz; i++) dW[i] += part[(size_t)n * wsz + i];
    free(part);

#pragma omp parallel for schedule(static)
    for (int n = 0; n < N; n++)
        sgemm_rm(ORC_NO_TRANS, ORC_NO_TRANS, Cin, sp, rows, Wt, rows,
                 col + (size_t)n * rows * sp, sp, 0.0f,
                 dX + (size_t)n * Cin * sp, sp);
    free(col);
}
