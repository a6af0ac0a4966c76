// pool.hip -- MaxPool2D forward / backward with the reference GPU engine's
// semantics (engine_cuda/src/maxPool.cu:9-77, bindings cuda_bindings.cpp:
// 337-351), the layer next to the convolutions in every CNN it trains.
//
// Forward, per output (b, c, ho, wo), window rows ho*sh - ph + r, columns
// wo*sw - pw + s (r < R, s < S):
//   * the running max starts at the window origin's value, or at 0 when the
//     origin lies in the padding (maxPool.cu:16-26);
//   * in-window elements are visited row by row; an element >= the running
//     max replaces it and becomes the argmax (ties go to the later element,
//     maxPool.cu:29-40); padding is skipped;
//   * mask [B, C, H, W] (int32) is 1 at an argmax and 0 elsewhere.
// The reference writes 0 to an element when it loses a comparison and 1 to
// the winner, from one thread per window with no ordering between windows;
// where windows overlap, an element that wins one window and loses another
// ends up 0 or 1 depending on the schedule. Here it is 1 (the outcome where
// every window's writes of 0 precede the writes of 1), so the result is
// deterministic. When the origin is in the padding and no in-window element
// reaches 0, the reference marks the origin itself -- an address outside the
// tensor or inside a neighbouring row; here no element is marked.
//
// Backward (maxPool.cu:56-77): dX[i] = sum over every window that covers i of
// dout * mask[i], the windows in (ho, wo) order, starting from +0; the
// reference adds the same terms with atomics, in any order.
//
// Two kernel pairs:
//   * cells (stride >= window on both axes, e.g. the usual 2x2 stride 2):
//     windows do not overlap, so the plane splits into one cell per output --
//     rows [ho*sh - ph, (ho+1)*sh - ph), the last output row also taking the
//     rows below, columns likewise, clipped to the image -- that holds its
//     window. One thread per output reads its cell once and writes every
//     mask (forward) or dX (backward) element of it: a single pass with no
//     mask clear, each byte of x, out, mask, dout and dX moved once.
//   * general (overlapping windows): the forward clears the mask and marks
//     argmaxes from one thread per output; the backward gathers, one thread
//     per input element, over the covering windows.
// Indices are 32-bit: the entry points reject tensors above INT_MAX elements.
#include "kernels.h"
#include "runtime.h"

namespace seera {
namespace {

struct PoolGeom {
    int H, W, R, S, ph, pw, sh, sw, Ho, Wo;
};

// Cell of output index o along one axis: [lo, hi) of the input, clipped.
__device__ __forceinline__ void cell_range(int o, int n_out, int stride, int pad, int n_in,
                                           int& lo, int& hi) {
    lo = max(o * stride - pad, 0);
    hi = o == n_out - 1 ? n_in : min((o + 1) * stride - pad, n_in);
}

__global__ __launch_bounds__(256) void maxpool_fwd_cells(const float* __restrict__ x,
                                                         float* __restrict__ out,
                                                         int* __restrict__ mask, PoolGeom g,
                                                         unsigned total) {
    const unsigned i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= total) return;
    const unsigned wo = i % g.Wo, t = i / g.Wo;
    const unsigned ho = t % g.Ho, bc = t / g.Ho;
    const unsigned plane = bc * (unsigned)(g.H * g.W);
    const float* xp = x + plane;
    int* mp = mask + plane;
    const int h0 = (int)ho * g.sh - g.ph, w0 = (int)wo * g.sw - g.pw;
    const bool origin_in = h0 >= 0 && h0 < g.H && w0 >= 0 && w0 < g.W;
    float best = origin_in ? xp[h0 * g.W + w0] : 0.f;
    int arg = -1;
    const int wr0 = max(h0, 0), wr1 = min(h0 + g.R, g.H);
    const int wc0 = max(w0, 0), wc1 = min(w0 + g.S, g.W);
    for (int h = wr0; h < wr1; ++h)
        for (int w = wc0; w < wc1; ++w) {
            const float v = xp[h * g.W + w];
            if (best <= v) {
                best = v;
                arg = h * g.W + w;
            }
        }
    out[i] = best;
    int r0, r1, c0, c1;
    cell_range((int)ho, g.Ho, g.sh, g.ph, g.H, r0, r1);
    cell_range((int)wo, g.Wo, g.sw, g.pw, g.W, c0, c1);
    for (int h = r0; h < r1; ++h)
        for (int w = c0; w < c1; ++w) mp[h * g.W + w] = (h * g.W + w) == arg ? 1 : 0;
}

__global__ __launch_bounds__(256) void maxpool_bwd_cells(const float* __restrict__ dout,
                                                         const int* __restrict__ mask,
                                                         float* __restrict__ dx, PoolGeom g,
                                                         unsigned total) {
    const unsigned i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= total) return;
    const unsigned wo = i % g.Wo, t = i / g.Wo;
    const unsigned ho = t % g.Ho, bc = t / g.Ho;
    const unsigned plane = bc * (unsigned)(g.H * g.W);
    const int* mp = mask + plane;
    float* dp = dx + plane;
    const float d = dout[i];
    const int h0 = (int)ho * g.sh - g.ph, w0 = (int)wo * g.sw - g.pw;
    int r0, r1, c0, c1;
    cell_range((int)ho, g.Ho, g.sh, g.ph, g.H, r0, r1);
    cell_range((int)wo, g.Wo, g.sw, g.pw, g.W, c0, c1);
    for (int h = r0; h < r1; ++h) {
        const bool row_in = h >= h0 && h < h0 + g.R;
        for (int w = c0; w < c1; ++w) {
            const int k = h * g.W + w;
            // One covering window (0 + term) or none (0). The mask is read
            // in both cases, as the general kernel does.
            const float m = (float)mp[k];
            const bool in = row_in && w >= w0 && w < w0 + g.S;
            dp[k] = in ? 0.f + d * m : 0.f;
        }
    }
}

__global__ __launch_bounds__(256) void maxpool_fwd_general(const float* __restrict__ x,
                                                           float* __restrict__ out,
                                                           int* __restrict__ mask, PoolGeom g,
                                                           unsigned total) {
    const unsigned i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= total) return;
    const unsigned wo = i % g.Wo, t = i / g.Wo;
    const unsigned ho = t % g.Ho, bc = t / g.Ho;
    const unsigned plane = bc * (unsigned)(g.H * g.W);
    const float* xp = x + plane;
    const int h0 = (int)ho * g.sh - g.ph, w0 = (int)wo * g.sw - g.pw;
    const bool origin_in = h0 >= 0 && h0 < g.H && w0 >= 0 && w0 < g.W;
    float best = origin_in ? xp[h0 * g.W + w0] : 0.f;
    int arg = -1;
    const int wr0 = max(h0, 0), wr1 = min(h0 + g.R, g.H);
    const int wc0 = max(w0, 0), wc1 = min(w0 + g.S, g.W);
    for (int h = wr0; h < wr1; ++h)
        for (int w = wc0; w < wc1; ++w) {
            const float v = xp[h * g.W + w];
            if (best <= v) {
                best = v;
                arg = h * g.W + w;
            }
        }
    out[i] = best;
    // Several windows may mark the same element; they all store 1.
    if (arg >= 0) mask[plane + (unsigned)arg] = 1;
}

// One thread per input element: the windows covering row h are
// ho in [ceil((h + ph - R + 1) / sh), floor((h + ph) / sh)] within [0, Ho).
__global__ __launch_bounds__(256) void maxpool_bwd_general(const float* __restrict__ dout,
                                                           const int* __restrict__ mask,
                                                           float* __restrict__ dx, PoolGeom g,
                                                           unsigned total) {
    const unsigned i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= total) return;
    // The reference's terms dout * (float)mask: for a 0 mask they still turn
    // a non-finite dout into NaN.
    const float m = (float)mask[i];
    const int w = (int)(i % g.W);
    const unsigned t = i / g.W;
    const int h = (int)(t % g.H);
    const unsigned bc = t / g.H;
    const float* gp = dout + bc * (unsigned)(g.Ho * g.Wo);
    auto lo = [](int num, int den) { return num <= 0 ? 0 : (num + den - 1) / den; };
    const int ho0 = lo(h + g.ph - g.R + 1, g.sh), ho1 = min(g.Ho - 1, (h + g.ph) / g.sh);
    const int wo0 = lo(w + g.pw - g.S + 1, g.sw), wo1 = min(g.Wo - 1, (w + g.pw) / g.sw);
    float sum = 0.f;
    for (int ho = ho0; ho <= ho1; ++ho)
        for (int wo = wo0; wo <= wo1; ++wo) sum += gp[ho * g.Wo + wo] * m;
    dx[i] = sum;
}

PoolGeom geom(int H, int W, int R, int S, int ph, int pw, int sh, int sw) {
    return {H, W, R, S, ph, pw, sh, sw, (H + 2 * ph - R) / sh + 1, (W + 2 * pw - S) / sw + 1};
}

unsigned blocks(unsigned n) { return (n + 255u) / 256u; }

}  // namespace

int maxpool_fwd(const float* x, float* out, int* mask, int B, int C, int H, int W, int R, int S,
                int ph, int pw, int sh, int sw, hipStream_t st) {
    const PoolGeom g = geom(H, W, R, S, ph, pw, sh, sw);
    const unsigned nin = (unsigned)B * C * H * W, nout = (unsigned)B * C * g.Ho * g.Wo;
    if (nout == 0) return SEERA_OK;
    if (sh >= R && sw >= S) {
        hipLaunchKernelGGL(maxpool_fwd_cells, dim3(blocks(nout)), dim3(256), 0, st, x, out, mask,
                           g, nout);
    } else {
        SEERA_HIP_TRY(hipMemsetAsync(mask, 0, sizeof(int) * (size_t)nin, st));
        hipLaunchKernelGGL(maxpool_fwd_general, dim3(blocks(nout)), dim3(256), 0, st, x, out,
                           mask, g, nout);
    }
    SEERA_HIP_TRY(hipGetLastError());
    return SEERA_OK;
}

int maxpool_bwd(const float* dout, const int* mask, float* dx, int B, int C, int H, int W, int R,
                int S, int ph, int pw, int sh, int sw, hipStream_t st) {
    const PoolGeom g = geom(H, W, R, S, ph, pw, sh, sw);
    const unsigned nin = (unsigned)B * C * H * W, nout = (unsigned)B * C * g.Ho * g.Wo;
    if (nin == 0) return SEERA_OK;
    if (sh >= R && sw >= S)
        hipLaunchKernelGGL(maxpool_bwd_cells, dim3(blocks(nout)), dim3(256), 0, st, dout, mask,
                           dx, g, nout);
    else
        hipLaunchKernelGGL(maxpool_bwd_general, dim3(blocks(nin)), dim3(256), 0, st, dout, mask,
                           dx, g, nin);
    SEERA_HIP_TRY(hipGetLastError());
    return SEERA_OK;
}

}  // namespace seera
