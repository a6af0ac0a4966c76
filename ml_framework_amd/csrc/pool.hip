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
// Kernel pairs:
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
//   * 3x3 stride 2 padding 1 (W % 4 == 0, 16-byte aligned): 16-byte
//     accesses; the forward writes every mask element once, no clear.
// Indices are 32-bit: the entry points reject tensors above INT_MAX elements.
#include "kernels.h"
#include "runtime.h"

namespace seera {
namespace {

// Unsigned 32-bit division by a divisor fixed at launch, as one multiply-high,
// an add and a shift (Granlund and Montgomery, "Division by Invariant
// Integers using Multiplication", PLDI 1994, section 4): with
// l = ceil(log2 d) and m = floor(2^32 (2^l - d) / d) + 1,
// n / d = (mulhi(n, m) + n) >> l for every 32-bit n (the sum taken in 64
// bits). A generic division costs about 25 VALU instructions per lane, and
// the pool kernels are otherwise memory-bound.
struct FastDiv {
    unsigned d, m, l;
};

FastDiv make_fastdiv(unsigned d) {
    unsigned l = 0;
    while ((1ull << l) < d) ++l;
    const unsigned m = (unsigned)(((1ull << 32) * ((1ull << l) - d)) / d + 1);
    return {d, m, l};
}

__device__ __forceinline__ unsigned fdiv(unsigned n, FastDiv f) {
    return (unsigned)(((unsigned long long)__umulhi(n, f.m) + n) >> f.l);
}

struct PoolGeom {
    int H, W, R, S, ph, pw, sh, sw, Ho, Wo;
    FastDiv dH, dW, dsh, dsw, dHo, dWo;
    FastDiv dW4, dWo2;  // W / 4 and Wo / 2 (the 3x3 stride-2 kernels)
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
    const unsigned t = fdiv(i, g.dWo), wo = i - t * g.Wo;
    const unsigned bc = fdiv(t, g.dHo), ho = t - bc * g.Ho;
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
    const unsigned t = fdiv(i, g.dWo), wo = i - t * g.Wo;
    const unsigned bc = fdiv(t, g.dHo), ho = t - bc * g.Ho;
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

// The cells kernels for 2x2 windows, stride 2, no padding and an even W
// (the reference's MaxPool2D default): every cell row is an aligned pair of
// elements, moved as one 8-byte access. With W even there is no column tail;
// with H odd the last output row's cell has a third row, all outside windows.
__global__ __launch_bounds__(256) void maxpool_fwd_2x2(const float* __restrict__ x,
                                                       float* __restrict__ out,
                                                       int* __restrict__ mask, PoolGeom g,
                                                       unsigned total) {
    const unsigned i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= total) return;
    const unsigned t = fdiv(i, g.dWo), wo = i - t * g.Wo;
    const unsigned bc = fdiv(t, g.dHo), ho = t - bc * g.Ho;
    const unsigned k0 = bc * (unsigned)(g.H * g.W) + 2 * ho * g.W + 2 * wo;
    const float2 a = *reinterpret_cast<const float2*>(x + k0);
    const float2 b = *reinterpret_cast<const float2*>(x + k0 + g.W);
    // Visit order (0,0) (0,1) (1,0) (1,1); the origin is (0,0), so it starts
    // as the argmax and each later element >= the max takes over.
    float best = a.x;
    int arg = 0;
    if (best <= a.y) best = a.y, arg = 1;
    if (best <= b.x) best = b.x, arg = 2;
    if (best <= b.y) best = b.y, arg = 3;
    out[i] = best;
    *reinterpret_cast<int2*>(mask + k0) = make_int2(arg == 0, arg == 1);
    *reinterpret_cast<int2*>(mask + k0 + g.W) = make_int2(arg == 2, arg == 3);
    if ((g.H & 1) && ho == (unsigned)g.Ho - 1)
        *reinterpret_cast<int2*>(mask + k0 + 2 * g.W) = make_int2(0, 0);
}

__global__ __launch_bounds__(256) void maxpool_bwd_2x2(const float* __restrict__ dout,
                                                       const int* __restrict__ mask,
                                                       float* __restrict__ dx, PoolGeom g,
                                                       unsigned total) {
    const unsigned i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= total) return;
    const unsigned t = fdiv(i, g.dWo), wo = i - t * g.Wo;
    const unsigned bc = fdiv(t, g.dHo), ho = t - bc * g.Ho;
    const unsigned k0 = bc * (unsigned)(g.H * g.W) + 2 * ho * g.W + 2 * wo;
    const float d = dout[i];
    const int2 m0 = *reinterpret_cast<const int2*>(mask + k0);
    const int2 m1 = *reinterpret_cast<const int2*>(mask + k0 + g.W);
    *reinterpret_cast<float2*>(dx + k0) =
        make_float2(0.f + d * (float)m0.x, 0.f + d * (float)m0.y);
    *reinterpret_cast<float2*>(dx + k0 + g.W) =
        make_float2(0.f + d * (float)m1.x, 0.f + d * (float)m1.y);
    if ((g.H & 1) && ho == (unsigned)g.Ho - 1)
        *reinterpret_cast<float2*>(dx + k0 + 2 * g.W) = make_float2(0.f, 0.f);
}

__global__ __launch_bounds__(256) void maxpool_fwd_general(const float* __restrict__ x,
                                                           float* __restrict__ out,
                                                           int* __restrict__ mask, PoolGeom g,
                                                           unsigned total) {
    const unsigned i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= total) return;
    const unsigned t = fdiv(i, g.dWo), wo = i - t * g.Wo;
    const unsigned bc = fdiv(t, g.dHo), ho = t - bc * g.Ho;
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

// The general kernels with the window (forward) or the covering-window count
// per axis (backward) fixed at compile time: every load of a thread is issued
// before the first is used. The loop kernels wait for each load in turn,
// which left them bound by memory latency.
template <int RR, int SS>
__global__ __launch_bounds__(256) void maxpool_fwd_general_t(const float* __restrict__ x,
                                                             float* __restrict__ out,
                                                             int* __restrict__ mask, PoolGeom g,
                                                             unsigned total) {
    const unsigned i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= total) return;
    const unsigned t = fdiv(i, g.dWo), wo = i - t * g.Wo;
    const unsigned bc = fdiv(t, g.dHo), ho = t - bc * g.Ho;
    const unsigned plane = bc * (unsigned)(g.H * g.W);
    const float* xp = x + plane;
    const int h0 = (int)ho * g.sh - g.ph, w0 = (int)wo * g.sw - g.pw;
    float v[RR][SS];
    bool ok[RR][SS];
#pragma unroll
    for (int r = 0; r < RR; ++r)
#pragma unroll
        for (int s = 0; s < SS; ++s) {
            const int h = h0 + r, w = w0 + s;
            ok[r][s] = h >= 0 && h < g.H && w >= 0 && w < g.W;
            v[r][s] = ok[r][s] ? xp[h * g.W + w] : 0.f;
        }
    float best = ok[0][0] ? v[0][0] : 0.f;  // the origin, or 0 in the padding
    int arg = -1;
#pragma unroll
    for (int r = 0; r < RR; ++r)
#pragma unroll
        for (int s = 0; s < SS; ++s)
            if (ok[r][s] && best <= v[r][s]) {
                best = v[r][s];
                arg = (h0 + r) * g.W + w0 + s;
            }
    out[i] = best;
    if (arg >= 0) mask[plane + (unsigned)arg] = 1;
}

// MH, MW: the most windows that cover one element along each axis,
// ceil(R / sh) and ceil(S / sw). Candidate windows outside the covering range
// add +0, which leaves the (ho, wo)-ordered sum unchanged (it starts at +0 and
// never becomes -0 under round-to-nearest). Each wave takes 64 columns of one
// input row (grid x: groups of 4 rows of all planes, grid y: 64-column
// tiles), so the row's plane, covering output rows and dout row are
// wave-uniform and only the column arithmetic is per lane.
template <int MH, int MW>
__global__ __launch_bounds__(256) void maxpool_bwd_general_t(const float* __restrict__ dout,
                                                             const int* __restrict__ mask,
                                                             float* __restrict__ dx, PoolGeom g,
                                                             unsigned nrows) {
    const unsigned row = __builtin_amdgcn_readfirstlane(blockIdx.x * 4 + (threadIdx.x >> 6));
    const int w = (int)(blockIdx.y * 64 + (threadIdx.x & 63));
    if (row >= nrows || w >= g.W) return;
    const unsigned bc = fdiv(row, g.dH);
    const int h = (int)(row - bc * g.H);
    const unsigned i = row * (unsigned)g.W + (unsigned)w;
    const float m = (float)mask[i];
    const float* gp = dout + bc * (unsigned)(g.Ho * g.Wo);
    auto lo = [](int num, int den, FastDiv f) {
        return num <= 0 ? 0 : (int)fdiv((unsigned)(num + den - 1), f);
    };
    const int ho0 = lo(h + g.ph - g.R + 1, g.sh, g.dsh);
    const int ho1 = min(g.Ho - 1, (int)fdiv((unsigned)(h + g.ph), g.dsh));
    const int wo0 = lo(w + g.pw - g.S + 1, g.sw, g.dsw);
    const int wo1 = min(g.Wo - 1, (int)fdiv((unsigned)(w + g.pw), g.dsw));
    float term[MH][MW];
#pragma unroll
    for (int a = 0; a < MH; ++a)
#pragma unroll
        for (int c = 0; c < MW; ++c) {
            const int ho = ho1 - (MH - 1) + a, wo = wo1 - (MW - 1) + c;
            term[a][c] = ho >= ho0 && wo >= wo0 ? gp[ho * g.Wo + wo] * m : 0.f;
        }
    float sum = 0.f;
#pragma unroll
    for (int a = 0; a < MH; ++a)
#pragma unroll
        for (int c = 0; c < MW; ++c) sum += term[a][c];
    dx[i] = sum;
}

// 3x3 windows, stride 2, padding 1 (the usual pooling after a stem
// convolution) with W a multiple of 4, in one pass that writes every mask
// element (no clear). A thread owns output pair (ho, 2p, 2p + 1) for the
// output rows ho of a segment [ha, hb) of kSegRows rows, and the mask of input
// columns 4p .. 4p + 3 in rows 2ho and 2ho + 1. Column 4p + j is covered by
// windows wo = 2p + k with j = 2k - 1 + s (s the column in the window), so the
// thread evaluates windows 2p, 2p + 1 and, for the mask only, 2p + 2 (input
// columns 4p - 1 .. 4p + 5: one 4-byte, one 16-byte and one 8-byte load per
// row). Row 2ho is covered by window row ho alone and row 2ho + 1 also by
// ho + 1, so the thread walks down its segment carrying the previous window
// row's argmaxes and evaluates window row hb as well when it exists (for the
// mask of row 2hb - 1, not stored). An element is 1 when it is the argmax of
// any window, the outcome the clear-and-mark kernels give; each window keeps
// their visit order and tie rule, so out and mask are the same bits. Wo = W / 2
// is even, so the pair is whole.
constexpr int kSegRows = 7;

__global__ __launch_bounds__(256) void maxpool_fwd_3x3s2p1(const float* __restrict__ x,
                                                           float* __restrict__ out,
                                                           int* __restrict__ mask, PoolGeom g,
                                                           FastDiv dseg, unsigned nthreads) {
    const unsigned i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= nthreads) return;
    const unsigned np = (unsigned)(g.W / 4);
    const unsigned t = fdiv(i, g.dW4), pp = i - t * np;
    const unsigned bc = fdiv(t, dseg), seg = t - bc * dseg.d;
    const unsigned plane = bc * (unsigned)(g.H * g.W);
    const float* xp = x + plane;
    int* mp = mask + plane;
    float* op = out + bc * (unsigned)(g.Ho * g.Wo) + 2 * pp;
    const int c0 = 4 * (int)pp;
    const bool has2 = c0 + 4 < g.W;  // window 2p + 2 exists
    const int ha = (int)seg * kSegRows, hb = min(ha + kSegRows, g.Ho);
    // Input row h at columns c0 - 1 .. c0 + 5 (zeros outside the image).
    auto load_row = [&](int h, float (&v)[7], bool& ok) {
        ok = h >= 0 && h < g.H;
        const float* row = xp + h * g.W;
        const float4 q = ok ? *reinterpret_cast<const float4*>(row + c0)
                            : make_float4(0.f, 0.f, 0.f, 0.f);
        const float2 e = ok && has2 ? *reinterpret_cast<const float2*>(row + c0 + 4)
                                    : make_float2(0.f, 0.f);
        v[0] = ok && c0 > 0 ? row[c0 - 1] : 0.f;
        v[1] = q.x; v[2] = q.y; v[3] = q.z; v[4] = q.w;
        v[5] = e.x; v[6] = e.y;
    };
    float rv[3][7];
    bool okr[3];
    load_row(2 * ha - 1, rv[0], okr[0]);
    // Window row ho's argmax (3 r + s, or -1) for windows 2p + k.
    int prev[3] = {-1, -1, -1};
    // Mask bits of the thread's 4 columns from window arg a's row r.
    auto mark = [](const int (&a)[3], int r, int (&m)[4]) {
#pragma unroll
        for (int k = 0; k < 3; ++k)
#pragma unroll
            for (int s = 0; s < 3; ++s) {
                const int j = 2 * k - 1 + s;
                if (j >= 0 && j < 4 && a[k] == 3 * r + s) m[j] = 1;
            }
    };
    auto store_mask = [&](int h, const int (&m)[4]) {
        if (h < g.H)
            *reinterpret_cast<int4*>(mp + h * g.W + c0) = make_int4(m[0], m[1], m[2], m[3]);
    };
    const int hend = hb < g.Ho ? hb : hb - 1;
    for (int ho = ha; ho <= hend; ++ho) {
        load_row(2 * ho, rv[1], okr[1]);
        load_row(2 * ho + 1, rv[2], okr[2]);
        int cur[3];
        float best[2];
#pragma unroll
        for (int k = 0; k < 3; ++k) {
            const int w0 = c0 - 1 + 2 * k;  // window's first column
            float b = okr[0] && w0 >= 0 ? rv[0][2 * k] : 0.f;  // the origin, or 0 in the padding
            int arg = -1;
#pragma unroll
            for (int r = 0; r < 3; ++r)
#pragma unroll
                for (int s = 0; s < 3; ++s)
                    if (okr[r] && w0 + s >= 0 && b <= rv[r][2 * k + s]) {
                        b = rv[r][2 * k + s];
                        arg = 3 * r + s;
                    }
            if (k < 2) best[k] = b;
            cur[k] = k < 2 || has2 ? arg : -1;
        }
        if (ho < hb) *reinterpret_cast<float2*>(op + ho * g.Wo) = make_float2(best[0], best[1]);
        if (ho > ha) {
            // rows 2(ho - 1) (window row ho - 1) and 2ho - 1 (ho - 1 and ho)
            int m0[4] = {0, 0, 0, 0}, m1[4] = {0, 0, 0, 0};
            mark(prev, 1, m0);
            mark(prev, 2, m1);
            mark(cur, 0, m1);
            store_mask(2 * ho - 2, m0);
            store_mask(2 * ho - 1, m1);
        }
#pragma unroll
        for (int k = 0; k < 3; ++k) prev[k] = cur[k];
#pragma unroll
        for (int q = 0; q < 7; ++q) rv[0][q] = rv[2][q];
        okr[0] = okr[2];
    }
    if (hb == g.Ho) {
        // the plane's last window row: rows 2(Ho - 1) and 2Ho - 1 (if < H)
        int m0[4] = {0, 0, 0, 0}, m1[4] = {0, 0, 0, 0};
        mark(prev, 1, m0);
        mark(prev, 2, m1);
        store_mask(2 * g.Ho - 2, m0);
        store_mask(2 * g.Ho - 1, m1);
    }
}

// Its backward: one thread per 4 columns 4q .. 4q + 3 of an input row. Row h
// lies in windows ho = h / 2 .. min(Ho - 1, (h + 1) / 2); column 4q + c in
// windows wo = 2q + o0[c] .. min(Wo - 1, 2q + o1[c]), o0 = (0, 0, 1, 1),
// o1 = (0, 1, 1, 2). The terms are added in (ho, wo) order as in the general
// kernel: the same bits with one 16-byte mask load, 6 dout loads and one
// 16-byte store per 4 elements.
__global__ __launch_bounds__(256) void maxpool_bwd_3x3s2p1(const float* __restrict__ dout,
                                                           const int* __restrict__ mask,
                                                           float* __restrict__ dx, PoolGeom g,
                                                           unsigned nquads) {
    const unsigned i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= nquads) return;
    const unsigned t = fdiv(i, g.dW4), q = i - t * (unsigned)(g.W / 4);  // t: plane row
    const unsigned bc = fdiv(t, g.dH);
    const int h = (int)(t - bc * g.H);
    const unsigned e = t * (unsigned)g.W + 4 * q;
    const int4 mk = *reinterpret_cast<const int4*>(mask + e);
    const float m[4] = {(float)mk.x, (float)mk.y, (float)mk.z, (float)mk.w};
    const float* gp = dout + bc * (unsigned)(g.Ho * g.Wo);
    const int ho_lo = h >> 1, ho_hi = min(g.Ho - 1, (h + 1) >> 1);
    const int wb = 2 * (int)q, wlim = g.Wo - 1;
    float d[2][3];
#pragma unroll
    for (int a = 0; a < 2; ++a)
#pragma unroll
        for (int j = 0; j < 3; ++j)
            d[a][j] = ho_lo + a <= ho_hi && wb + j <= wlim ? gp[(ho_lo + a) * g.Wo + wb + j] : 0.f;
    constexpr int o0[4] = {0, 0, 1, 1}, o1[4] = {0, 1, 1, 2};
    float r[4];
#pragma unroll
    for (int c = 0; c < 4; ++c) {
        float sum = 0.f;
#pragma unroll
        for (int a = 0; a < 2; ++a)
#pragma unroll
            for (int j = o0[c]; j <= o1[c]; ++j)
                if (ho_lo + a <= ho_hi && wb + j <= wlim) sum += d[a][j] * m[c];
        r[c] = sum;
    }
    *reinterpret_cast<float4*>(dx + e) = make_float4(r[0], r[1], r[2], r[3]);
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
    const unsigned t = fdiv(i, g.dW), bc = fdiv(t, g.dH);
    const int w = (int)(i - t * g.W), h = (int)(t - bc * g.H);
    const float* gp = dout + bc * (unsigned)(g.Ho * g.Wo);
    // ceil(num / den) for num > 0, else 0; num + den - 1 < 2^22 here.
    auto lo = [](int num, int den, FastDiv f) {
        return num <= 0 ? 0 : (int)fdiv((unsigned)(num + den - 1), f);
    };
    const int ho0 = lo(h + g.ph - g.R + 1, g.sh, g.dsh);
    const int ho1 = min(g.Ho - 1, (int)fdiv((unsigned)(h + g.ph), g.dsh));
    const int wo0 = lo(w + g.pw - g.S + 1, g.sw, g.dsw);
    const int wo1 = min(g.Wo - 1, (int)fdiv((unsigned)(w + g.pw), g.dsw));
    float sum = 0.f;
    for (int ho = ho0; ho <= ho1; ++ho)
        for (int wo = wo0; wo <= wo1; ++wo) sum += gp[ho * g.Wo + wo] * m;
    dx[i] = sum;
}

PoolGeom geom(int H, int W, int R, int S, int ph, int pw, int sh, int sw) {
    const int Ho = (H + 2 * ph - R) / sh + 1, Wo = (W + 2 * pw - S) / sw + 1;
    return {H, W, R, S, ph, pw, sh, sw, Ho, Wo,
            make_fastdiv(H), make_fastdiv(W), make_fastdiv(sh), make_fastdiv(sw),
            make_fastdiv(Ho), make_fastdiv(Wo),
            make_fastdiv((unsigned)std::max(W / 4, 1)), make_fastdiv((unsigned)std::max(Wo / 2, 1))};
}

unsigned blocks(unsigned n) { return (n + 255u) / 256u; }

template <int MH, int MW>
void launch_bwd_t(const float* dout, const int* mask, float* dx, const PoolGeom& g, unsigned n,
                  hipStream_t st) {
    const unsigned nrows = n / (unsigned)g.W;  // B * C * H
    hipLaunchKernelGGL((maxpool_bwd_general_t<MH, MW>),
                       dim3((nrows + 3) / 4, (unsigned)((g.W + 63) / 64)), dim3(256), 0, st, dout,
                       mask, dx, g, nrows);
}

template <int MH>
void launch_bwd_mw(int mw, const float* dout, const int* mask, float* dx, const PoolGeom& g,
                   unsigned n, hipStream_t st) {
    if (mw == 1) launch_bwd_t<MH, 1>(dout, mask, dx, g, n, st);
    else if (mw == 2) launch_bwd_t<MH, 2>(dout, mask, dx, g, n, st);
    else launch_bwd_t<MH, 3>(dout, mask, dx, g, n, st);
}

int launch_bwd_general(const float* dout, const int* mask, float* dx, const PoolGeom& g,
                       unsigned n, hipStream_t st) {
    const int mh = (g.R + g.sh - 1) / g.sh, mw = (g.S + g.sw - 1) / g.sw;
    if (mh > 3 || mw > 3)
        hipLaunchKernelGGL(maxpool_bwd_general, dim3(blocks(n)), dim3(256), 0, st, dout, mask,
                           dx, g, n);
    else if (mh == 1) launch_bwd_mw<1>(mw, dout, mask, dx, g, n, st);
    else if (mh == 2) launch_bwd_mw<2>(mw, dout, mask, dx, g, n, st);
    else launch_bwd_mw<3>(mw, dout, mask, dx, g, n, st);
    SEERA_HIP_TRY(hipGetLastError());
    return SEERA_OK;
}

bool s2p1_path(int R, int S, int ph, int pw, int sh, int sw, int W, const void* p0, const void* p1,
               const void* p2) {
    return R == 3 && S == 3 && sh == 2 && sw == 2 && ph == 1 && pw == 1 && W % 4 == 0 && W > 0 &&
           ((uintptr_t)p0 | (uintptr_t)p1 | (uintptr_t)p2) % 16 == 0;
}

bool pair_path(int R, int S, int ph, int pw, int sh, int sw, int W, const void* p0, const void* p1) {
    return R == 2 && S == 2 && sh == 2 && sw == 2 && ph == 0 && pw == 0 && W % 2 == 0 &&
           ((uintptr_t)p0 | (uintptr_t)p1) % 8 == 0;
}

}  // namespace

int maxpool_fwd(const float* x, float* out, int* mask, int B, int C, int H, int W, int R, int S,
                int ph, int pw, int sh, int sw, hipStream_t st) {
    const PoolGeom g = geom(H, W, R, S, ph, pw, sh, sw);
    const unsigned nin = (unsigned)B * C * H * W, nout = (unsigned)B * C * g.Ho * g.Wo;
    if (nout == 0) return SEERA_OK;
    if (pair_path(R, S, ph, pw, sh, sw, W, x, mask)) {
        hipLaunchKernelGGL(maxpool_fwd_2x2, dim3(blocks(nout)), dim3(256), 0, st, x, out, mask,
                           g, nout);
    } else if (sh >= R && sw >= S) {
        hipLaunchKernelGGL(maxpool_fwd_cells, dim3(blocks(nout)), dim3(256), 0, st, x, out, mask,
                           g, nout);
    } else if (s2p1_path(R, S, ph, pw, sh, sw, W, x, mask, out)) {
        const unsigned nseg = (unsigned)((g.Ho + kSegRows - 1) / kSegRows);
        const unsigned nt = (unsigned)B * C * nseg * (unsigned)(W / 4);
        hipLaunchKernelGGL(maxpool_fwd_3x3s2p1, dim3(blocks(nt)), dim3(256), 0, st, x, out, mask,
                           g, make_fastdiv(nseg), nt);
    } else {
        // Clear with a kernel (all-zero bits are int 0), not a memset node,
        // so that the call can be captured into a graph.
        SEERA_TRY(fill_f32(reinterpret_cast<float*>(mask), 0.f, (size_t)nin, st));
        if (R == 2 && S == 2)
            hipLaunchKernelGGL((maxpool_fwd_general_t<2, 2>), dim3(blocks(nout)), dim3(256), 0,
                               st, x, out, mask, g, nout);
        else if (R == 3 && S == 3)
            hipLaunchKernelGGL((maxpool_fwd_general_t<3, 3>), dim3(blocks(nout)), dim3(256), 0,
                               st, x, out, mask, g, nout);
        else
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
    if (pair_path(R, S, ph, pw, sh, sw, W, mask, dx))
        hipLaunchKernelGGL(maxpool_bwd_2x2, dim3(blocks(nout)), dim3(256), 0, st, dout, mask, dx,
                           g, nout);
    else if (sh >= R && sw >= S)
        hipLaunchKernelGGL(maxpool_bwd_cells, dim3(blocks(nout)), dim3(256), 0, st, dout, mask,
                           dx, g, nout);
    else if (s2p1_path(R, S, ph, pw, sh, sw, W, mask, dx, mask))
        hipLaunchKernelGGL(maxpool_bwd_3x3s2p1, dim3(blocks(nin / 4)), dim3(256), 0, st, dout,
                           mask, dx, g, nin / 4);
    else
        SEERA_TRY(launch_bwd_general(dout, mask, dx, g, nin, st));
    SEERA_HIP_TRY(hipGetLastError());
    return SEERA_OK;
}

}  // namespace seera
