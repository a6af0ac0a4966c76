// conv.hip -- Conv2D and ConvTranspose2D forward/backward as implicit GEMMs on
// the fp16 MFMA tile engine, with im2col / col2im folded into the operand
// gathers (no column buffer in HBM, no atomics).
//
// Reference: engine_cuda/src/convolution.cu and upsampling.cu. The eight
// reference passes reduce to three GEMM shapes:
//   forward  out[b,f,p] = sum_{c,r,s} W[f,c,r,s] X[b,c, ho*sh-ph+r, wo*sw-pw+s]
//            = conv2d fwd (convolution.cu:15-101, 367-389)
//            = convT dX    (upsampling.cu:128-197, 337-346; W read [Cin,Cout,..])
//   dgrad    out[b,c,h,w] = sum_{f,r,s} W[f,c,r,s] Y[b,f,(h+ph-r)/sh,(w+pw-s)/sw]
//            (only taps where the division is exact and in range)
//            = conv2d dX   (convolution.cu:144-265, 401-429)
//            = convT fwd   (upsampling.cu:15-126, 376-401)
//   wgrad    dW[f,c,r,s] = sum_{b,ho,wo} Y[b,f,ho,wo] X[b,c,ho*sh-ph+r,wo*sw-pw+s]
//            = conv2d dW   (convolution.cu:268-366, 431-452)
//            = convT dW    (upsampling.cu:202-301, 354-374; roles of X, dY swapped)
#include "conv_band.h"
#include "gather.h"
#include "kernels.h"
#include "plan.h"

namespace seera {
namespace {

constexpr int kFar = 1 << 29;  // offset that fails every bounds test

// Forward im2col gather: rows are output pixels q = (b, ho, wo), k = (c, r, s)
// over the [B, C, H, W] input X.
struct FwdGather {
    const float* X;
    int C, H, W, R, S, Wo, HWo, sh, sw, ph, pw, npix;
    struct Row {
        int64_t base;
        int h0, w0;
    };
    struct Kin {
        int64_t coff;
        int r, s;
    };
    __device__ __forceinline__ Row row_info(int q) const {
        if (q >= npix) return {0, -kFar, -kFar};
        const int b = q / HWo, p = q - b * HWo;
        const int ho = p / Wo, wo = p - ho * Wo;
        return {(int64_t)b * C * H * W, ho * sh - ph, wo * sw - pw};
    }
    __device__ __forceinline__ Kin k_info(int k, int kmax) const {
        if (k >= kmax) return {0, -kFar, -kFar};
        const int rs = R * S;
        const int c = k / rs, t = k - c * rs;
        const int r = t / S;
        return {(int64_t)c * H * W, r, t - r * S};
    }
    __device__ __forceinline__ float fetch(const Row& ro, const Kin& ki) const {
        const int h = ro.h0 + ki.r, w = ro.w0 + ki.s;
        if ((unsigned)h < (unsigned)H && (unsigned)w < (unsigned)W)
            return X[ro.base + ki.coff + (int64_t)h * W + w];
        return 0.f;
    }
};

// Transposed gather: rows are output pixels (b, h, w) of the [B, Cout, Hd, Wd]
// result, k = (f, r, s) over the [B, F, Hi, Wi] input Y.
struct DgradGather {
    const float* Y;
    int F, Hi, Wi, R, S, Wd, HWd, sh, sw, ph, pw, npix;
    struct Row {
        int64_t base;
        int hp, wp;
    };
    struct Kin {
        int64_t foff;
        int r, s;
    };
    __device__ __forceinline__ Row row_info(int q) const {
        if (q >= npix) return {0, -kFar, -kFar};
        const int b = q / HWd, p = q - b * HWd;
        const int h = p / Wd, w = p - h * Wd;
        return {(int64_t)b * F * Hi * Wi, h + ph, w + pw};
    }
    __device__ __forceinline__ Kin k_info(int k, int kmax) const {
        if (k >= kmax) return {0, kFar, kFar};
        const int rs = R * S;
        const int f = k / rs, t = k - f * rs;
        const int r = t / S;
        return {(int64_t)f * Hi * Wi, r, t - r * S};
    }
    __device__ __forceinline__ float fetch(const Row& ro, const Kin& ki) const {
        const int hn = ro.hp - ki.r, wn = ro.wp - ki.s;
        if (hn < 0 || wn < 0) return 0.f;
        const int hi = hn / sh, wi = wn / sw;
        if (hi * sh != hn || wi * sw != wn || hi >= Hi || wi >= Wi) return 0.f;
        return Y[ro.base + ki.foff + (int64_t)hi * Wi + wi];
    }
};

// Weight-gradient A operand: rows f, k = pixel q = (b, p) of Y [B, F, HWo].
struct WgradYGather {
    const float* Y;
    int F, HWo;
    struct Row {
        int64_t foff;  // -1: row outside [0, F)
    };
    struct Kin {
        int64_t off;  // -1: k outside the slice
    };
    __device__ __forceinline__ Row row_info(int f) const { return {f < F ? (int64_t)f * HWo : -1}; }
    __device__ __forceinline__ Kin k_info(int q, int kmax) const {
        if (q >= kmax) return {-1};
        const int b = q / HWo;
        return {(int64_t)b * F * HWo + (q - b * HWo)};
    }
    __device__ __forceinline__ float fetch(const Row& ro, const Kin& ki) const {
        return (ro.foff >= 0 && ki.off >= 0) ? Y[ro.foff + ki.off] : 0.f;
    }
};

// Weight-gradient B operand: rows (c, r, s), k = output pixel q = (b, ho, wo);
// element X[b, c, ho*sh-ph+r, wo*sw-pw+s].
struct WgradXGather {
    const float* X;
    int C, H, W, R, S, Wo, HWo, sh, sw, ph, pw, crs;
    struct Row {
        int64_t coff;
        int r, s;
    };
    struct Kin {
        int64_t base;
        int h0, w0;
    };
    __device__ __forceinline__ Row row_info(int row) const {
        if (row >= crs) return {0, -kFar, -kFar};
        const int rs = R * S;
        const int c = row / rs, t = row - c * rs;
        const int r = t / S;
        return {(int64_t)c * H * W, r, t - r * S};
    }
    __device__ __forceinline__ Kin k_info(int q, int kmax) const {
        if (q >= kmax) return {0, -kFar, -kFar};
        const int b = q / HWo, p = q - b * HWo;
        const int ho = p / Wo, wo = p - ho * Wo;
        return {(int64_t)b * C * H * W, ho * sh - ph, wo * sw - pw};
    }
    __device__ __forceinline__ float fetch(const Row& ro, const Kin& ki) const {
        const int h = ki.h0 + ro.r, w = ki.w0 + ro.s;
        if ((unsigned)h < (unsigned)H && (unsigned)w < (unsigned)W)
            return X[ki.base + ro.coff + (int64_t)h * W + w];
        return 0.f;
    }
};

// out[b, m, p] = sum_k Wm[m, k] * G(q = b*HW + p, k): the weights are a
// row-major [M, K] matrix, the other operand a pixel gather, and the result an
// NCHW tensor with M channels and HW pixels per image.
template <int VA, class G>
struct PixelProblem {
    const float* Wm;
    int64_t ldw;
    G g;
    float* C;
    int out_hw;
    int M, N, K;
    int64_t ldc, split_stride;  // unused: this problem is never split
    int tiles_n, k_split, gm;
    ConvEpi epi;                // forward only: bias [M] and activation

    template <int R, int BK, int NT>
    using SA = StageKC<R, BK, NT, VA>;
    template <int R, int BK, int NT>
    using SB = StageGatherMN<R, BK, NT, G>;

    template <class S>
    __device__ __forceinline__ void init_a(S&, int, int) const {}
    template <class S>
    __device__ __forceinline__ void init_b(S& s, int n0, int tid) const { s.init(g, n0, tid); }
    template <class S>
    __device__ __forceinline__ void load_a(S& s, int m0, int k0, int k1, int tid) const {
        s.load(Wm, ldw, m0, M, k0, k1, tid);
    }
    template <class S>
    __device__ __forceinline__ void load_b(S& s, int, int k0, int k1, int tid) const {
        s.load(g, k0, k1, tid);
    }
    __device__ __forceinline__ void store(int m, int n, int, float v) const {
        const int b = n / out_hw;
        const int64_t i = ((int64_t)b * M + m) * out_hw + (n - b * out_hw);
        if (epi.bias || epi.act)
            epilogue(C + i, epi.mask ? epi.mask + i : nullptr, v, epi.bias ? epi.bias[m] : 0.f,
                     epi.act);
        else
            C[i] = v;
    }
};

// dW[m, n] = sum_q Yg(m, q) * Xg(n, q), row-major output, split over q.
struct WgradProblem {
    WgradYGather ga;
    WgradXGather gb;
    float* C;
    int M, N, K;
    int64_t ldc, split_stride;
    int tiles_n, k_split, gm;

    template <int R, int BK, int NT>
    using SA = StageGatherKC<R, BK, NT, WgradYGather>;
    template <int R, int BK, int NT>
    using SB = StageGatherKC<R, BK, NT, WgradXGather>;

    template <class S>
    __device__ __forceinline__ void init_a(S& s, int m0, int tid) const { s.init(ga, m0, tid); }
    template <class S>
    __device__ __forceinline__ void init_b(S& s, int n0, int tid) const { s.init(gb, n0, tid); }
    template <class S>
    __device__ __forceinline__ void load_a(S& s, int, int k0, int k1, int tid) const {
        s.load(ga, k0, k1, tid);
    }
    template <class S>
    __device__ __forceinline__ void load_b(S& s, int, int k0, int k1, int tid) const {
        s.load(gb, k0, k1, tid);
    }
    __device__ __forceinline__ void store(int m, int n, int z, float v) const {
        C[z * split_stride + (int64_t)m * ldc + n] = v;
    }
};

// Wt[c, f*RS + t] = W[f, c, t]: the [F, C, R, S] weight re-laid out as a
// row-major [C, F*R*S] matrix for the dgrad GEMM.
__global__ void relayout_dgrad_weight(const float* __restrict__ W, float* __restrict__ Wt, int F,
                                      int C, int RS) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    const int64_t n = (int64_t)F * C * RS;
    if (i >= n) return;
    const int t = (int)(i % RS);
    const int64_t fc = i / RS;
    const int c = (int)(fc % C), f = (int)(fc / C);
    Wt[((int64_t)c * F + f) * RS + t] = W[i];
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

// out [rows, Wp] = in [rows, W] with zeros in columns W..Wp-1 (Wp % 4 == 0):
// a copy whose rows are float4-aligned for the band and row-streaming kernels.
__global__ __launch_bounds__(256) void widen_rows(const float* __restrict__ in,
                                                  float* __restrict__ out, int64_t rows, int W,
                                                  int Wp) {
    const int nq = Wp >> 2;
    const int64_t n = rows * nq;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
         i += (int64_t)gridDim.x * blockDim.x) {
        const int64_t row = i / nq;
        const int c0 = (int)(i - row * nq) * 4;
        const float* src = in + row * W;
        floatx4 v;
#pragma unroll
        for (int j = 0; j < 4; ++j) v[j] = c0 + j < W ? src[c0 + j] : 0.f;
        *reinterpret_cast<floatx4*>(out + row * Wp + c0) = v;
    }
}

// A staging buffer for a re-laid-out operand; *got is false (and nothing is
// reported) when it cannot be had (out of memory, or a grow under graph
// capture), so that the caller takes the path that needs no copy.
int stage(size_t bytes, void** out, hipStream_t st, bool* got) {
    return staging_workspace_try(bytes, out, st, got);
}

// Copies `n` tensors of rows[i] rows x W[i] floats into one staging buffer,
// each widened to Wp[i] (a multiple of 4) with zero columns; out[i] receives
// the copy's address.
int widen_all(int n, const float* const* in, const int64_t* rows, const int* W, const int* Wp,
              float** out, hipStream_t st, bool* got) {
    size_t total = 0;
    for (int i = 0; i < n; ++i) total += ((size_t)rows[i] * Wp[i] * 4 + 255) & ~(size_t)255;
    void* ws = nullptr;
    SEERA_TRY(stage(std::max<size_t>(total, 256), &ws, st, got));
    if (!*got) return SEERA_OK;
    char* p = static_cast<char*>(ws);
    for (int i = 0; i < n; ++i) {
        out[i] = reinterpret_cast<float*>(p);
        const int64_t quads = rows[i] * (Wp[i] / 4);
        const int blocks = (int)std::min<int64_t>((quads + 255) / 256, 4096);
        if (quads > 0)
            hipLaunchKernelGGL(widen_rows, dim3(blocks), dim3(256), 0, st, in[i], out[i], rows[i],
                               W[i], Wp[i]);
        SEERA_HIP_TRY(hipGetLastError());
        p += ((size_t)rows[i] * Wp[i] * 4 + 255) & ~(size_t)255;
    }
    return SEERA_OK;
}

// ---------------------------------------------------------------------------
// Space-to-depth form of a stride-2 convolution with a large kernel (the 7x7
// stem on 3 channels): the input's 2x2 pixel blocks become 4C channels and the
// kernel's taps (2t + dy, 2u + dx) become channel (c, dy, dx) of a T2 x U2 =
// ceil(R/2) x ceil(S/2) kernel, so that
//   Y[b, f, oh, ow] = sum_{c2, t, u} W2[f, c2, t, u] * X2[b, c2, oh + t, ow + u]
// with X2[b, (c*2 + dy)*2 + dx, i, j] = X[b, c, 2i + dy - ph, 2j + dx - pw]
// (0 outside X) and W2[f, (c*2 + dy)*2 + dx, t, u] = W[f, c, 2t + dy, 2u + dx]
// (0 past the kernel): a stride-1, pad-0 convolution of at most 16 taps,
// which the band kernels take. dX and dW map back through the same index
// maps (every X and W element has exactly one image in X2 / W2).
// ---------------------------------------------------------------------------
struct S2dGeom {
    int C2, H2, W2, Wp2, T2, U2;  // X2 is [B, C2, H2, Wp2]: channels 4C.., columns W2.. zero
};

// Channels rounded up to a multiple of 8 and rows to a multiple of 4 floats:
// the shapes the row-streaming kernels take.
S2dGeom s2d_geom(int C, int R, int S, int Ho, int Wo) {
    S2dGeom g;
    g.C2 = (4 * C + 7) & ~7;
    g.T2 = (R + 1) / 2;
    g.U2 = (S + 1) / 2;
    g.H2 = Ho + g.T2 - 1;
    g.W2 = Wo + g.U2 - 1;
    g.Wp2 = (g.W2 + 3) & ~3;
    return g;
}

__global__ __launch_bounds__(256) void s2d_input(const float* __restrict__ X, float* __restrict__ X2,
                                                 int B, int C, int H, int W, int ph, int pw, int C2,
                                                 int H2, int W2, int Wp2) {
    const int64_t n = (int64_t)B * C2 * H2 * Wp2;
    for (int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; e < n;
         e += (int64_t)gridDim.x * blockDim.x) {
        const int j = (int)(e % Wp2);
        int64_t r = e / Wp2;
        const int i = (int)(r % H2);
        r /= H2;
        const int c2 = (int)(r % C2);
        const int64_t b = r / C2;
        const int c = c2 >> 2, dy = (c2 >> 1) & 1, dx = c2 & 1;
        const int h = 2 * i + dy - ph, w = 2 * j + dx - pw;
        float v = 0.f;
        if (c < C && j < W2 && (unsigned)h < (unsigned)H && (unsigned)w < (unsigned)W)
            v = X[((b * C + c) * H + h) * W + w];
        X2[e] = v;
    }
}

__global__ __launch_bounds__(256) void s2d_weights(const float* __restrict__ Wt, float* __restrict__ W2,
                                                   int F, int C, int R, int S, int C2, int T2, int U2) {
    const int n = F * C2 * T2 * U2;
    const int e = blockIdx.x * blockDim.x + threadIdx.x;
    if (e >= n) return;
    const int u = e % U2, t = (e / U2) % T2, c2 = (e / (U2 * T2)) % C2, f = e / (U2 * T2 * C2);
    const int c = c2 >> 2, r = 2 * t + ((c2 >> 1) & 1), q = 2 * u + (c2 & 1);
    W2[e] = c < C && r < R && q < S ? Wt[((f * C + c) * R + r) * S + q] : 0.f;
}

// dX[b, c, h, w] = dX2[b, (c*2 + dy)*2 + dx, i, j] with 2i + dy = h + ph, 2j + dx = w + pw
// (dX2 is [B, C2, H2, W2]).
__global__ __launch_bounds__(256) void d2s_input(const float* __restrict__ dX2, float* __restrict__ dX,
                                                 int B, int C, int H, int W, int ph, int pw, int C2,
                                                 int H2, int W2) {
    const int64_t n = (int64_t)B * C * H * W;
    for (int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; e < n;
         e += (int64_t)gridDim.x * blockDim.x) {
        const int w = (int)(e % W);
        int64_t r = e / W;
        const int h = (int)(r % H);
        const int64_t bc = r / H;  // b * C + c
        const int c = (int)(bc % C);
        const int64_t b = bc / C;
        const int pr = h + ph, pc = w + pw;
        const int c2 = (c * 2 + (pr & 1)) * 2 + (pc & 1);
        const int i = pr >> 1, j = pc >> 1;
        dX[e] = i < H2 && j < W2 ? dX2[((b * C2 + c2) * H2 + i) * W2 + j] : 0.f;
    }
}

// dW[f, c, r, s] = dW2[f, (c*2 + r%2)*2 + s%2, r/2, s/2] (dW2 is [F, C2, T2, U2]).
__global__ __launch_bounds__(256) void d2s_weights(const float* __restrict__ dW2, float* __restrict__ dW,
                                                   int F, int C, int R, int S, int C2, int T2, int U2) {
    const int n = F * C * R * S;
    const int e = blockIdx.x * blockDim.x + threadIdx.x;
    if (e >= n) return;
    const int q = e % S, r = (e / S) % R, c = (e / (S * R)) % C, f = e / (S * R * C);
    const int c2 = (c * 2 + (r & 1)) * 2 + (q & 1);
    dW[e] = dW2[((f * C2 + c2) * T2 + (r >> 1)) * U2 + (q >> 1)];
}

// Whether a stride-2 convolution takes the space-to-depth form: a kernel with
// more taps than the direct band kernels hold (16) whose halves fit them.
bool s2d_applies(int R, int S, int sh, int sw) {
    return sh == 2 && sw == 2 && R * S > 16 && ((R + 1) / 2) * ((S + 1) / 2) <= 16;
}

unsigned grid_for(int64_t n) { return (unsigned)std::min<int64_t>((n + 255) / 256, 8192); }

}  // namespace

namespace {

int conv_fwd_epi(const float* X, const float* Wt, float* Y, int B, int C, int H, int W, int F,
                 int R, int S, int sh, int sw, int ph, int pw, const ConvEpi& epi,
                 hipStream_t st) {
    const int Ho = (H + 2 * ph - R) / sh + 1, Wo = (W + 2 * pw - S) / sw + 1;
    const int64_t npix = (int64_t)B * Ho * Wo, K = (int64_t)C * R * S;
    if (npix > 0x7fffffff || K > 0x7fffffff || (int64_t)B * C * H * W > (int64_t)1 << 40)
        return fail(SEERA_ERR_INVALID_ARGUMENT, "conv extent exceeds int range");
    if (npix == 0 || F == 0) return SEERA_OK;
    bool used = false;
    SEERA_TRY(band_conv_fwd(X, Wt, Y, B, C, H, W, F, R, S, sh, sw, ph, pw, st, &used, epi));
    if (used) return SEERA_OK;
    if (s2d_applies(R, S, sh, sw)) {
        const int Ho2 = (H + 2 * ph - R) / sh + 1, Wo2 = (W + 2 * pw - S) / sw + 1;
        const S2dGeom g = s2d_geom(C, R, S, Ho2, Wo2);
        const int64_t xn = (int64_t)B * g.C2 * g.H2 * g.Wp2, wn = (int64_t)F * g.C2 * g.T2 * g.U2;
        void* ws = nullptr;
        bool got = false;
        if (xn * 4 < kMaxTileSpanBytes)
            SEERA_TRY(stage(sizeof(float) * (size_t)(xn + wn), &ws, st, &got));
        if (got) {
            float* X2 = static_cast<float*>(ws);
            float* W2 = X2 + xn;
            hipLaunchKernelGGL(s2d_input, dim3(grid_for(xn)), dim3(256), 0, st, X, X2, B, C, H, W, ph,
                               pw, g.C2, g.H2, g.W2, g.Wp2);
            hipLaunchKernelGGL(s2d_weights, dim3(grid_for(wn)), dim3(256), 0, st, Wt, W2, F, C, R, S,
                               g.C2, g.T2, g.U2);
            SEERA_HIP_TRY(hipGetLastError());
            SEERA_TRY(band_conv_fwd(X2, W2, Y, B, g.C2, g.H2, g.W2, F, g.T2, g.U2, 1, 1, 0, 0, st,
                                    &used, epi, g.Wp2));
            if (used) return SEERA_OK;
        }
    }
    if (W % 4 != 0 && R * S <= 16) {
        // Rows that are not float4-aligned: the band path on a copy of X
        // widened to a multiple of 4 columns (zeros past W, where the
        // convolution reads its own zero padding), storing Y at its width.
        const int Wp = (W + 3) & ~3;
        const int64_t rows = (int64_t)B * C * H;
        float* Xw = nullptr;
        bool got = false;
        SEERA_TRY(widen_all(1, &X, &rows, &W, &Wp, &Xw, st, &got));
        if (got) {
            SEERA_TRY(band_conv_fwd(Xw, Wt, Y, B, C, H, W, F, R, S, sh, sw, ph, pw, st, &used, epi,
                                    Wp));
            if (used) return SEERA_OK;
        }
    }
    // Gather path: any width, any tile size.
    FwdGather g{X, C, H, W, R, S, Wo, Ho * Wo, sh, sw, ph, pw, (int)npix};
    const Plan pl = plan_tiles(F, (int)npix, (int)K, true, false);
    const bool va = aligned16(Wt) && K % 4 == 0;
    auto fill = [&](auto p) {
        p.Wm = Wt; p.ldw = K; p.g = g; p.C = Y; p.out_hw = Ho * Wo;
        p.M = F; p.N = (int)npix; p.K = (int)K; p.ldc = 0; p.split_stride = 0;
        p.epi = epi;
        return p;
    };
    if (va) return run_plan<true>(fill(PixelProblem<4, FwdGather>{}), pl, st);
    return run_plan<true>(fill(PixelProblem<1, FwdGather>{}), pl, st);
}

// db[f] = sum over (b, p) of dY[b, f, p], in a fixed order: block (f, g)
// adds images [g*per, (g+1)*per) -- each thread a strided subset, then a
// tree over the block -- into part[f, g]; a second kernel adds the G parts
// of each f in g order.
constexpr int kCbThreads = 256;

// VEC: HW % 4 == 0 and dY 16-byte aligned; each thread adds float4s, the
// four lanes of one in sequence.
template <bool VEC>
__global__ __launch_bounds__(kCbThreads) void conv_bias_partial(const float* __restrict__ dY,
                                                                float* __restrict__ part, int B,
                                                                int F, int HW, int per, int G) {
    __shared__ float red[kCbThreads];
    const int f = blockIdx.x / G, g = blockIdx.x % G;
    const int b0 = g * per, b1 = min(B, b0 + per);
    float s = 0.f;
    for (int b = b0; b < b1; ++b) {
        const float* row = dY + ((int64_t)b * F + f) * HW;
        if constexpr (VEC) {
            const float4* row4 = reinterpret_cast<const float4*>(row);
            for (int p = threadIdx.x; p < HW / 4; p += kCbThreads) {
                const float4 v = row4[p];
                s += v.x;
                s += v.y;
                s += v.z;
                s += v.w;
            }
        } else {
            for (int p = threadIdx.x; p < HW; p += kCbThreads) s += row[p];
        }
    }
    red[threadIdx.x] = s;
    __syncthreads();
#pragma unroll
    for (int w = kCbThreads / 2; w > 0; w >>= 1) {
        if ((int)threadIdx.x < w) red[threadIdx.x] += red[threadIdx.x + w];
        __syncthreads();
    }
    if (threadIdx.x == 0) part[blockIdx.x] = red[0];
}

__global__ void conv_bias_finish(const float* __restrict__ part, float* __restrict__ db, int F,
                                 int G) {
    const int f = blockIdx.x * blockDim.x + threadIdx.x;
    if (f >= F) return;
    float t = 0.f;
    for (int g = 0; g < G; ++g) t += part[(int64_t)f * G + g];
    db[f] = t;
}

}  // namespace

int conv_fwd(const float* X, const float* Wt, float* Y, int B, int C, int H, int W, int F, int R,
             int S, int sh, int sw, int ph, int pw, hipStream_t st) {
    return conv_fwd_epi(X, Wt, Y, B, C, H, W, F, R, S, sh, sw, ph, pw, ConvEpi{}, st);
}

int conv_fwd_bias_act(const float* X, const float* Wt, const float* bias, float* Y, float* mask,
                      int B, int C, int H, int W, int F, int R, int S, int sh, int sw, int ph,
                      int pw, int act, hipStream_t st) {
    return conv_fwd_epi(X, Wt, Y, B, C, H, W, F, R, S, sh, sw, ph, pw, ConvEpi{bias, mask, act},
                        st);
}

int conv_bias_grad(const float* dY, float* db, int B, int F, int HW, hipStream_t st) {
    if (F == 0) return SEERA_OK;
    if (B == 0 || HW == 0) return fill_f32(db, 0.f, (size_t)F, st);
    // About 2048 blocks in all, at least one image each.
    const int G = std::max(1, std::min(B, 2048 / F));
    const int per = (B + G - 1) / G;
    const int Gu = (B + per - 1) / per;  // groups that hold an image
    void* ws = nullptr;
    SEERA_TRY(workspace(sizeof(float) * (size_t)F * Gu, &ws, st));
    float* part = static_cast<float*>(ws);
    if (HW % 4 == 0 && aligned16(dY))
        hipLaunchKernelGGL(conv_bias_partial<true>, dim3((unsigned)(F * Gu)), dim3(kCbThreads), 0,
                           st, dY, part, B, F, HW, per, Gu);
    else
        hipLaunchKernelGGL(conv_bias_partial<false>, dim3((unsigned)(F * Gu)), dim3(kCbThreads), 0,
                           st, dY, part, B, F, HW, per, Gu);
    SEERA_HIP_TRY(hipGetLastError());
    hipLaunchKernelGGL(conv_bias_finish, dim3((unsigned)((F + 255) / 256)), dim3(256), 0, st, part,
                       db, F, Gu);
    SEERA_HIP_TRY(hipGetLastError());
    return SEERA_OK;
}

int conv_dgrad(const float* Yin, const float* Wconv, float* out, int B, int F, int Hi, int Wi,
               int C, int H, int W, int R, int S, int sh, int sw, int ph, int pw,
               hipStream_t st) {
    const int64_t npix = (int64_t)B * H * W, K = (int64_t)F * R * S;
    if (npix > 0x7fffffff || K > 0x7fffffff)
        return fail(SEERA_ERR_INVALID_ARGUMENT, "conv extent exceeds int range");
    if (npix == 0 || C == 0) return SEERA_OK;
    bool used = false;
    if (s2d_applies(R, S, sh, sw) && Wi % 4 == 0) {
        // dX2 = the stride-1 transposed convolution of dY with W2, then back
        // to the input's layout
        // (dX2 is computed Wp2 columns wide: the columns past W2 read only dY
        // positions past its edge, and are never read back)
        const S2dGeom g = s2d_geom(C, R, S, Hi, Wi);
        const int64_t xn = (int64_t)B * g.C2 * g.H2 * g.Wp2, wn = (int64_t)F * g.C2 * g.T2 * g.U2;
        void* ws = nullptr;
        bool got = false;
        SEERA_TRY(stage(sizeof(float) * (size_t)(xn + wn), &ws, st, &got));
        float* dX2 = static_cast<float*>(ws);
        float* W2 = dX2 + xn;
        if (got) {
            hipLaunchKernelGGL(s2d_weights, dim3(grid_for(wn)), dim3(256), 0, st, Wconv, W2, F, C, R,
                               S, g.C2, g.T2, g.U2);
            SEERA_HIP_TRY(hipGetLastError());
            SEERA_TRY(band_conv_dgrad(Yin, W2, dX2, B, F, Hi, Wi, g.C2, g.H2, g.Wp2, g.T2, g.U2, 1, 1,
                                      0, 0, st, &used));
        }
        if (used) {
            const int64_t n = (int64_t)B * C * H * W;
            hipLaunchKernelGGL(d2s_input, dim3(grid_for(n)), dim3(256), 0, st, dX2, out, B, C, H, W,
                               ph, pw, g.C2, g.H2, g.Wp2);
            SEERA_HIP_TRY(hipGetLastError());
            return SEERA_OK;
        }
    }
    SEERA_TRY(band_conv_dgrad(Yin, Wconv, out, B, F, Hi, Wi, C, H, W, R, S, sh, sw, ph, pw, st,
                              &used));
    if (used) return SEERA_OK;
    if (Wi % 4 != 0) {
        // dY rows that are not float4-aligned: the same on a copy widened to
        // a multiple of 4 columns (the added columns are zeros, as the dY
        // positions past Wi are in the transposed convolution).
        const int Wp = (Wi + 3) & ~3;
        const int64_t rows = (int64_t)B * F * Hi;
        float* Yw = nullptr;
        bool got = false;
        SEERA_TRY(widen_all(1, &Yin, &rows, &Wi, &Wp, &Yw, st, &got));
        if (got) {
            SEERA_TRY(band_conv_dgrad(Yw, Wconv, out, B, F, Hi, Wp, C, H, W, R, S, sh, sw, ph, pw,
                                      st, &used));
            if (used) return SEERA_OK;
        }
    }
    // Gather path: any width, any stride.
    void* ws = nullptr;
    const int64_t wn = (int64_t)F * C * R * S;
    SEERA_TRY(workspace(sizeof(float) * (size_t)std::max<int64_t>(wn, 1), &ws, st));
    float* Wt = static_cast<float*>(ws);
    if (wn > 0) {
        hipLaunchKernelGGL(relayout_dgrad_weight, dim3((unsigned)((wn + 255) / 256)), dim3(256), 0,
                           st, Wconv, Wt, F, C, R * S);
        SEERA_HIP_TRY(hipGetLastError());
    }
    DgradGather g{Yin, F, Hi, Wi, R, S, W, H * W, sh, sw, ph, pw, (int)npix};
    const Plan pl = plan_tiles(C, (int)npix, (int)K, true, false);
    auto fill = [&](auto p) {
        p.Wm = Wt; p.ldw = K; p.g = g; p.C = out; p.out_hw = H * W;
        p.M = C; p.N = (int)npix; p.K = (int)K; p.ldc = 0; p.split_stride = 0;
        return p;
    };
    if (K % 4 == 0) return run_plan<true>(fill(PixelProblem<4, DgradGather>{}), pl, st);
    return run_plan<true>(fill(PixelProblem<1, DgradGather>{}), pl, st);
}

int conv_bwd(const float* dY, const float* Wconv, const float* X, float* dX, float* dW,
             float* db, int B, int C, int H, int W, int F, int R, int S, int sh, int sw, int ph,
             int pw, hipStream_t st) {
    const int Ho = (H + 2 * ph - R) / sh + 1, Wo = (W + 2 * pw - S) / sw + 1;
    if ((int64_t)B * H * W <= 0x7fffffff && (int64_t)B * Ho * Wo <= 0x7fffffff) {
        bool fused = false;
        SEERA_TRY(fused_conv_bwd(dY, Wconv, X, dX, dW, db, B, C, H, W, F, R, S, sh, sw, ph, pw, st,
                                 &fused));
        if (fused) return SEERA_OK;
    }
    SEERA_TRY(conv_dgrad(dY, Wconv, dX, B, F, Ho, Wo, C, H, W, R, S, sh, sw, ph, pw, st));
    return conv_wgrad(dY, X, dW, db, B, C, H, W, F, R, S, sh, sw, ph, pw, st);
}

int conv_wgrad(const float* Y, const float* X, float* dW, float* db, int B, int C, int H, int W,
               int F, int R, int S, int sh, int sw, int ph, int pw, hipStream_t st) {
    const int Ho = (H + 2 * ph - R) / sh + 1, Wo = (W + 2 * pw - S) / sw + 1;
    const int64_t npix = (int64_t)B * Ho * Wo, crs = (int64_t)C * R * S;
    if (npix > 0x7fffffff || crs > 0x7fffffff)
        return fail(SEERA_ERR_INVALID_ARGUMENT, "conv extent exceeds int range");
    if (F == 0 || crs == 0) return SEERA_OK;
    WgradProblem p{};
    p.ga = WgradYGather{Y, F, Ho * Wo};
    p.gb = WgradXGather{X, C, H, W, R, S, Wo, Ho * Wo, sh, sw, ph, pw, (int)crs};
    p.C = dW;
    p.M = F;
    p.N = (int)crs;
    p.K = (int)npix;
    p.ldc = crs;
    p.split_stride = 0;
    if (npix == 0) {
        // Empty contraction: dW = 0 (and db = 0).
        SEERA_TRY(fill_f32(dW, 0.f, (size_t)F * crs, st));  // a kernel: safe under graph capture
        if (db) SEERA_TRY(fill_f32(db, 0.f, (size_t)F, st));
        return SEERA_OK;
    }
    bool used = false, db_done = false;
    SEERA_TRY(band_conv_wgrad(Y, X, dW, db, B, C, H, W, F, R, S, sh, sw, ph, pw, st, &used,
                              &db_done));
    if (!used && s2d_applies(R, S, sh, sw) && Wo % 4 == 0) {
        // dW2 = the stride-1 dW of (dY, X2), then back to W's layout
        const S2dGeom g = s2d_geom(C, R, S, Ho, Wo);
        const int64_t xn = (int64_t)B * g.C2 * g.H2 * g.Wp2, wn = (int64_t)F * g.C2 * g.T2 * g.U2;
        void* ws = nullptr;
        bool got = false;
        if (xn * 4 < kMaxTileSpanBytes)
            SEERA_TRY(stage(sizeof(float) * (size_t)(xn + wn), &ws, st, &got));
        if (got) {
            float* X2 = static_cast<float*>(ws);
            float* dW2 = X2 + xn;
            hipLaunchKernelGGL(s2d_input, dim3(grid_for(xn)), dim3(256), 0, st, X, X2, B, C, H, W, ph,
                               pw, g.C2, g.H2, g.W2, g.Wp2);
            SEERA_HIP_TRY(hipGetLastError());
            SEERA_TRY(band_conv_wgrad(Y, X2, dW2, nullptr, B, g.C2, g.H2, g.Wp2, F, g.T2, g.U2, 1, 1,
                                      0, 0, st, &used, &db_done, Wo));
            if (used) {
                const int n = F * C * R * S;
                hipLaunchKernelGGL(d2s_weights, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st,
                                   dW2, dW, F, C, R, S, g.C2, g.T2, g.U2);
                SEERA_HIP_TRY(hipGetLastError());
            }
        }
    }
    if (!used && (W % 4 != 0 || Wo % 4 != 0)) {
        // Rows that are not float4-aligned: the band / row-streaming dW on
        // copies of X and dY widened with zero columns to a width W2 >= W
        // (a multiple of 4) whose output width Wo2 >= Wo is one too. The
        // added dY columns are zero, so they add nothing; the X columns
        // past W are zeros, as the convolution's padding reads.
        int W2 = (W + 3) & ~3, Wo2 = 0;
        for (; W2 < W + 4 * sw + 4; W2 += 4) {
            Wo2 = (W2 + 2 * pw - S) / sw + 1;
            if (Wo2 % 4 == 0) break;
        }
        if (Wo2 % 4 == 0 && Wo2 >= Wo) {
            const float* src[2] = {X, Y};
            const int64_t rows[2] = {(int64_t)B * C * H, (int64_t)B * F * Ho};
            const int w0[2] = {W, Wo}, w1[2] = {W2, Wo2};
            float* dst[2] = {nullptr, nullptr};
            bool got = false;
            SEERA_TRY(widen_all(2, src, rows, w0, w1, dst, st, &got));
            if (got)
                SEERA_TRY(band_conv_wgrad(dst[1], dst[0], dW, db, B, C, H, W2, F, R, S, sh, sw, ph,
                                          pw, st, &used, &db_done));
        }
    }
    if (!used) {
        // Gather path: any width, any kernel size.
        // Gathers only: the 64x64 tile, split over pixels.
        const Plan pl = plan_tiles(F, (int)crs, (int)npix, false, true);
        SEERA_TRY(run_plan<false>(p, pl, st));
    }
    // Paths that do not fuse the bias gradient: its own pass over dY.
    if (db && !db_done) return conv_bias_grad(Y, db, B, F, Ho * Wo, st);
    return SEERA_OK;
}

}  // namespace seera
