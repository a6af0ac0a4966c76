// conv_wgrad_s2.hip -- weight gradient of a 4x4 convolution at stride 2,
// padding 1, by row streaming (convolution.cu:268-366 for the convolution;
// upsampling.cu:202-301, 354-374 for a 4x4 stride-2 transposed convolution,
// whose dW is this one with the roles of X and dY swapped):
//   dW[f, c, r, s] = sum_{b, oh, ow} Y[b, f, oh, ow] * X[b, c, 2*oh - 1 + r, 2*ow - 1 + s]
// a GEMM with M = filters, N = (tap, channel), K = pixels of Y.
//
// A block owns a 64-filter x CT-channel tile of dW (all 16 taps) and a strip
// of output rows of one image (or several strips in turn), and streams:
//   * 4 consumer waves, one per tap row r. Per output row (one K-slice of 32
//     pixels, zero past the row) a wave reads the 4 filter-group fragments
//     of Y and, for each column tap s, the CT/16 channel-group fragments of
//     the input row 2*oh - 1 + r, and accumulates 64 filters x CT channels x
//     4 taps in registers (v_mfma_f32_16x16x32_f16, Y as A, X as B);
//   * 4 producer waves stage the next step's 2 rows of Y and 4 input rows of
//     X (fp16). The input rows are kept as four frames per channel, frame s
//     holding X[c, row, 2*x - 1 + s] at pixel x, so every B fragment (8
//     consecutive pixels of one channel) is one aligned 16-byte read.
// Each block writes its partial sums; wgrad_reduce4 (conv_band.hip) adds the
// partials of a tile in a fixed order.
#include "conv_band.h"
#include "mfma_core.h"

namespace seera {
namespace {

typedef float floatx4_t __attribute__((ext_vector_type(4)));

__device__ __forceinline__ floatx4_t mfma16x16x32(half8 a, half8 b, floatx4_t c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}

constexpr int kRows = 2;          // output rows (K-slices) per step
constexpr int kIn = 2 * kRows;    // new input rows per step
constexpr int kCons = 4 * 64;
constexpr int kProd = 256;
constexpr int kNT = kCons + kProd;
constexpr int kWC = 32;           // output columns per item (one K-slice)
// Halves per LDS pixel row: 96 bytes. A fragment read (16 rows x 4 chunks of
// 16 bytes) is served per half-wave in two passes of 16 lanes, 8 rows x 2
// chunks each; rows 96 bytes apart put those 16 lanes on 16 distinct 16-byte
// slots of a 256-byte window (an 80-byte stride puts two lanes on a slot).
constexpr int kPx = 48;
constexpr int kNR = 2 * kIn + 2;  // ring rows of X

// Row (filter or channel) of an LDS item from its index: bits 0 and 1 swapped,
// so that the 8 lanes of a ds_write_b128 group (4 octets of rows r and r + 2,
// 192 bytes apart) hit 8 distinct 16-byte slots of a 128-byte window (rows r
// and r + 1, 96 bytes apart, put two lanes on each of two slots).
__device__ __forceinline__ int item_row(int i) {
    return (i & ~3) | ((i >> 1) & 1) | ((i & 1) << 1);
}

struct WgradS2Args {
    const float* y;      // [B, F, Ho, Wo]
    const float* x;      // [B, C, H, W]
    float* part;         // [ftile*nctile + ctile][nsplit][64][CT*16]
    int B, F, Ho, Wo, C, H, W;
    int L;               // output rows per strip
    int nstrips, ncb;    // strips and column tiles per image
    int items, ips, nsplit;
    int nctile;
};

template <int CG>
__global__ __launch_bounds__(kNT) void wgrad_s2_kernel(const WgradS2Args a) {
    constexpr int CT = 16 * CG;                   // channels per tile
    constexpr int ys_half = kRows * 64 * kPx;     // halves per Y stage
    constexpr int xs_row = 4 * CT * kPx;          // halves per ring row ([frame][c][px])
    extern __shared__ __attribute__((aligned(16))) half_t smem[];
    half_t* const ys = smem;                      // [2 stages][kRows][64 f][kPx]
    half_t* const xs = smem + 2 * ys_half;        // [kNR][4 frames][CT][kPx]

    const int split = blockIdx.x, ty = blockIdx.y;
    const int ftile = ty / a.nctile, ctile = ty - ftile * a.nctile;
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int it0 = split * a.ips, it1 = min(a.items, it0 + a.ips);

    if (wave < 4) {
        // ---------------- consumers: tap row r = wave ----------------
        const int r = wave, kc = lane >> 4;
        floatx4_t acc[4][4][CG];  // [filter group][column tap s][channel group]
#pragma unroll
        for (int fg = 0; fg < 4; ++fg)
#pragma unroll
            for (int s = 0; s < 4; ++s)
#pragma unroll
                for (int cg = 0; cg < CG; ++cg) acc[fg][s][cg] = floatx4_t{0.f, 0.f, 0.f, 0.f};
        const int aoff = (lane & 15) * kPx + 8 * kc;   // + fg*16*kPx
        for (int item = it0; item < it1; ++item) {
            const int strip = item / a.ncb % a.nstrips;
            const int Lb = min(a.L, a.Ho - strip * a.L);
            const int nsteps = (Lb + kRows - 1) / kRows;
            for (int st = 0; st < nsteps; ++st) {
                __syncthreads();  // step st's rows are staged
#pragma unroll
                for (int o = 0; o < kRows; ++o) {
                    const half_t* yl = ys + (st & 1) * ys_half + o * 64 * kPx;
                    const half_t* xl = xs + ((4 * st + 2 * o + r) % kNR) * xs_row;
                    half8 fa[4], fb[4][CG];
#pragma unroll
                    for (int fg = 0; fg < 4; ++fg)
                        fa[fg] = *reinterpret_cast<const half8*>(yl + fg * 16 * kPx + aoff);
#pragma unroll
                    for (int s = 0; s < 4; ++s)
#pragma unroll
                        for (int cg = 0; cg < CG; ++cg)
                            fb[s][cg] = *reinterpret_cast<const half8*>(
                                xl + (s * CT + cg * 16) * kPx + aoff);
#pragma unroll
                    for (int s = 0; s < 4; ++s)
#pragma unroll
                        for (int cg = 0; cg < CG; ++cg)
#pragma unroll
                            for (int fg = 0; fg < 4; ++fg)
                                acc[fg][s][cg] = mfma16x16x32(fa[fg], fb[s][cg], acc[fg][s][cg]);
                }
            }
            __syncthreads();  // this item's last step is done with the ring
        }
        // Partial sums: lane holds filters fg*16 + 4*kc + i, channel
        // cg*16 + lane%16 of tap (r, s); column (r*4 + s)*CT + channel.
        constexpr int ntot = CT * 16;
        float* const dst = a.part + ((int64_t)ty * a.nsplit + split) * 64 * ntot;
#pragma unroll
        for (int fg = 0; fg < 4; ++fg)
#pragma unroll
            for (int s = 0; s < 4; ++s)
#pragma unroll
                for (int cg = 0; cg < CG; ++cg) {
                    const int n = (r * 4 + s) * CT + cg * 16 + (lane & 15);
#pragma unroll
                    for (int i = 0; i < 4; ++i)
                        dst[(int64_t)(fg * 16 + 4 * kc + i) * ntot + n] = acc[fg][s][cg][i];
                }
        return;
    }

    // ---------------- producers ----------------
    // Y items: (row o, filter f, octet k): 8 pixels, 2 float4 loads; 512 per
    // step, 2 per thread (filters in item_row order). X items: (input row,
    // channel, octet k): the 24
    // columns 2*(ow0 + 8k) - 4 .. +23 (6 float4 loads), written as the four
    // frames' octets; 16*CT per step, CG per thread.
    const int ptid = tid - kCons;
    const int f_lim = a.F - ftile * 64;
    const int c_base = ctile * CT;
    for (int item = it0; item < it1; ++item) {
        const int cb = item % a.ncb;
        const int strip = item / a.ncb % a.nstrips;
        const int b = item / a.ncb / a.nstrips;
        const int oh0 = strip * a.L;
        const int Lb = min(a.L, a.Ho - oh0);
        const int nsteps = (Lb + kRows - 1) / kRows;
        const int ow0 = cb * kWC;
        const int need = 2 * Lb + 2;              // strip input rows used
        const int hin0 = 2 * oh0 - 1;             // image row of strip input row 0
        const rsrc_t ysrc = make_rsrc_in(a.y, (int64_t)a.B * a.F * a.Ho * a.Wo, ((int64_t)b * a.F + ftile * 64) * a.Ho * a.Wo);
        const rsrc_t xsrc = make_rsrc_in(a.x, (int64_t)a.B * a.C * a.H * a.W, ((int64_t)b * a.C + c_base) * a.H * a.W);

        floatx4 yv[2][2];
        floatx4 xv[CG][6];
        // Y rows of step G into registers / into stage G & 1.
        auto y_load = [&](int G) {
#pragma unroll
            for (int k = 0; k < 2; ++k) {
                const int it = ptid + k * kProd;  // (o, f, octet): octet fastest
                const int oct = it & 3, f = item_row(it >> 2) & 63, o = it >> 8;
                const int oh = oh0 + G * kRows + o, ow = ow0 + 8 * oct;
                const bool ok = G * kRows + o < Lb && f < f_lim;
                const uint32_t off = (uint32_t)(((f * a.Ho + oh) * a.Wo + ow) * 4);
#pragma unroll
                for (int h = 0; h < 2; ++h)
                    yv[k][h] = buf_load4(ysrc, ok && ow + 4 * h < a.Wo ? off + 16u * h : kBufOOB);
            }
        };
        auto y_store = [&](int G) {
#pragma unroll
            for (int k = 0; k < 2; ++k) {
                const int it = ptid + k * kProd;
                const int oct = it & 3, f = item_row(it >> 2) & 63, o = it >> 8;
                float v8[8];
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    v8[q] = yv[k][0][q];
                    v8[4 + q] = yv[k][1][q];
                }
                *reinterpret_cast<half8*>(ys + (G & 1) * ys_half + (o * 64 + f) * kPx + 8 * oct) =
                    pack8(v8);
            }
        };
        // X input rows [I0, I0 + NROWS) of the strip.
        auto x_load = [&](int I0, int NROWS) {
#pragma unroll
            for (int k = 0; k < CG; ++k) {
                const int it = ptid + k * kProd;  // (row, c, octet): octet fastest
                const int oct = it & 3, c = item_row((it >> 2) % CT), row = (it >> 2) / CT;
                const int i = I0 + row, hin = hin0 + i;
                const int col0 = 2 * (ow0 + 8 * oct) - 4;
                const bool ok = row < NROWS && i < need && (unsigned)hin < (unsigned)a.H &&
                                c_base + c < a.C;
                const int base = (c * a.H + hin) * a.W + col0;
#pragma unroll
                for (int q = 0; q < 6; ++q) {
                    const int col = col0 + 4 * q;
                    xv[k][q] = buf_load4(xsrc, ok && (unsigned)col < (unsigned)a.W
                                                   ? (uint32_t)((base + 4 * q) * 4) : kBufOOB);
                }
            }
        };
        auto x_store = [&](int I0, int NROWS) {
#pragma unroll
            for (int k = 0; k < CG; ++k) {
                const int it = ptid + k * kProd;
                const int oct = it & 3, c = item_row((it >> 2) % CT), row = (it >> 2) / CT;
                const int i = I0 + row;
                // Rows past the strip are written too (as zeros: their loads
                // read 0), so every ring row a step reads holds finite values.
                if (row < NROWS) {
                    half_t* dst = xs + (i % kNR) * xs_row + c * kPx + 8 * oct;
#pragma unroll
                    for (int s = 0; s < 4; ++s) {
                        float v8[8];
#pragma unroll
                        for (int j = 0; j < 8; ++j) {
                            const int e = 3 + s + 2 * j;  // column 2*x - 1 + s of the window
                            v8[j] = xv[k][e >> 2][e & 3];
                        }
                        *reinterpret_cast<half8*>(dst + s * CT * kPx) = pack8(v8);
                    }
                }
            }
        };
        // Prologue: input rows 0..5 and Y of step 0. (X items per call cover
        // kIn rows, so the six rows take two calls.)
        x_load(0, kIn);
        y_load(0);
        x_store(0, kIn);
        y_store(0);
        x_load(kIn, 2);
        x_store(kIn, 2);
        __syncthreads();  // releases step 0
        // Step g's input rows beyond the previous step's are 4g+2 .. 4g+5.
        if (nsteps > 1) {
            x_load(4 + 2, kIn);
            y_load(1);
        }
        for (int g = 1; g < nsteps; ++g) {
            x_store(4 * g + 2, kIn);
            y_store(g);
            if (g + 1 < nsteps) {
                x_load(4 * (g + 1) + 2, kIn);
                y_load(g + 1);
            }
            __syncthreads();  // releases step g
        }
        __syncthreads();  // the consumers are done with this item's ring
    }
}

template <int CG>
hipError_t launch_cg(const WgradS2Args& a, int nty, int64_t lds, hipStream_t st) {
    auto k = wgrad_s2_kernel<CG>;
    hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(k),
                                       hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL(k, dim3(a.nsplit, nty), dim3(kNT), (size_t)lds, st, a);
    return hipGetLastError();
}

}  // namespace

int wgrad_s2_partials(const float* Y, const float* X, int B, int C, int H, int W, int F,
                      hipStream_t st, WgradPartials* out, bool* used) {
    *used = false;
    const int Ho = (H + 2 - 4) / 2 + 1, Wo = (W + 2 - 4) / 2 + 1;
    if (B <= 0 || F <= 0 || C <= 0 || Ho <= 0 || Wo <= 0 || W % 4 != 0 || Wo % 4 != 0) return SEERA_OK;
    if ((reinterpret_cast<uintptr_t>(Y) & 15) != 0 || (reinterpret_cast<uintptr_t>(X) & 15) != 0)
        return SEERA_OK;
    // Buffer resources span one image's X planes (plus a partial tile's
    // overrun) and a 64-filter slice of Y.
    if ((int64_t)(C + 32) * H * W * 4 >= kMaxTileSpanBytes ||
        (int64_t)64 * Ho * Wo * 4 >= kMaxTileSpanBytes)
        return SEERA_OK;
    const int CG = 1;  // 16-channel tiles: half the partial sums of 32-channel ones
    const int CT = 16 * CG;
    WgradS2Args a{};
    a.y = Y; a.x = X;
    a.B = B; a.F = F; a.Ho = Ho; a.Wo = Wo; a.C = C; a.H = H; a.W = W;
    a.ncb = (Wo + kWC - 1) / kWC;
    const int nftile = (F + 63) / 64;
    a.nctile = (C + CT - 1) / CT;
    const int tiles = nftile * a.nctile;
    // Strips: enough blocks to cover the chip (about 256 with one strip per
    // block), each strip an even number of rows.
    const int want = std::max(1, (256 + tiles - 1) / tiles);
    const int per_img = std::max(1, (want + B * a.ncb - 1) / (B * a.ncb));
    a.L = std::max(kRows, ((Ho + per_img - 1) / per_img + 1) & ~1);
    a.nstrips = (Ho + a.L - 1) / a.L;
    a.items = B * a.nstrips * a.ncb;
    a.nsplit = std::max(1, std::min(a.items, want));
    a.ips = (a.items + a.nsplit - 1) / a.nsplit;
    a.nsplit = (a.items + a.ips - 1) / a.ips;
    const int64_t lds = ((int64_t)2 * kRows * 64 * kPx + (int64_t)kNR * 4 * CT * kPx) * 2;
    if (lds > kBandMaxLds) return SEERA_OK;
    const int ntot = CT * 16;
    const size_t part_bytes = sizeof(float) * (size_t)tiles * a.nsplit * 64 * ntot;
    void* ws = nullptr;
    SEERA_TRY(workspace(part_bytes, &ws, st));
    a.part = static_cast<float*>(ws);
    const hipError_t e = launch_cg<CG>(a, tiles, lds, st);
    if (e != hipSuccess) return fail_hip(e, "stride-2 wgrad launch");
    out->part = a.part;
    out->dbpart = nullptr;
    out->CT = CT;
    out->nctile = a.nctile;
    out->ntiles = tiles;
    out->nsplit = a.nsplit;
    *used = true;
    return SEERA_OK;
}

}  // namespace seera
