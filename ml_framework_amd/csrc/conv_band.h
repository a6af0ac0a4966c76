// conv_band.h -- LDS-band convolution (conv_band.hip): argument block and
// host entry points.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <algorithm>

#include "runtime.h"

namespace seera {

typedef _Float16 half_t;

constexpr int kBandMaxPhases = 16;
constexpr int64_t kBandMaxLds = 160 * 1024;

// One stride phase of a launch: the output sub-grid it writes and how its
// taps read the input (see conv_band.hip for the formula).
struct BandPhase {
    int Ho, Wo;      // phase output grid
    int T, U;        // taps along rows / columns
    int iph, ipw;    // input row = oh*ish + t - iph
    int oph, opw;    // output row = oh*osh + oph
    int64_t woff;    // offset (halves) of this phase's prepared weights
    int nrb, ncb;    // row / column tiles of the phase grid
    int block0;      // first blockIdx.x of the phase
};

// Fused forward epilogue of a Conv2D layer (Seera.py:254-257: conv2d, then
// + bias [1, F, 1, 1], then the activation): bias [F] (nullptr: none) added in
// fp32 to each output of filter f, then act (0 none, 1 ReLU: out = v > 0 ? v
// : 0, mask = v > 0 ? 1 : 0 when mask [B, F, Hout, Wout] is not nullptr).
// All zero: a plain convolution.
struct ConvEpi {
    const float* bias;
    float* mask;
    int act;
};

struct BandConvArgs {
    const float* in;     // [B, C, H, W] fp32
    const half_t* wk;    // prepared fp16 weights
    float* out;          // [B, F, Hout, Wout] fp32
    int B, C, H, W;
    int F, Hout, Wout;
    int ish, isw, osh, osw;
    int TH, WC;          // output tile rows / columns per block
    int BR, BC4;         // input band rows / columns (BC4 % 4 == 0)
    int max_taps;
    int nchunks, nftiles, nblocks;
    int64_t lds_bytes;
    int nphase;
    BandPhase ph[kBandMaxPhases];
    ConvEpi epi;         // forward only; zero for the transposed launches
};

// Forward convolution Y = conv(X, W) (W [F, C, R, S]) when the band path
// applies (input row pitch % 4 == 0, tile fits LDS); *used reports whether it
// ran. x_pitch > W_in: X's rows are x_pitch floats long, columns past W_in
// zero (a copy widened to a float4 multiple); the output is W_in's.
int band_conv_fwd(const float* X, const float* W, float* Y, int B, int C, int H, int W_in, int F,
                  int R, int S, int sh, int sw, int ph, int pw, hipStream_t st, bool* used,
                  const ConvEpi& epi = {}, int x_pitch = 0);

// Transposed convolution out[B, Cc, H, W] of Y [B, Fc, Hi, Wi] with the conv
// weight W [Fc, Cc, R, S] (stride, pad of the forward conv), by stride phases.
int band_conv_dgrad(const float* Y, const float* W, float* out, int B, int Fc, int Hi, int Wi,
                    int Cc, int H, int W_out, int R, int S, int sh, int sw, int ph, int pw,
                    hipStream_t st, bool* used);

// Stride-2 transposed convolution of band_conv_dgrad's form with all four
// stride phases per block (conv_phase2.hip): in [B, C, H, W], W [C, F, R, S]
// read at taps (r0h[a] + 2*(T[a]-1-t), r0w[c] + 2*(U[c]-1-u)), out [B, F,
// Hout, Wout]; runs when C % 32 == 0, C <= 128, T, U in {1, 2}, Hout even and
// Wout % 8 == 0; *used reports whether it ran.
int phase2_conv(const float* in, const float* W, float* out, int B, int C, int H, int W_in, int F,
                int Hout, int Wout, int R, int S, const int T[2], const int iph[2],
                const int r0h[2], const int U[2], const int ipw[2], const int r0w[2],
                hipStream_t st, bool* used);

// 4x4 convolution at stride 2, padding 1 (conv_stride2.hip): out [B, F, Ho,
// Wo] of in [B, C, H, W] and W [F, C, 4, 4]; runs when C is 32 or 64, W % 4
// == 0 and Wo % 4 == 0; *used reports whether it ran.
int stride2_conv(const float* in, const float* W, float* out, int B, int C, int H, int W_in, int F,
                 hipStream_t st, bool* used);

// Row-streaming variant (conv_stream.hip) of the launch `band` describes
// (weights already prepared in band.wk): runs when every phase reads its input
// with stride 1 and the weights plus an input-row ring fit in LDS; *used
// reports whether it ran.
int stream_conv(const BandConvArgs& band, hipStream_t st, bool* used);

// Three-role row streaming (conv_split.hip) of a 3x3, stride 1, pad 1 launch
// of 64k input channels (W % 4 == 0; rows wider than 56 in column tiles; one
// launch per 64-channel slice, each after the first adding to the output):
// the matrix-core waves hand their results to storer waves through LDS;
// *used reports whether it ran.
int split_conv(const BandConvArgs& band, hipStream_t st, bool* used);

}  // namespace seera

namespace seera {

// Weight-gradient band kernel arguments (conv_band.hip).
struct WgradArgs {
    const float* dy;    // [B, F, Ho, Wo]
    const float* x;     // [B, C, H, W]
    float* part;        // [tiles][nsplit][64][CT*R*S] partial sums
    int B, C, H, W, F, Ho, Wo, R, S, sh, sw, ph, pw;
    int TH, WC8, BR;    // output tile (TH rows x WC8 columns, WC8 % 8 == 0), X rows per band
    int KS;             // 32-pixel k-steps per tile
    int nrb, ncb, items, ips, nsplit;
    int nftile, nctile, CT;
    int dy_stride;      // halves per filter row of the dY tile
    int xrow;           // halves per row of a shifted X copy (WC8 rounded to whole items)
    int x_plane;        // halves per (s, channel) plane of the shifted X copies
    int64_t lds_bytes;
};

// Per-block partial sums of dW written by stream_wgrad_partials
// (conv_wgrad.hip): part[tile][split][64 f][CT*R*S], column (r*S + s)*CT + c.
struct WgradPartials {
    float* part;
    float* dbpart;  // [ftiles][nsplit][64] bias-gradient partials, or nullptr
    int CT, nctile, ntiles, nsplit;
};

// Row-streaming dW partials of a stride-1 convolution (R, S <= 3, rows
// float4-aligned), and with with_db the bias-gradient partials of dY; *used
// reports whether it ran. The caller reduces them.
int stream_wgrad_partials(const float* Y, const float* X, int B, int C, int H, int W, int F,
                          int R, int S, int ph, int pw, bool with_db, hipStream_t st,
                          WgradPartials* out, bool* used);

// Sums the partials into dW [F, C, R, S] in a fixed order (and, with dbpart,
// the bias-gradient partials into db), one launch (conv_band.hip).
int reduce_wgrad_partials(const float* part, float* dW, int F, int C, int R, int S, int CT,
                          int nctile, int ntiles, int nsplit, hipStream_t st, const float* dbpart,
                          float* db);

// Conv2D backward of a 3x3, stride 1, pad 1, 64 -> 64 channel layer in one
// pass over dY (conv_bwd_fused.hip): dX [B, 64, H, W], dW [64, 64, 3, 3] and,
// when db is not nullptr, db [64]; runs when W % 4 == 0, W <= 56 and the
// tensors are 16-byte aligned; *used reports whether it ran.
int fused_conv_bwd(const float* dY, const float* Wconv, const float* X, float* dX, float* dW,
                   float* db, int B, int C, int H, int W, int F, int R, int S, int sh, int sw,
                   int ph, int pw, hipStream_t st, bool* used);

// Row-streaming dW partials of a 4x4 stride-2 padding-1 convolution
// (conv_wgrad_s2.hip): Y [B, F, Ho, Wo], X [B, C, H, W]; runs when W and Wo
// are multiples of 4; *used reports whether it ran. The caller reduces them.
int wgrad_s2_partials(const float* Y, const float* X, int B, int C, int H, int W, int F,
                      hipStream_t st, WgradPartials* out, bool* used);

// dW [F, C, R, S] = sum over (b, oh, ow) of dY[b, f, oh, ow] *
// X[b, c, oh*sh - ph + r, ow*sw - pw + s], when the band path applies. With a
// non-null db and the row-streaming path, also db[f] = sum of dY[b, f, ...]
// from the same pass (*db_done reports it; otherwise the caller computes db).
// wo_override > 0: dY rows hold that many columns, fewer than W's geometry
// gives (X's rows are a widened copy: W is their pitch).
int band_conv_wgrad(const float* Y, const float* X, float* dW, float* db, int B, int C, int H,
                    int W, int F, int R, int S, int sh, int sw, int ph, int pw, hipStream_t st,
                    bool* used, bool* db_done, int wo_override = 0);

}  // namespace seera
