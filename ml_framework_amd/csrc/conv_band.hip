// conv_band.hip -- LDS-band implicit-GEMM convolution for gfx950.
//
// One kernel covers every convolution-shaped pass of the hot path whose input
// rows are float4-aligned (W % 4 == 0):
//   conv2d forward       (convolution.cu:15-101, 367-389)
//   conv2d dX            (convolution.cu:144-265, 401-429)   flipped weights
//   convT forward        (upsampling.cu:15-126, 376-401)     = conv2d dX
//   convT dX             (upsampling.cu:128-197, 337-346)    = conv2d forward
//
// General form computed by one launch, per phase z (stride phases of the
// transposed convolutions; a plain forward convolution has one phase):
//   out[b, f, oh*osh + oph_z, ow*osw + opw_z] =
//     sum_{c < Cin, t < T_z, u < U_z} Wk_z[f, t, u, c] *
//                                     in[b, c, oh*ish + t - iph_z, ow*isw + u - ipw_z]
// with zero outside the input. Wk_z is the prepared fp16 weight tensor.
//
// A block owns one image, a TH x WC tile of the phase's output grid and 64
// output channels. For each chunk of 32 input channels it stages
//   * the input band those outputs read (rows x cols x 32 channels, rounded
//     to fp16, channel-last so that 8 channels of one pixel are 16 bytes), and
//   * the 64 x taps x 32 weight slice
// in LDS once; every tap then reads shifted 16-byte windows of the band as
// the B operand of v_mfma_f32_16x16x32_f16 (32 channels of one tap per MFMA).
// HBM sees each input element once per output-channel tile (plus the halo
// rows of neighbouring bands, mostly served by L2) and each output once: the
// im2col matrix is never formed.
#include "conv_band.h"
#include "mfma_core.h"

namespace seera {
namespace {

typedef float floatx4_t __attribute__((ext_vector_type(4)));

__device__ __forceinline__ floatx4_t mfma16x16x32(half8 a, half8 b, floatx4_t c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}

// Band layout: pixel p (row-major over the band's rows x BC4 columns) holds 32
// channels = four 16-byte chunks. Two pixels share a 128-byte bank window; the
// chunk order inside a pixel is rotated by (p >> 1) & 3, which makes any eight
// consecutive pixels at one chunk hit eight distinct 16-byte slots (the MFMA B
// reads of a stride-1 convolution). Stride-2 reads touch pixels of one parity
// and see two-way conflicts.
__device__ __forceinline__ int band_off(int p, int chunk) {
    return p * 32 + ((chunk ^ ((p >> 1) & 3)) << 3);
}

constexpr int kNT = 256;  // threads per block (4 waves: 2 filter halves x 2 pixel halves)
constexpr int kBandMaxTaps = 16;  // taps per phase the band kernel handles (weights in LDS)

template <int PGW>
__global__ __launch_bounds__(kNT) void band_conv_kernel(const BandConvArgs a) {
    extern __shared__ __attribute__((aligned(16))) half_t smem[];

    // Phase and tile of this block.
    const int bx = blockIdx.x;
    int z = 0;
    while (z + 1 < a.nphase && bx >= a.ph[z + 1].block0) ++z;
    const BandPhase& P = a.ph[z];
    int local = bx - P.block0;
    const int cb = local % P.ncb;
    local /= P.ncb;
    const int rb = local % P.nrb;
    const int b = local / P.nrb;
    const int oh0 = rb * a.TH, ow0 = cb * a.WC;
    const int ftile = blockIdx.y;
    const int taps = P.T * P.U;

    half_t* const wl = smem;                         // taps x 64 f x 32 c
    half_t* const bl = smem + a.max_taps * 2048;     // BR x BC4 pixels x 32 c

    const int ir0 = oh0 * a.ish - P.iph;             // input row of band row 0
    const int icr = ow0 * a.isw - P.ipw;             // input col of output col ow0, tap 0
    const int ic0 = icr >= 0 ? (icr & ~3) : -((-icr + 3) & ~3);  // floor to a multiple of 4
    const int coff = icr - ic0;                      // 0..3

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wf = wave & 1, wp = wave >> 1;
    const int tile_px = a.TH * a.WC;

    // Band pixel of each of this lane's output pixels at tap (0, 0).
    int pbase[PGW];
#pragma unroll
    for (int i = 0; i < PGW; ++i) {
        int px = (wp * PGW + i) * 16 + (lane & 15);
        if (px >= tile_px) px = 0;  // padding lanes: computed, never stored
        const int ohl = px / a.WC, owl = px - ohl * a.WC;
        pbase[i] = ohl * a.ish * a.BC4 + owl * a.isw + coff;
    }

    floatx4_t acc[2][PGW];
#pragma unroll
    for (int fi = 0; fi < 2; ++fi)
#pragma unroll
        for (int i = 0; i < PGW; ++i) acc[fi][i] = floatx4_t{0.f, 0.f, 0.f, 0.f};

    const int64_t in_img = (int64_t)b * a.C * a.H * a.W;
    const int nq = a.BC4 >> 2;                       // column quads per band row
    const int band_items = a.BR * nq * 4;            // (row, quad, 8-channel group)
    const half_t* wsrc_base = a.wk + P.woff + (int64_t)ftile * a.nchunks * taps * 2048;

    for (int ch = 0; ch < a.nchunks; ++ch) {
        __syncthreads();  // the previous chunk's MFMAs are done with the LDS tiles

        // Weights: taps x 2048 halves, contiguous in Wk; 16-byte pieces, one
        // per tap for each thread (taps <= kBandMaxTaps), all loads issued
        // before the LDS writes.
        const half_t* wsrc = wsrc_base + (int64_t)ch * taps * 2048;
        {
            half8 wv[kBandMaxTaps];
#pragma unroll
            for (int tp = 0; tp < kBandMaxTaps; ++tp)
                if (tp < taps) wv[tp] = *reinterpret_cast<const half8*>(wsrc + (tp * 256 + tid) * 8);
#pragma unroll
            for (int tp = 0; tp < kBandMaxTaps; ++tp)
                if (tp < taps) lds_write8<32>(wl + tp * 2048, tid >> 2, tid & 3, wv[tp]);
        }

        // Input band: each item is 4 consecutive columns x 8 channels, loaded
        // as 8 float4 rows of the NCHW tensor and transposed into 4 pixels.
        const int cbase = ch * 32;
        for (int it = tid; it < band_items; it += kNT) {
            const int cg = it & 3;
            const int rq = it >> 2;
            const int r = rq / nq, q4 = rq - r * nq;
            const int hin = ir0 + r;
            const int win = ic0 + q4 * 4;
            const bool rowok = (unsigned)hin < (unsigned)a.H && (unsigned)win < (unsigned)a.W;
            float v[8][4];
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                const int c = cbase + cg * 8 + j;
                floatx4 x = {0.f, 0.f, 0.f, 0.f};
                if (rowok && c < a.C)
                    x = *reinterpret_cast<const floatx4*>(a.in + in_img +
                                                          ((int64_t)c * a.H + hin) * a.W + win);
#pragma unroll
                for (int q = 0; q < 4; ++q) v[j][q] = x[q];
            }
            const int p0 = r * a.BC4 + q4 * 4;
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                float col[8];
#pragma unroll
                for (int j = 0; j < 8; ++j) col[j] = v[j][q];
                *reinterpret_cast<half8*>(bl + band_off(p0 + q, cg)) = pack8(col);
            }
        }
        __syncthreads();

        // MFMAs over every tap of this channel chunk.
        for (int t = 0; t < P.T; ++t) {
            for (int u = 0; u < P.U; ++u) {
                const int tap = t * P.U + u;
                const int tapoff = t * a.BC4 + u;
                half8 fa[2], fb[PGW];
#pragma unroll
                for (int fi = 0; fi < 2; ++fi)
                    fa[fi] = lds_read8<32>(wl + tap * 2048, (wf * 2 + fi) * 16 + (lane & 15),
                                           lane >> 4);
#pragma unroll
                for (int i = 0; i < PGW; ++i)
                    fb[i] = *reinterpret_cast<const half8*>(bl + band_off(pbase[i] + tapoff,
                                                                          lane >> 4));
#pragma unroll
                for (int fi = 0; fi < 2; ++fi)
#pragma unroll
                    for (int i = 0; i < PGW; ++i) acc[fi][i] = mfma16x16x32(fa[fi], fb[i], acc[fi][i]);
            }
        }
    }

    // Store: lane holds rows f = 4*(lane/16) + r of a 16x16 tile, column = pixel lane%16.
#pragma unroll
    for (int i = 0; i < PGW; ++i) {
        const int px = (wp * PGW + i) * 16 + (lane & 15);
        if (px >= tile_px) continue;
        const int ohl = px / a.WC, owl = px - ohl * a.WC;
        const int oh = oh0 + ohl, ow = ow0 + owl;
        if (oh >= P.Ho || ow >= P.Wo) continue;
        const int64_t opix = (int64_t)(oh * a.osh + P.oph) * a.Wout + ow * a.osw + P.opw;
#pragma unroll
        for (int fi = 0; fi < 2; ++fi) {
            const int fb0 = ftile * 64 + (wf * 2 + fi) * 16 + 4 * (lane >> 4);
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int f = fb0 + r;
                if (f >= a.F) continue;
                const int64_t oi = ((int64_t)b * a.F + f) * a.Hout * a.Wout + opix;
                if (a.epi.bias || a.epi.act)
                    epilogue(a.out + oi, a.epi.mask ? a.epi.mask + oi : nullptr, acc[fi][i][r],
                             a.epi.bias ? a.epi.bias[f] : 0.f, a.epi.act);
                else
                    a.out[oi] = acc[fi][i][r];
            }
        }
    }
}

// Wk[ftile][chunk][tap][f64][c32] for a forward convolution: W is [F, C, R, S].
// Index math is 32-bit (the host keeps the prepared tensor below 2^31
// elements): 64-bit division is a long software sequence on the GPU.
__global__ void prep_fwd_weights(const float* __restrict__ W, half_t* __restrict__ wk, int F, int C,
                                 int R, int S, int nchunks, int total) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= total) return;
    const int c32 = i & 31, f64 = (i >> 5) & 63;
    int rest = i >> 11;
    const int taps = R * S;
    const int tap = rest % taps;
    rest /= taps;
    const int chunk = rest % nchunks;
    const int ftile = rest / nchunks;
    const int f = ftile * 64 + f64, c = chunk * 32 + c32;
    const int t = tap / S, u = tap - t * S;
    float v = 0.f;
    if (f < F && c < C) v = W[(((int64_t)f * C + c) * R + t) * S + u];
    wk[i] = to_half(v);
}

// Tap geometry of the stride phases of a dX weight preparation: phase z's
// prepared weights are halves [begin[z], begin[z+1]) of Wk, in phase order.
struct DgradPrepPhases {
    int nphase;
    int64_t begin[kBandMaxPhases + 1];
    int T[kBandMaxPhases], U[kBandMaxPhases], r0h[kBandMaxPhases], r0w[kBandMaxPhases];
};

// Wk for the stride phases of the transposed convolution (conv dX), all
// phases in one launch: the band kernel's output channel is the conv input
// channel c (< Cc), its input channel is the conv output channel f (< Fc);
// tap (t, u) of phase z reads W[f, c, r0h + sh*(T-1-t), r0w + sw*(U-1-u)]
// (W is [Fc, Cc, R, S]).
__global__ void prep_dgrad_weights(const float* __restrict__ W, half_t* __restrict__ wk, int Fc,
                                   int Cc, int R, int S, int sh, int sw, int nchunks,
                                   const DgradPrepPhases pp) {
    const int gi = blockIdx.x * blockDim.x + threadIdx.x;  // < 2^31 (host check)
    if (gi >= pp.begin[pp.nphase]) return;
    int z = 0;
    while (z + 1 < pp.nphase && gi >= pp.begin[z + 1]) ++z;
    const int i = gi - (int)pp.begin[z];
    const int T = pp.T[z], U = pp.U[z];
    const int k32 = i & 31, o64 = (i >> 5) & 63;
    int rest = i >> 11;
    const int taps = T * U;
    const int tap = rest % taps;
    rest /= taps;
    const int chunk = rest % nchunks;
    const int otile = rest / nchunks;
    const int c = otile * 64 + o64;   // conv input channel = band output channel
    const int f = chunk * 32 + k32;   // conv output channel = band input channel
    const int t = tap / U, u = tap - t * U;
    const int r = pp.r0h[z] + sh * (T - 1 - t), s = pp.r0w[z] + sw * (U - 1 - u);
    float v = 0.f;
    if (c < Cc && f < Fc) v = W[(((int64_t)f * Cc + c) * R + r) * S + s];
    wk[gi] = to_half(v);
}

int ceil_div(int a, int b) { return (a + b - 1) / b; }

// Chooses the output tile (TH x WC, at most 224 pixels so that each wave owns
// at most 7 pixel groups of 16) and checks the LDS budget.
bool plan_tile(BandConvArgs& a) {
    int max_ho = 0, max_wo = 0;
    a.max_taps = 0;
    for (int z = 0; z < a.nphase; ++z) {
        max_ho = std::max(max_ho, a.ph[z].Ho);
        max_wo = std::max(max_wo, a.ph[z].Wo);
        a.max_taps = std::max(a.max_taps, a.ph[z].T * a.ph[z].U);
    }
    if (a.max_taps > kBandMaxTaps) return false;
    if (max_ho == 0 || max_wo == 0) return true;
    int max_t = 0, max_u = 0;
    for (int z = 0; z < a.nphase; ++z) {
        max_t = std::max(max_t, a.ph[z].T);
        max_u = std::max(max_u, a.ph[z].U);
    }
    a.WC = std::min(max_wo, 224);
    // The tallest tile whose band fits half the LDS (two blocks per CU: one
    // block's loads run under the other's taps; 3x3 s2 64 -> 128 at 56^2
    // forward 61 -> 50 us), else the whole LDS.
    for (int cap : {kBandMaxLds / 2, kBandMaxLds}) {
        for (a.TH = std::max(1, std::min(max_ho, 224 / a.WC)); a.TH >= 1; --a.TH) {
            a.BR = (a.TH - 1) * a.ish + std::max(max_t, 1);
            a.BC4 = ((a.WC - 1) * a.isw + std::max(max_u, 1) + 3 + 3) & ~3;
            a.lds_bytes = (int64_t)a.max_taps * 2048 * 2 + (int64_t)a.BR * a.BC4 * 64;
            if (a.lds_bytes <= cap) break;
        }
        if (a.TH >= 1) break;
    }
    if (a.TH < 1) return false;
    for (int z = 0, blocks = 0; z < a.nphase; ++z) {
        BandPhase& p = a.ph[z];
        p.nrb = ceil_div(p.Ho, a.TH);
        p.ncb = ceil_div(p.Wo, a.WC);
        p.block0 = blocks;
        blocks += a.B * p.nrb * p.ncb;
        a.nblocks = blocks;
    }
    return true;
}

// Software-pipelined variant of band_conv_kernel for small bands (the stride
// phases of a transposed convolution): the loads of chunk ch+1 (weights and
// band, into registers) are issued before the taps of chunk ch and written to
// the other of two LDS stages after them, so the load latency hides behind
// the MFMAs; one barrier per chunk. Same arithmetic, in the same order, as
// band_conv_kernel. TAPS >= taps of every phase and ITEMS >= band items per
// thread (host checks); the band is read through a buffer resource over one
// image (host check: the image spans less than kMaxTileSpanBytes), so rows,
// columns and channels outside it read 0.
template <int PGW, int TAPS, int ITEMS>
__global__ __launch_bounds__(kNT) void band_conv_pipe(const BandConvArgs a) {
    extern __shared__ __attribute__((aligned(16))) half_t smem[];
    const int bx = blockIdx.x;
    int z = 0;
    while (z + 1 < a.nphase && bx >= a.ph[z + 1].block0) ++z;
    const BandPhase& P = a.ph[z];
    int local = bx - P.block0;
    const int cb = local % P.ncb;
    local /= P.ncb;
    const int rb = local % P.nrb;
    const int b = local / P.nrb;
    const int oh0 = rb * a.TH, ow0 = cb * a.WC;
    const int ftile = blockIdx.y;
    const int taps = P.T * P.U;
    const int stage = a.max_taps * 2048 + a.BR * a.BC4 * 32;  // halves per LDS stage

    const int ir0 = oh0 * a.ish - P.iph;
    const int icr = ow0 * a.isw - P.ipw;
    const int ic0 = icr >= 0 ? (icr & ~3) : -((-icr + 3) & ~3);
    const int coff = icr - ic0;

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wf = wave & 1, wp = wave >> 1;
    const int tile_px = a.TH * a.WC;
    int pbase[PGW];
#pragma unroll
    for (int i = 0; i < PGW; ++i) {
        int px = (wp * PGW + i) * 16 + (lane & 15);
        if (px >= tile_px) px = 0;
        const int ohl = px / a.WC, owl = px - ohl * a.WC;
        pbase[i] = ohl * a.ish * a.BC4 + owl * a.isw + coff;
    }
    floatx4_t acc[2][PGW];
#pragma unroll
    for (int fi = 0; fi < 2; ++fi)
#pragma unroll
        for (int i = 0; i < PGW; ++i) acc[fi][i] = floatx4_t{0.f, 0.f, 0.f, 0.f};

    const int nq = a.BC4 >> 2;
    const int band_items = a.BR * nq * 4;
    const half_t* wsrc_base = a.wk + P.woff + (int64_t)ftile * a.nchunks * taps * 2048;
    const rsrc_t isrc = make_rsrc_in(a.in, (int64_t)a.B * a.C * a.H * a.W, (int64_t)b * a.C * a.H * a.W);
    const uint32_t cstride = (uint32_t)(a.H * a.W * 4);
    // Per item: (row, quad, 8-channel group); the byte offset of its first
    // element at channel 0 (kBufOOB: outside the image) and its band pixel.
    uint32_t ioff[ITEMS];
    int icg[ITEMS], ip0[ITEMS];
    bool ilive[ITEMS];
#pragma unroll
    for (int k = 0; k < ITEMS; ++k) {
        const int it = tid + k * kNT;
        ilive[k] = it < band_items;
        const int cg = it & 3, rq = it >> 2;
        const int r = rq / nq, q4 = rq - r * nq;
        const int hin = ir0 + r, win = ic0 + q4 * 4;
        const bool ok = ilive[k] && (unsigned)hin < (unsigned)a.H && (unsigned)win < (unsigned)a.W;
        ioff[k] = ok ? (uint32_t)(((cg * 8) * a.H + hin) * a.W + win) * 4u : kBufOOB;
        icg[k] = cg;
        ip0[k] = r * a.BC4 + q4 * 4;
    }
    half8 wv[TAPS];
    floatx4 bv[ITEMS][8];
    auto load_chunk = [&](int ch) {
        const half_t* wsrc = wsrc_base + (int64_t)ch * taps * 2048;
#pragma unroll
        for (int tp = 0; tp < TAPS; ++tp)
            if (tp < taps) wv[tp] = *reinterpret_cast<const half8*>(wsrc + (tp * 256 + tid) * 8);
        const uint32_t cbase = (uint32_t)(ch * 32) * cstride;
#pragma unroll
        for (int k = 0; k < ITEMS; ++k)
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                // channel ch*32 + 8*cg + j: out of range channels read 0
                const bool cok = ch * 32 + icg[k] * 8 + j < a.C;
                bv[k][j] = buf_load4s(isrc, cok ? ioff[k] : kBufOOB, cbase + j * cstride);
            }
    };
    auto store_chunk = [&](int stg) {
        half_t* const wl = smem + stg * stage;
        half_t* const bl = wl + a.max_taps * 2048;
#pragma unroll
        for (int tp = 0; tp < TAPS; ++tp)
            if (tp < taps) lds_write8<32>(wl + tp * 2048, tid >> 2, tid & 3, wv[tp]);
#pragma unroll
        for (int k = 0; k < ITEMS; ++k) {
            if (!ilive[k]) continue;
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                float col[8];
#pragma unroll
                for (int j = 0; j < 8; ++j) col[j] = bv[k][j][q];
                *reinterpret_cast<half8*>(bl + band_off(ip0[k] + q, icg[k])) = pack8(col);
            }
        }
    };
    load_chunk(0);
    store_chunk(0);
    __syncthreads();
    for (int ch = 0; ch < a.nchunks; ++ch) {
        const bool more = ch + 1 < a.nchunks;
        if (more) load_chunk(ch + 1);  // registers of chunk ch were written to LDS
        const half_t* const wl = smem + (ch & 1) * stage;
        const half_t* const bl = wl + a.max_taps * 2048;
        for (int t = 0; t < P.T; ++t) {
            for (int u = 0; u < P.U; ++u) {
                const int tap = t * P.U + u;
                const int tapoff = t * a.BC4 + u;
                half8 fa[2], fb[PGW];
#pragma unroll
                for (int fi = 0; fi < 2; ++fi)
                    fa[fi] = lds_read8<32>(wl + tap * 2048, (wf * 2 + fi) * 16 + (lane & 15), lane >> 4);
#pragma unroll
                for (int i = 0; i < PGW; ++i)
                    fb[i] = *reinterpret_cast<const half8*>(bl + band_off(pbase[i] + tapoff, lane >> 4));
#pragma unroll
                for (int fi = 0; fi < 2; ++fi)
#pragma unroll
                    for (int i = 0; i < PGW; ++i) acc[fi][i] = mfma16x16x32(fa[fi], fb[i], acc[fi][i]);
            }
        }
        if (more) store_chunk((ch + 1) & 1);
        __syncthreads();
    }
#pragma unroll
    for (int i = 0; i < PGW; ++i) {
        const int px = (wp * PGW + i) * 16 + (lane & 15);
        if (px >= tile_px) continue;
        const int ohl = px / a.WC, owl = px - ohl * a.WC;
        const int oh = oh0 + ohl, ow = ow0 + owl;
        if (oh >= P.Ho || ow >= P.Wo) continue;
        const int64_t opix = (int64_t)(oh * a.osh + P.oph) * a.Wout + ow * a.osw + P.opw;
#pragma unroll
        for (int fi = 0; fi < 2; ++fi) {
            const int fb0 = ftile * 64 + (wf * 2 + fi) * 16 + 4 * (lane >> 4);
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int f = fb0 + r;
                if (f >= a.F) continue;
                const int64_t oi = ((int64_t)b * a.F + f) * a.Hout * a.Wout + opix;
                if (a.epi.bias || a.epi.act)
                    epilogue(a.out + oi, a.epi.mask ? a.epi.mask + oi : nullptr, acc[fi][i][r],
                             a.epi.bias ? a.epi.bias[f] : 0.f, a.epi.act);
                else
                    a.out[oi] = acc[fi][i][r];
            }
        }
    }
}

template <int PGW>
hipError_t launch_pgw(const BandConvArgs& a, hipStream_t st) {
    auto kern = band_conv_kernel<PGW>;
    if (a.lds_bytes > 65536) {
        hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(kern),
                                           hipFuncAttributeMaxDynamicSharedMemorySize,
                                           (int)a.lds_bytes);
        if (e != hipSuccess) return e;
    }
    hipLaunchKernelGGL(kern, dim3(a.nblocks, a.nftiles), dim3(kNT), (size_t)a.lds_bytes, st, a);
    return hipGetLastError();
}

constexpr int kPipeTaps = 4, kPipeItems = 2;

template <int PGW>
hipError_t launch_pipe(const BandConvArgs& a, hipStream_t st) {
    auto kern = band_conv_pipe<PGW, kPipeTaps, kPipeItems>;
    hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(kern),
                                       hipFuncAttributeMaxDynamicSharedMemorySize,
                                       (int)a.lds_bytes);
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL(kern, dim3(a.nblocks, a.nftiles), dim3(kNT), (size_t)a.lds_bytes, st, a);
    return hipGetLastError();
}

int launch_band(const BandConvArgs& a, hipStream_t st) {
    if (a.nblocks == 0 || a.nftiles == 0) return SEERA_OK;
    const int pgw = ceil_div(ceil_div(a.TH * a.WC, 16), 2);
    hipError_t e;
    const int items = ceil_div(a.BR * (a.BC4 >> 2) * 4, kNT);
    if (a.max_taps <= kPipeTaps && items <= kPipeItems && 2 * a.lds_bytes <= kBandMaxLds &&
        (int64_t)a.C * a.H * a.W * 4 < kMaxTileSpanBytes) {
        BandConvArgs p = a;
        p.lds_bytes = 2 * a.lds_bytes;  // two stages
        switch (pgw) {
            case 1: e = launch_pipe<1>(p, st); break;
            case 2: e = launch_pipe<2>(p, st); break;
            case 3: e = launch_pipe<3>(p, st); break;
            case 4: e = launch_pipe<4>(p, st); break;
            case 5: e = launch_pipe<5>(p, st); break;
            case 6: e = launch_pipe<6>(p, st); break;
            default: e = launch_pipe<7>(p, st); break;
        }
        if (e != hipSuccess) return fail_hip(e, "band conv launch");
        return SEERA_OK;
    }
    switch (pgw) {
        case 1: e = launch_pgw<1>(a, st); break;
        case 2: e = launch_pgw<2>(a, st); break;
        case 3: e = launch_pgw<3>(a, st); break;
        case 4: e = launch_pgw<4>(a, st); break;
        case 5: e = launch_pgw<5>(a, st); break;
        case 6: e = launch_pgw<6>(a, st); break;
        default: e = launch_pgw<7>(a, st); break;
    }
    if (e != hipSuccess) return fail_hip(e, "band conv launch");
    return SEERA_OK;
}


// ---------------------------------------------------------------------------
// Weight gradient (convolution.cu:268-366, 431-452; upsampling.cu:202-301):
//   dW[f, c, r, s] = sum_{b, oh, ow} dY[b, f, oh, ow] * X[b, c, oh*sh - ph + r, ow*sw - pw + s]
// a GEMM with M = filters, N = (tap, channel), K = output pixels. A block owns
// 64 filters x CT channels x all taps and walks `ips` output tiles (TH x WC8
// pixels of one image), accumulating in registers. Per tile it stages the
// dY tile [64 f][pixels] and, per 32-channel chunk, S column-shifted fp16
// copies of the X band: copy s holds X[c, row, ow*sw - pw + s] at column ow,
// so every tap's B fragment (8 consecutive pixels of one channel) is one
// aligned 16-byte LDS read. Row strides are 16 bytes past a multiple of
// 128 bytes, so the 16 lanes of a fragment read (16 filters or 16 channels
// at one pixel chunk) hit distinct banks. Each block writes its partial sum;
// wgrad_reduce adds the partials in a fixed order.
// ---------------------------------------------------------------------------

// The loaded columns of one X item, held as one vector value (never an
// addressable array, so it stays in registers).
typedef float floatx44 __attribute__((ext_vector_type(44)));

// v[j] = element O + j*SW of the window (0 past its end); compile-time indices.
template <int O, int SW>
__device__ __forceinline__ void pick_at(const floatx44& w, float (&v)[8]) {
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        const int e = O + j * SW;
        v[j] = e < 44 ? w[e] : 0.f;
    }
}

// Writes octets OC.. of one X item into shifted copy O - (band alignment):
// octet m = grp*OCT + OC holds w[O + 8*OC*SW + j*SW]. Copy rows are padded to
// a whole number of items (xrow), so every octet of an item has a slot.
template <int O, int OC, int SW, int OCT>
__device__ __forceinline__ void write_octets(const floatx44& w, int grp, half_t* dst) {
    if constexpr (OC < OCT) {
        float v[8];
        pick_at<O + 8 * OC * SW, SW>(w, v);
        *reinterpret_cast<half8*>(dst + 8 * (grp * OCT + OC)) = pack8(v);
        write_octets<O, OC + 1, SW, OCT>(w, grp, dst);
    }
}

// Writes the S (<= 7) tap-shifted copies of one X item; OFF is the band's
// column alignment (0..3), so every register index is a compile-time constant.
template <int OFF, int SI, int SW, int OCT>
__device__ __forceinline__ void write_shifts(const floatx44& w, int S, int grp, half_t* dst,
                                             int plane) {
    if constexpr (SI < 7) {
        if (SI < S) {
            write_octets<OFF + SI, 0, SW, OCT>(w, grp, dst + SI * plane);
            write_shifts<OFF, SI + 1, SW, OCT>(w, S, grp, dst, plane);
        }
    }
}

// X item = OCT 8-column octets of one channel row; its F4 float4 loads cover
// the octets' columns for every tap shift (offset <= 3 + S - 1 <= 9, S <= 7).
template <int SW>
struct XItem {
    static constexpr int OCT = SW == 1 ? 4 : 2;
    static constexpr int F4 = (9 + (8 * OCT - 1) * SW + 1 + 3) / 4;
};

// As write_octets, zeroing the columns >= valid_cols (edge tiles only).
template <int O, int OC, int SW, int OCT>
__device__ __forceinline__ void write_octets_edge(const floatx44& w, int grp, int valid_cols,
                                                  half_t* dst) {
    if constexpr (OC < OCT) {
        const int m = grp * OCT + OC;
        float v[8];
        pick_at<O + 8 * OC * SW, SW>(w, v);
#pragma unroll
        for (int j = 0; j < 8; ++j)
            if (8 * m + j >= valid_cols) v[j] = 0.f;
        *reinterpret_cast<half8*>(dst + 8 * m) = pack8(v);
        write_octets_edge<O, OC + 1, SW, OCT>(w, grp, valid_cols, dst);
    }
}

template <int OFF, int SI, int SW, int OCT>
__device__ __forceinline__ void write_shifts_edge(const floatx44& w, int S, int grp,
                                                  int valid_cols, half_t* dst, int plane) {
    if constexpr (SI < 7) {
        if (SI < S) {
            write_octets_edge<OFF + SI, 0, SW, OCT>(w, grp, valid_cols, dst + SI * plane);
            write_shifts_edge<OFF, SI + 1, SW, OCT>(w, S, grp, valid_cols, dst, plane);
        }
    }
}

constexpr int kWgNT = 512;    // 4 consumer waves (MFMA) + 4 producer waves (loads, fp16 copies)
constexpr int kWgProd = 256;  // producer threads
constexpr int kWgDyMax = 4;   // dY items (8 columns of one filter row) per producer thread
constexpr int kWgKsMax = 7;   // 32-pixel k-steps per tile

// Warp-specialised pipeline over steps (tile, 32-channel chunk) of this block.
// At step k the consumer waves run the MFMAs of step k from LDS stage k&1
// while the producer waves write step k+1 (fp16 dY tile on a tile's first
// chunk, S shifted fp16 X copies) into stage (k+1)&1 from registers loaded
// during step k-1, then issue the global loads of step k+2. One barrier per
// step; a consumer and a producer share each SIMD, so the conversion VALU
// work and the MFMAs run side by side and HBM loads stay in flight.
template <int NGW, int SW, int NCH>
__global__ __launch_bounds__(kWgNT) void band_wgrad_kernel(const WgradArgs a) {
    using XI = XItem<SW>;
    static_assert(XI::F4 <= 11, "window exceeds 44 floats");
    extern __shared__ __attribute__((aligned(16))) half_t smem[];
    const int dy_stage = 64 * a.dy_stride;              // halves per dY buffer
    const int x_stage = a.S * 32 * a.x_plane;           // halves per X copies buffer
    half_t* const dyb = smem;                           // [2] dY tile, by tile parity
    half_t* const xb2 = smem + 2 * dy_stage;            // [2] X copies, by step parity

    const int split = blockIdx.x, ty = blockIdx.y;
    const int ftile = ty / a.nctile, ctile = ty - ftile * a.nctile;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const bool consumer = wave < 4;
    const int it0 = split * a.ips, it1 = min(a.items, it0 + a.ips);
    const int nsteps = max(0, it1 - it0) * NCH;

    auto tile_b = [&](int item) { return item / a.ncb / a.nrb; };
    auto tile_oh0 = [&](int item) { return (item / a.ncb % a.nrb) * a.TH; };
    auto tile_ow0 = [&](int item) { return item % a.ncb * a.WC8; };
    auto floor4 = [](int v) { return v >= 0 ? (v & ~3) : -((-v + 3) & ~3); };

    if (consumer) {
        // ---------------- consumer: MFMAs ----------------
        const int ngc = 2 * a.R * a.S;                  // 16-channel groups per chunk
        int boff[NGW];
        bool gon[NGW];
#pragma unroll
        for (int i = 0; i < NGW; ++i) {
            const int g = wave + 4 * i;
            const int tap = g >> 1, half = g & 1;
            const int r = tap / a.S, sc = tap - r * a.S;
            gon[i] = g < ngc;
            boff[i] = (sc * 32 + half * 16 + (lane & 15)) * a.x_plane + r * a.xrow;
        }
        int apx[kWgKsMax], xpix[kWgKsMax];
#pragma unroll
        for (int ks = 0; ks < kWgKsMax; ++ks) {
            const int px0 = ks * 32 + 8 * (lane >> 4);
            const int ohl = px0 / a.WC8, owl = px0 - ohl * a.WC8;
            apx[ks] = px0;
            xpix[ks] = ohl * a.sh * a.xrow + owl;
        }
        floatx4_t acc[NCH][NGW][4];
#pragma unroll
        for (int c = 0; c < NCH; ++c)
#pragma unroll
            for (int i = 0; i < NGW; ++i)
#pragma unroll
                for (int fg = 0; fg < 4; ++fg) acc[c][i][fg] = floatx4_t{0.f, 0.f, 0.f, 0.f};

        __syncthreads();  // stage 0 written
        for (int k = 0; k < nsteps; ++k) {
            const int item = it0 + k / NCH;
            const half_t* const dyl = dyb + ((item - it0) & 1) * dy_stage;
            const half_t* const xl = xb2 + (k & 1) * x_stage;
#pragma unroll
            for (int c = 0; c < NCH; ++c) {
                if (c != k % NCH) continue;
#pragma unroll
                for (int ks = 0; ks < kWgKsMax; ++ks) {
                    if (ks >= a.KS) break;
                    half8 fa[4], fb[NGW];
#pragma unroll
                    for (int fg = 0; fg < 4; ++fg)
                        fa[fg] = *reinterpret_cast<const half8*>(
                            dyl + (fg * 16 + (lane & 15)) * a.dy_stride + apx[ks]);
#pragma unroll
                    for (int i = 0; i < NGW; ++i)
                        if (gon[i]) fb[i] = *reinterpret_cast<const half8*>(xl + boff[i] + xpix[ks]);
#pragma unroll
                    for (int i = 0; i < NGW; ++i) {
                        if (!gon[i]) continue;
#pragma unroll
                        for (int fg = 0; fg < 4; ++fg)
                            acc[c][i][fg] = mfma16x16x32(fa[fg], fb[i], acc[c][i][fg]);
                    }
                }
            }
            __syncthreads();
        }
        // Partial sums: part[ty][split][f64][n], n = tap * CT + channel in the tile.
        const int ntot = a.CT * a.R * a.S;
        float* const dst = a.part + ((int64_t)ty * a.nsplit + split) * 64 * ntot;
#pragma unroll
        for (int c = 0; c < NCH; ++c)
#pragma unroll
            for (int i = 0; i < NGW; ++i) {
                if (!gon[i]) continue;
                const int g = wave + 4 * i;
                const int n = (g >> 1) * a.CT + c * 32 + (g & 1) * 16 + (lane & 15);
#pragma unroll
                for (int fg = 0; fg < 4; ++fg)
#pragma unroll
                    for (int r = 0; r < 4; ++r)
                        dst[(int64_t)(fg * 16 + 4 * (lane >> 4) + r) * ntot + n] = acc[c][i][fg][r];
            }
        return;
    }

    // ---------------- producer: loads and fp16 copies ----------------
    const int ptid = tid - 256;
    const int noct = a.WC8 >> 3;
    const int ngrp = (noct + XI::OCT - 1) / XI::OCT;
    const int dy_items = 64 * a.TH * noct;
    const int x_items = 32 * a.BR * ngrp;
    const int f_lim = a.F - ftile * 64;
    int dyit[kWgDyMax];
#pragma unroll
    for (int kk = 0; kk < kWgDyMax; ++kk) {
        const int it = ptid + kk * kWgProd;
        const int m = it % noct, rest = it / noct;
        dyit[kk] = it < dy_items ? ((rest / a.TH) | (rest % a.TH) << 8 | m << 16) : -1;
    }
    // Channel fastest across lanes: the copy planes of consecutive channels are
    // 16 bytes apart modulo 128, so a wave's 16-byte copy writes spread over
    // all banks.
    int xit = -1;
    if (ptid < x_items) {
        const int cl = ptid % 32, rest = ptid / 32;
        xit = cl | (rest % a.BR) << 8 | (rest / a.BR) << 16;
    }
    // Two register sets: the loads of step j+2 are issued right after step j
    // is written, so each load has two consumer steps to arrive.
    floatx4 dyv0[kWgDyMax][2], dyv1[kWgDyMax][2];
    floatx44 xw0, xw1;

    // Write step J (registers DYV/XW -> LDS stage J&1).
#define SEERA_WG_WRITE(J, DYV, XW)                                                          \
    {                                                                                       \
        const int item = it0 + (J) / NCH, ch = (J) % NCH;                                   \
        const int ow0 = tile_ow0(item);                                                     \
        if (ch == 0) {                                                                      \
            half_t* const dyl = dyb + ((item - it0) & 1) * dy_stage;                        \
            _Pragma("unroll") for (int kk = 0; kk < kWgDyMax; ++kk) {                       \
                if (dyit[kk] < 0) continue;                                                 \
                const int fl = dyit[kk] & 255, ohl = (dyit[kk] >> 8) & 255, m = dyit[kk] >> 16; \
                float f8[8];                                                                \
                _Pragma("unroll") for (int q = 0; q < 4; ++q) {                             \
                    f8[q] = DYV[kk][0][q];                                                  \
                    f8[4 + q] = DYV[kk][1][q];                                              \
                }                                                                           \
                *reinterpret_cast<half8*>(dyl + fl * a.dy_stride + ohl * a.WC8 + 8 * m) =   \
                    pack8(f8);                                                              \
            }                                                                               \
        }                                                                                   \
        if (xit >= 0) {                                                                     \
            const int cl = xit & 255, row = (xit >> 8) & 255, grp = xit >> 16;              \
            half_t* const dst = xb2 + ((J) & 1) * x_stage + cl * a.x_plane + row * a.xrow;  \
            const int plane = 32 * a.x_plane;                                               \
            const int xc0 = ow0 * a.sw - a.pw;                                              \
            const int valid_cols = a.Wo - ow0;                                              \
            if (valid_cols >= a.WC8) {                                                      \
                switch (xc0 - floor4(xc0)) { /* uniform across the block */                 \
                    case 0: write_shifts<0, 0, SW, XI::OCT>(XW, a.S, grp, dst, plane); break; \
                    case 1: write_shifts<1, 0, SW, XI::OCT>(XW, a.S, grp, dst, plane); break; \
                    case 2: write_shifts<2, 0, SW, XI::OCT>(XW, a.S, grp, dst, plane); break; \
                    default: write_shifts<3, 0, SW, XI::OCT>(XW, a.S, grp, dst, plane); break; \
                }                                                                           \
            } else {                                                                        \
                /* Edge tile: columns past the output width get 0 (their dY is */          \
                /* zero; this keeps 0 * inf from turning into NaN). */                      \
                switch (xc0 - floor4(xc0)) {                                                \
                    case 0: write_shifts_edge<0, 0, SW, XI::OCT>(XW, a.S, grp, valid_cols, dst, plane); break; \
                    case 1: write_shifts_edge<1, 0, SW, XI::OCT>(XW, a.S, grp, valid_cols, dst, plane); break; \
                    case 2: write_shifts_edge<2, 0, SW, XI::OCT>(XW, a.S, grp, valid_cols, dst, plane); break; \
                    default: write_shifts_edge<3, 0, SW, XI::OCT>(XW, a.S, grp, valid_cols, dst, plane); break; \
                }                                                                           \
            }                                                                               \
        }                                                                                   \
    }
    // Issue the global loads of step J into DYV/XW. Every lane issues the same
    // loads in every step (out-of-range elements, lanes without an item and
    // the X tail beyond XI::F4 get offsets past num_records and read 0): with
    // a fixed load count the compiler's vmcnt waits stay exact, and a write
    // waits only for its own step's loads, not for the step issued after it.
    // Buffer resources cover this image's dY rows of the filter tile and its
    // X planes (host check: each spans less than kMaxTileSpanBytes).
#define SEERA_WG_LOAD(J, DYV, XW)                                                           \
    {                                                                                       \
        const int item = it0 + (J) / NCH, ch = (J) % NCH;                                   \
        const int b = tile_b(item), oh0 = tile_oh0(item), ow0 = tile_ow0(item);             \
        if (ch == 0) {                                                                      \
            const rsrc_t dsrc = make_rsrc_in(a.dy, (int64_t)a.B * a.F * a.Ho * a.Wo, ((int64_t)b * a.F + ftile * 64) * a.Ho * a.Wo); \
            _Pragma("unroll") for (int kk = 0; kk < kWgDyMax; ++kk) {                       \
                const int fl = dyit[kk] & 255, ohl = (dyit[kk] >> 8) & 255, m = dyit[kk] >> 16; \
                const int oh = oh0 + ohl, ow = ow0 + 8 * m;                                 \
                const bool ok = dyit[kk] >= 0 && fl < f_lim && oh < a.Ho;                   \
                const uint32_t off = (uint32_t)(((fl * a.Ho + oh) * a.Wo + ow) * 4);        \
                _Pragma("unroll") for (int h = 0; h < 2; ++h)                               \
                    DYV[kk][h] = buf_load4(dsrc,                          \
                                           ok && ow + 4 * h < a.Wo ? off + 16u * h : kBufOOB); \
            }                                                                               \
        }                                                                                   \
        {                                                                                   \
            const int cl = xit & 255, row = (xit >> 8) & 255, grp = xit >> 16;              \
            const int c = ctile * a.CT + ch * 32 + cl, hin = oh0 * a.sh - a.ph + row;       \
            const int a0 = floor4(ow0 * a.sw - a.pw) + 8 * XI::OCT * grp * SW;              \
            const bool rowok = xit >= 0 && c < a.C && (unsigned)hin < (unsigned)a.H;        \
            const rsrc_t xsrc = make_rsrc_in(a.x, (int64_t)a.B * a.C * a.H * a.W, (int64_t)b * a.C * a.H * a.W); \
            const int rbase = rowok ? (c * a.H + hin) * a.W : 0;                            \
            _Pragma("unroll") for (int q = 0; q < 11; ++q) {                                \
                const int col = a0 + 4 * q;                                                 \
                floatx4 x4 = {0.f, 0.f, 0.f, 0.f};                                          \
                if (q < XI::F4)                                                             \
                    x4 = buf_load4(xsrc, rowok && (unsigned)col < (unsigned)a.W             \
                                             ? (uint32_t)((rbase + col) * 4) : kBufOOB);    \
                _Pragma("unroll") for (int e = 0; e < 4; ++e) XW[4 * q + e] = x4[e];        \
            }                                                                               \
        }                                                                                   \
    }

    // Steps 0 and 1 in flight, then per step j: write j, load j+2 into the
    // registers j just freed (past the last step: the last step again, never
    // written), and meet the consumers at the barrier that releases step j.
    if (nsteps == 0) return;
    SEERA_WG_LOAD(0, dyv0, xw0)
    SEERA_WG_LOAD(min(1, nsteps - 1), dyv1, xw1)
    int j = 0;
    for (; j + 1 < nsteps; j += 2) {
        SEERA_WG_WRITE(j, dyv0, xw0)
        SEERA_WG_LOAD(min(j + 2, nsteps - 1), dyv0, xw0)
        __syncthreads();
        SEERA_WG_WRITE(j + 1, dyv1, xw1)
        SEERA_WG_LOAD(min(j + 3, nsteps - 1), dyv1, xw1)
        __syncthreads();
    }
    if (j < nsteps) {
        SEERA_WG_WRITE(j, dyv0, xw0)
        __syncthreads();
    }
#undef SEERA_WG_WRITE
#undef SEERA_WG_LOAD
    __builtin_amdgcn_s_waitcnt(0);  // the unused last loads land before the wave ends
    __syncthreads();  // matches the consumers' final barrier
}

// dW[f, c, r, s] = sum over splits of the partials, in a fixed order. A block
// covers 64 consecutive partial columns (contiguous reads across the wave)
// and four groups of splits; each thread sums its group with several loads in
// flight, then the four group sums are added in LDS in group order.
constexpr int kRedCols = 64, kRedGroups = 4;
__global__ __launch_bounds__(kRedCols * kRedGroups) void wgrad_reduce(
    const float* __restrict__ part, float* __restrict__ dW, int F, int C, int R, int S, int CT,
    int nctile, int ntiles, int nsplit) {
    __shared__ float red[kRedGroups][kRedCols];
    const int ntot = CT * R * S;
    const int col = threadIdx.x % kRedCols, grp = threadIdx.x / kRedCols;
    const int64_t i = (int64_t)blockIdx.x * kRedCols + col;
    const bool live = i < (int64_t)ntiles * 64 * ntot;
    const int n = live ? (int)(i % ntot) : 0;
    const int f64 = live ? (int)((i / ntot) % 64) : 0;
    const int ty = live ? (int)(i / ((int64_t)64 * ntot)) : 0;
    const float* p = part + ((int64_t)ty * nsplit * 64 + f64) * ntot + n;
    const int64_t zstride = (int64_t)64 * ntot;
    const int per = (nsplit + kRedGroups - 1) / kRedGroups;
    const int z0 = grp * per, z1 = min(nsplit, z0 + per);
    float acc = 0.f;
    if (live) {
        int z = z0;
        for (; z + 8 <= z1; z += 8) {
            float v[8];
#pragma unroll
            for (int u = 0; u < 8; ++u) v[u] = p[(z + u) * zstride];
#pragma unroll
            for (int u = 0; u < 8; ++u) acc += v[u];
        }
        for (; z < z1; ++z) acc += p[z * zstride];
    }
    red[grp][col] = acc;
    __syncthreads();
    if (grp != 0 || !live) return;
    float sum = red[0][col];
#pragma unroll
    for (int g = 1; g < kRedGroups; ++g) sum += red[g][col];
    const int f = (ty / nctile) * 64 + f64;
    const int c = (ty % nctile) * CT + n % CT;
    if (f < F && c < C) dW[((int64_t)f * C + c) * R * S + n / CT] = sum;
}

// Same sum with four consecutive partial columns per lane (16-byte loads;
// needs CT*R*S % 4 == 0, so a lane's columns share one (tile, filter) row)
// and eight groups of splits (measured: 7.3-7.8 us for cfg4's 37.7 MB; sixteen
// groups with 16 loads in flight per thread were slower, 8.4-9.0 us). The
// group sums are added in group order, as above.
constexpr int kRed4Lanes = 64, kRed4Groups = 8, kRed4Unroll = 8;

// The blocks past dW's (nb_dw of them) add the bias-gradient partials
// dbpart[ftile][split][64]: db[f] = sum over splits in split order, as eight
// groups of splits added in group order.
__device__ void db_reduce_block(const float* __restrict__ dbpart, float* __restrict__ db, int F,
                                int nsplit, int blk, floatx4 (*red)[kRed4Lanes]) {
    const int lane = threadIdx.x % kRed4Lanes, grp = threadIdx.x / kRed4Lanes;
    const int f = blk * 64 + lane;
    const int per = (nsplit + kRed4Groups - 1) / kRed4Groups;
    const int z0 = grp * per, z1 = min(nsplit, z0 + per);
    float acc = 0.f;
    if (f < F)
        for (int z = z0; z < z1; ++z) acc += dbpart[((int64_t)blk * nsplit + z) * 64 + lane];
    red[grp][lane][0] = acc;
    __syncthreads();
    if (grp != 0 || f >= F) return;
    float sum = red[0][lane][0];
#pragma unroll
    for (int g = 1; g < kRed4Groups; ++g) sum += red[g][lane][0];
    db[f] = sum;
}

__global__ __launch_bounds__(kRed4Lanes * kRed4Groups) void wgrad_reduce4(
    const float* __restrict__ part, float* __restrict__ dW, int F, int C, int R, int S, int CT,
    int nctile, int ntiles, int nsplit, const float* __restrict__ dbpart, float* __restrict__ db,
    int nb_dw) {
    __shared__ floatx4 red[kRed4Groups][kRed4Lanes];
    if ((int)blockIdx.x >= nb_dw) {
        db_reduce_block(dbpart, db, F, nsplit, (int)blockIdx.x - nb_dw, red);
        return;
    }
    const int ntot = CT * R * S;
    const int lane = threadIdx.x % kRed4Lanes, grp = threadIdx.x / kRed4Lanes;
    const int64_t i = ((int64_t)blockIdx.x * kRed4Lanes + lane) * 4;  // first of 4 columns
    const bool live = i < (int64_t)ntiles * 64 * ntot;
    const int n = live ? (int)(i % ntot) : 0;
    const int f64 = live ? (int)((i / ntot) % 64) : 0;
    const int ty = live ? (int)(i / ((int64_t)64 * ntot)) : 0;
    const float* p = part + ((int64_t)ty * nsplit * 64 + f64) * ntot + n;
    const int64_t zstride = (int64_t)64 * ntot;
    const int per = (nsplit + kRed4Groups - 1) / kRed4Groups;
    const int z0 = grp * per, z1 = min(nsplit, z0 + per);
    floatx4 acc = {0.f, 0.f, 0.f, 0.f};
    if (live) {
        int z = z0;
        for (; z + kRed4Unroll <= z1; z += kRed4Unroll) {
            floatx4 v[kRed4Unroll];
#pragma unroll
            for (int u = 0; u < kRed4Unroll; ++u)
                v[u] = *reinterpret_cast<const floatx4*>(p + (z + u) * zstride);
#pragma unroll
            for (int u = 0; u < kRed4Unroll; ++u) acc += v[u];
        }
        for (; z < z1; ++z) acc += *reinterpret_cast<const floatx4*>(p + z * zstride);
    }
    red[grp][lane] = acc;
    __syncthreads();
    if (grp != 0 || !live) return;
    floatx4 sum = red[0][lane];
#pragma unroll
    for (int g = 1; g < kRed4Groups; ++g) sum += red[g][lane];
    const int f = (ty / nctile) * 64 + f64;
    if (f >= F) return;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        const int nq = n + q;
        const int c = (ty % nctile) * CT + nq % CT;
        if (c < C) dW[((int64_t)f * C + c) * R * S + nq / CT] = sum[q];
    }
}

// Adds the partials of `ntiles` (tile, filter) rows of CT*R*S columns, and
// with dbpart the bias-gradient partials into db (CT*R*S % 4 == 0 only: the
// stride-1 row-streaming path, whose tiles are 64 channels wide).
hipError_t launch_wgrad_reduce(const float* part, float* dW, int F, int C, int R, int S, int CT,
                               int nctile, int ntiles, int nsplit, hipStream_t st,
                               const float* dbpart, float* db) {
    const int64_t total = (int64_t)ntiles * 64 * CT * R * S;
    if ((CT * R * S) % 4 == 0) {
        const int64_t cols = kRed4Lanes * 4;
        const int nb_dw = (int)((total + cols - 1) / cols);
        const int nb_db = dbpart ? (F + 63) / 64 : 0;
        hipLaunchKernelGGL(wgrad_reduce4, dim3((unsigned)(nb_dw + nb_db)),
                           dim3(kRed4Lanes * kRed4Groups), 0, st, part, dW, F, C, R, S, CT,
                           nctile, ntiles, nsplit, dbpart, db, nb_dw);
    } else {
        if (dbpart) return hipErrorInvalidValue;  // not produced on this path
        hipLaunchKernelGGL(wgrad_reduce, dim3((unsigned)((total + kRedCols - 1) / kRedCols)),
                           dim3(kRedCols * kRedGroups), 0, st, part, dW, F, C, R, S, CT, nctile,
                           ntiles, nsplit);
    }
    return hipGetLastError();
}

template <int SW, int NCH>
hipError_t launch_wgrad_sw(const WgradArgs& a, int ngw, hipStream_t st) {
    const void* k = nullptr;
    switch (ngw) {
        case 1: k = reinterpret_cast<const void*>(band_wgrad_kernel<1, SW, NCH>); break;
        case 2: k = reinterpret_cast<const void*>(band_wgrad_kernel<2, SW, NCH>); break;
        case 3: k = reinterpret_cast<const void*>(band_wgrad_kernel<3, SW, NCH>); break;
        case 4: k = reinterpret_cast<const void*>(band_wgrad_kernel<4, SW, NCH>); break;
        case 5: k = reinterpret_cast<const void*>(band_wgrad_kernel<5, SW, NCH>); break;
        default:
            // Two-chunk tiles are planned only for R*S <= 9 (at most 5 groups).
            if constexpr (NCH == 1) {
                if (ngw == 6) k = reinterpret_cast<const void*>(band_wgrad_kernel<6, SW, NCH>);
                else if (ngw == 7) k = reinterpret_cast<const void*>(band_wgrad_kernel<7, SW, NCH>);
                else k = reinterpret_cast<const void*>(band_wgrad_kernel<8, SW, NCH>);
            } else {
                return hipErrorInvalidValue;
            }
            break;
    }
    if (a.lds_bytes > 65536) {
        hipError_t e = hipFuncSetAttribute(k, hipFuncAttributeMaxDynamicSharedMemorySize,
                                           (int)a.lds_bytes);
        if (e != hipSuccess) return e;
    }
    void* args[] = {const_cast<WgradArgs*>(&a)};
    return hipLaunchKernel(k, dim3(a.nsplit, a.nftile * a.nctile), dim3(kWgNT), args,
                           (size_t)a.lds_bytes, st);
}

// Smallest stride >= n halves that is 16 bytes past a multiple of 128 bytes.
int stride16(int n) {
    n = (n + 7) & ~7;
    return n + ((8 - n % 64) + 64) % 64;
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

}  // namespace

int reduce_wgrad_partials(const float* part, float* dW, int F, int C, int R, int S, int CT,
                          int nctile, int ntiles, int nsplit, hipStream_t st, const float* dbpart,
                          float* db) {
    SEERA_HIP_TRY(launch_wgrad_reduce(part, dW, F, C, R, S, CT, nctile, ntiles, nsplit, st, dbpart,
                                      db));
    return SEERA_OK;
}

int band_conv_fwd(const float* X, const float* Wt, float* Y, int B, int C, int H, int W, int F,
                  int R, int S, int sh, int sw, int ph, int pw, hipStream_t st, bool* used,
                  const ConvEpi& epi, int x_pitch) {
    *used = false;
    const int Wx = x_pitch > W ? x_pitch : W;  // row pitch of X (zeros past W)
    if (Wx % 4 != 0 || !aligned16(X)) return SEERA_OK;
    if (R == 4 && S == 4 && sh == 2 && sw == 2 && ph == 1 && pw == 1 && !epi.bias && !epi.act &&
        Wx == W) {
        // Row streaming with column-parity planes (conv_stride2.hip) when it applies.
        bool done = false;
        SEERA_TRY(stride2_conv(X, Wt, Y, B, C, H, W, F, st, &done));
        if (done) {
            *used = true;
            return SEERA_OK;
        }
    }
    BandConvArgs a{};
    a.in = X;
    a.out = Y;
    a.epi = epi;
    a.B = B; a.C = C; a.H = H; a.W = Wx;
    a.F = F;
    a.Hout = (H + 2 * ph - R) / sh + 1;
    a.Wout = (W + 2 * pw - S) / sw + 1;
    a.ish = sh; a.isw = sw; a.osh = 1; a.osw = 1;
    a.nphase = 1;
    a.ph[0] = BandPhase{a.Hout, a.Wout, R, S, ph, pw, 0, 0, 0, 0, 0, 0};
    a.nchunks = ceil_div(C, 32);
    a.nftiles = ceil_div(F, 64);
    if (!plan_tile(a)) return SEERA_OK;
    const int64_t wsz = (int64_t)a.nftiles * a.nchunks * R * S * 2048;
    if (wsz > 0x7fffffff) return SEERA_OK;  // prep kernel indexes in 32 bits
    void* ws = nullptr;
    SEERA_TRY(workspace(sizeof(half_t) * (size_t)wsz, &ws, st));
    a.wk = static_cast<const half_t*>(ws);
    hipLaunchKernelGGL(prep_fwd_weights, dim3((unsigned)((wsz + 255) / 256)), dim3(256), 0, st, Wt,
                       static_cast<half_t*>(ws), F, C, R, S, a.nchunks, (int)wsz);
    SEERA_HIP_TRY(hipGetLastError());
    bool streamed = false;
    SEERA_TRY(stream_conv(a, st, &streamed));
    if (!streamed) SEERA_TRY(launch_band(a, st));
    *used = true;
    return SEERA_OK;
}

int band_conv_dgrad(const float* Yin, const float* Wconv, float* out, int B, int Fc, int Hi, int Wi,
                    int Cc, int H, int W, int R, int S, int sh, int sw, int ph, int pw,
                    hipStream_t st, bool* used) {
    *used = false;
    if (Wi % 4 != 0 || !aligned16(Yin) || sh * sw > kBandMaxPhases) return SEERA_OK;
    BandConvArgs a{};
    a.in = Yin;
    a.out = out;
    a.B = B; a.C = Fc; a.H = Hi; a.W = Wi;
    a.F = Cc; a.Hout = H; a.Wout = W;
    a.ish = 1; a.isw = 1; a.osh = sh; a.osw = sw;
    a.nchunks = ceil_div(Fc, 32);
    a.nftiles = ceil_div(Cc, 64);
    struct Axis { int r0, T, q, n; };
    auto axis = [](int phi, int p, int s, int K, int out_len) {
        Axis x;
        x.r0 = (phi + p) % s;
        x.T = K > x.r0 ? (K - x.r0 + s - 1) / s : 0;
        x.q = (phi + p - x.r0) / s;
        x.n = out_len > phi ? (out_len - phi + s - 1) / s : 0;
        return x;
    };
    int64_t woff = 0;
    int zi = 0;
    Axis ax[kBandMaxPhases][2];
    for (int phh = 0; phh < sh; ++phh)
        for (int phw = 0; phw < sw; ++phw, ++zi) {
            const Axis xh = axis(phh, ph, sh, R, H), xw = axis(phw, pw, sw, S, W);
            ax[zi][0] = xh;
            ax[zi][1] = xw;
            BandPhase& p = a.ph[zi];
            p.Ho = xh.n; p.Wo = xw.n;
            p.T = xh.T; p.U = xw.T;
            p.iph = xh.T - 1 - xh.q;
            p.ipw = xw.T - 1 - xw.q;
            p.oph = phh; p.opw = phw;
            p.woff = woff;
            woff += (int64_t)a.nftiles * a.nchunks * xh.T * xw.T * 2048;
        }
    a.nphase = zi;
    if (sh == 2 && sw == 2) {
        // All four stride phases in one block (conv_phase2.hip) when it applies.
        const int T2[2] = {ax[0][0].T, ax[2][0].T}, iph2[2] = {a.ph[0].iph, a.ph[2].iph};
        const int r0h2[2] = {ax[0][0].r0, ax[2][0].r0};
        const int U2[2] = {ax[0][1].T, ax[1][1].T}, ipw2[2] = {a.ph[0].ipw, a.ph[1].ipw};
        const int r0w2[2] = {ax[0][1].r0, ax[1][1].r0};
        bool done = false;
        SEERA_TRY(phase2_conv(Yin, Wconv, out, B, Fc, Hi, Wi, Cc, H, W, R, S, T2, iph2, r0h2, U2,
                              ipw2, r0w2, st, &done));
        if (done) {
            *used = true;
            return SEERA_OK;
        }
    }
    if (!plan_tile(a)) return SEERA_OK;
    if (woff > 0x7fffffff) return SEERA_OK;  // prep kernel indexes in 32 bits
    void* ws = nullptr;
    SEERA_TRY(workspace(sizeof(half_t) * (size_t)std::max<int64_t>(woff, 1), &ws, st));
    a.wk = static_cast<const half_t*>(ws);
    if (woff > 0) {
        // One launch for every phase's weights (they sit back to back in ws).
        DgradPrepPhases pp{};
        pp.nphase = a.nphase;
        for (int z = 0; z < a.nphase; ++z) {
            pp.begin[z] = a.ph[z].woff;
            pp.T[z] = a.ph[z].T;
            pp.U[z] = a.ph[z].U;
            pp.r0h[z] = ax[z][0].r0;
            pp.r0w[z] = ax[z][1].r0;
        }
        pp.begin[a.nphase] = woff;
        hipLaunchKernelGGL(prep_dgrad_weights, dim3((unsigned)((woff + 255) / 256)), dim3(256), 0,
                           st, Wconv, static_cast<half_t*>(ws), Fc, Cc, R, S, sh, sw, a.nchunks, pp);
        SEERA_HIP_TRY(hipGetLastError());
    }
    bool streamed = false;
    SEERA_TRY(stream_conv(a, st, &streamed));
    if (!streamed) SEERA_TRY(launch_band(a, st));
    *used = true;
    return SEERA_OK;
}


int band_conv_wgrad(const float* Y, const float* X, float* dW, float* db, int B, int C, int H,
                    int W, int F, int R, int S, int sh, int sw, int ph, int pw, hipStream_t st,
                    bool* used, bool* db_done, int wo_override) {
    *used = false;
    *db_done = false;
    const int Wo_nat = (W + 2 * pw - S) / sw + 1;
    const int Ho = (H + 2 * ph - R) / sh + 1, Wo = wo_override > 0 ? wo_override : Wo_nat;
    if (Wo > Wo_nat) return SEERA_OK;  // an output column would read past X's pitch
    if (sh == 1 && sw == 1 && Wo == Wo_nat) {
        WgradPartials wp{};
        bool streamed = false;
        SEERA_TRY(stream_wgrad_partials(Y, X, B, C, H, W, F, R, S, ph, pw, db != nullptr, st, &wp,
                                        &streamed));
        if (streamed) {
            SEERA_HIP_TRY(launch_wgrad_reduce(wp.part, dW, F, C, R, S, wp.CT, wp.nctile, wp.ntiles,
                                              wp.nsplit, st, wp.dbpart, db));
            *used = true;
            *db_done = wp.dbpart != nullptr;
            return SEERA_OK;
        }
    }
    if (R == 4 && S == 4 && sh == 2 && sw == 2 && ph == 1 && pw == 1) {
        WgradPartials wp{};
        bool streamed = false;
        SEERA_TRY(wgrad_s2_partials(Y, X, B, C, H, W, F, st, &wp, &streamed));
        if (streamed) {
            SEERA_HIP_TRY(launch_wgrad_reduce(wp.part, dW, F, C, R, S, wp.CT, wp.nctile, wp.ntiles,
                                              wp.nsplit, st, nullptr, nullptr));
            *used = true;
            return SEERA_OK;
        }
    }
    if (Wo % 4 != 0 || W % 4 != 0 || sw > 2 || S > 7 || R * S > 18 || !aligned16(Y) ||
        !aligned16(X) || B == 0)
        return SEERA_OK;
    // The producers' buffer resources span one image's X planes and 65 dY
    // planes (a 64-filter tile plus the row overrun of a partial tile).
    if ((int64_t)(C + 64) * H * W * 4 >= kMaxTileSpanBytes ||
        (int64_t)65 * Ho * Wo * 4 >= kMaxTileSpanBytes)
        return SEERA_OK;
    WgradArgs a{};
    a.dy = Y; a.x = X;
    a.B = B; a.C = C; a.H = H; a.W = W; a.F = F; a.Ho = Ho; a.Wo = Wo;
    a.R = R; a.S = S; a.sh = sh; a.sw = sw; a.ph = ph; a.pw = pw;
    // Channels per block tile: two 32-channel chunks when the consumer
    // accumulators (2 chunks x ceil(2*R*S/4) groups x 16 floats) fit.
    a.CT = (R * S <= 9 && C > 32) ? 64 : 32;
    const int nch = a.CT / 32;
    const int ngw = ceil_div(2 * R * S, 4);
    if (ngw > 8) return SEERA_OK;
    a.nftile = ceil_div(F, 64);
    a.nctile = ceil_div(C, a.CT);
    // Output tile TH x WC8 (TH * WC8 a multiple of 32): the largest one whose
    // producer loads fit the per-thread budgets and whose two LDS stages fit.
    const int oct = sw == 1 ? 4 : 2;  // octets per X item (XItem<sw>::OCT)
    const int wo_cap = std::min(Wo, 224);
    // Tile widths: the whole (capped) row, or 64 / 32 columns when S shifted
    // copies of a whole row do not fit (large S on wide rows).
    const int wc_opts[4] = {(wo_cap + 7) & ~7, (wo_cap + 31) & ~31, std::min(64, (wo_cap + 31) & ~31),
                            32};
    int best_px = 0;
    WgradArgs best = a;
    for (int wc : wc_opts) {
        const int noct = wc / 8, ngrp = ceil_div(noct, oct);
        const int th_mult = wc % 32 == 0 ? 1 : wc % 16 == 0 ? 2 : 4;
        for (int th = th_mult; th * wc <= kWgKsMax * 32; th += th_mult) {
            WgradArgs t = a;
            t.WC8 = wc;
            t.TH = th;
            t.BR = (th - 1) * sh + R;
            t.dy_stride = stride16(th * wc);
            t.xrow = ceil_div(wc, 8 * oct) * 8 * oct;
            t.x_plane = stride16(t.BR * t.xrow);
            t.lds_bytes = 2 * 2 * ((int64_t)64 * t.dy_stride + (int64_t)S * 32 * t.x_plane);
            const bool fits = t.lds_bytes <= kBandMaxLds && 64 * th * noct <= kWgDyMax * kWgProd &&
                              32 * t.BR * ngrp <= kWgProd;
            if (!fits) break;
            const int px = std::min(th, Ho) * std::min(wc, Wo);  // useful pixels
            if (px > best_px) {
                best_px = px;
                best = t;
            }
            if (th >= Ho) break;
        }
    }
    if (best_px == 0) return SEERA_OK;
    a = best;
    a.KS = a.TH * a.WC8 / 32;
    a.ncb = ceil_div(Wo, a.WC8);
    a.nrb = ceil_div(Ho, a.TH);
    a.items = B * a.nrb * a.ncb;
    const int tiles = a.nftile * a.nctile;
    int nsplit = std::max(1, std::min(a.items, ceil_div(256, tiles)));
    a.ips = ceil_div(a.items, nsplit);
    a.nsplit = ceil_div(a.items, a.ips);
    const int ntot = a.CT * R * S;
    void* ws = nullptr;
    SEERA_TRY(workspace(sizeof(float) * (size_t)tiles * a.nsplit * 64 * ntot, &ws, st));
    a.part = static_cast<float*>(ws);
    hipError_t e;
    if (sw == 1) e = nch == 2 ? launch_wgrad_sw<1, 2>(a, ngw, st) : launch_wgrad_sw<1, 1>(a, ngw, st);
    else e = nch == 2 ? launch_wgrad_sw<2, 2>(a, ngw, st) : launch_wgrad_sw<2, 1>(a, ngw, st);
    if (e != hipSuccess) return fail_hip(e, "band wgrad launch");
    SEERA_HIP_TRY(launch_wgrad_reduce(a.part, dW, F, C, R, S, a.CT, a.nctile, tiles, a.nsplit, st,
                                      nullptr, nullptr));
    *used = true;
    return SEERA_OK;
}

}  // namespace seera
