// conv_stream.hip -- row-streaming implicit-GEMM convolution for gfx950.
//
// Serves the same launches as the LDS-band kernel (conv_band.hip: conv2d
// forward, conv2d dX / convT forward by stride phases) when every phase reads
// its input with stride 1 and a whole 64-filter weight slice fits in LDS next
// to a ring of input rows:
//   out[b, f, oh*osh + oph, ow*osw + opw] =
//     sum_{c, t < T, u < U} Wk[f, t, u, c] * in[b, c, oh + t - iph, ow + u - ipw]
// (convolution.cu:15-101 forward, convolution.cu:144-265 dX, upsampling.cu:
// 15-126 transposed forward).
//
// A block owns one image, a strip of L output rows of one phase, up to 64
// output columns and 64 output channels, and runs warp-specialised, 4 rows per
// step:
//   * 8 consumer waves, two per output row (one per half of its pixels, so
//     the two waves of a SIMD cover each other's LDS and store stalls): in
//     step s, wave w computes half w/4 of output row 4s + w%4 of the strip
//     (64 filters, v_mfma_f32_16x16x32_f16 with 16 pixels x 32 channels of the
//     ring as A and the weights as B, so each lane ends with 4 consecutive
//     pixels of one filter) and stores it as float4s;
//   * 4 producer waves: while the consumers work on step s, they write the 4
//     input rows of step s+1 (loaded into registers during step s-1, rounded
//     to fp16, channel-last) into the ring and issue the loads of step s+2.
// The ring holds 2*4 + T - 1 rows, so one barrier per step suffices, and the
// consumers never wait on the input loads nor the producers on the output
// stores. The weights are loaded once per block, ahead of any input row, and
// stay resident; every input row is read from HBM once per strip (plus T-1
// halo rows), so HBM sees each input and output element about once.
#include "conv_band.h"
#include "mfma_core.h"

namespace seera {
namespace {

typedef float floatx4_t __attribute__((ext_vector_type(4)));
typedef uint32_t uintx4_t __attribute__((ext_vector_type(4)));

__device__ __forceinline__ floatx4_t mfma16x16x32(half8 a, half8 b, floatx4_t c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}

// Ring plane layout: pixel p holds 32 channels as four 16-byte chunks, the
// chunk order rotated by (p >> 1) & 3. Measured on gfx950: a ds_read_b128 is
// served per 32-lane half-wave at 2 lanes per 16-byte slot of a 256-byte bank
// window per cycle, which the B reads (16 consecutive pixels at each of 2
// chunks per half-wave, any start) meet; a ds_write_b128 is conflict-free only
// when the 8 lanes of each group hit 8 distinct 16-byte slots of a 128-byte
// window. The item writes (4 channel groups of two adjacent column quads per
// 8 lanes) meet that because odd quads write their four pixels with the pairs
// swapped: in quad order the two quads' pixels sit 256 bytes apart, on the
// same 4 slots.
__device__ __forceinline__ int ring_off(int p, int chunk) {
    return p * 32 + ((chunk ^ ((p >> 1) & 3)) << 3);
}

constexpr int kG = 4;              // output rows per step
constexpr int kCons = 2 * kG * 64; // consumer threads (two waves per row)
constexpr int kProd = 256;         // producer threads
constexpr int kNT = kCons + kProd;
constexpr int kItems = 2;          // input items per producer thread per step
constexpr int kPreW = 12;          // weight pieces (16 B) per thread, prologue
constexpr int kPreItems = 2;       // input items per thread, prologue
constexpr int kTailPad = 1024;     // LDS bytes past the ring (reads of padding lanes)

struct StreamArgs {
    const float* in;    // [B, C, H, W] fp32
    const half_t* wk;   // prepared fp16 weights (conv_band.hip layout)
    float* out;         // [B, F, Hout, Wout] fp32
    int B, C, H, W;
    int F, Hout, Wout;
    int osh, osw;
    int nchunks;        // 32-channel chunks of C
    int WC;             // output columns per block (<= 64)
    int BC4;            // ring pixels per plane (multiple of 4)
    int NR;             // ring rows
    int L;              // output rows per strip
    int wl_halves;      // LDS halves reserved for weights
    int nblocks;
    int64_t lds_bytes;
    int nphase;
    BandPhase ph[kBandMaxPhases];  // nrb = strips, ncb = column tiles
    ConvEpi epi;                   // fused bias / activation (zero: none)
};

// UC: every phase has 3 column taps (0: any).
// Epilogue kinds (template argument of the kernel): none, + bias, + bias
// then ReLU (the mask, when asked for, with the last).
constexpr int kEpiNone = 0, kEpiBias = 1, kEpiBiasRelu = 2;

template <int PXG, int UC, int EPI>
__global__ __launch_bounds__(kNT) void stream_conv_kernel(const StreamArgs a) {
    extern __shared__ __attribute__((aligned(16))) half_t smem[];
    const int bx = blockIdx.x;
    int z = 0;
    while (z + 1 < a.nphase && bx >= a.ph[z + 1].block0) ++z;
    const BandPhase& P = a.ph[z];
    int local = bx - P.block0;
    const int cb = local % P.ncb;
    local /= P.ncb;
    const int strip = local % P.nrb;
    const int b = local / P.nrb;
    const int ftile = blockIdx.y;
    const int ohA = strip * a.L;
    const int Lb = min(a.L, P.Ho - ohA);        // output rows of this strip
    // Rows the first step is short of (a block with sh > 0 runs out of phase
    // with one with sh = 0; all blocks currently start in phase).
    const int sh = 0;
    const int nsteps = (Lb + sh + kG - 1) / kG;
    const int ow0 = cb * a.WC;
    const int T = P.T, U = P.U, taps = T * U;
    const int icr = ow0 - P.ipw;                 // input column of ow0 at tap u = 0
    const int ic0 = icr >= 0 ? (icr & ~3) : -((-icr + 3) & ~3);
    const int coff = icr - ic0;                  // 0..3
    const int nq = a.BC4 >> 2;
    const int plane = a.BC4 * 32;                // halves per (ring row, chunk) plane
    // Strip input row i sits in ring slot i % NR; group g (the rows written
    // during step g-1) starts at row g0 + g*kG, after T-1 halo rows [-sh, g0).
    const int g0 = T - 1 - sh;

    half_t* const wl = smem;
    half_t* const ring = smem + a.wl_halves;
    const int tid = threadIdx.x, lane = tid & 63;
    // Wave index as a scalar: the role branch and everything derived from the
    // wave (output row, ring slots) stay wave-uniform in SGPRs.
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);

    // ---- prologue, by all waves: the weights and the first T-1+kG input
    // rows (halo and group 0) are requested at once, then written to LDS;
    // the producers then request group 1 and release step 0 ----
    {
        const half_t* wsrc = a.wk + P.woff + (int64_t)ftile * a.nchunks * taps * 2048;
        const int n16 = a.nchunks * taps * 256;  // <= kPreW * kNT (host check)
        half8 wv[kPreW];
#pragma unroll
        for (int k = 0; k < kPreW; ++k) {
            const int i = k * kNT + tid;
            if (i < n16) wv[k] = *reinterpret_cast<const half8*>(wsrc + (int64_t)i * 8);
        }
        // Items as the producers' (row, chunk, 8-channel group cg, column
        // quad q4), cg fastest, over strip input rows [-sh, g0 + kG).
        const rsrc_t src = make_rsrc_in(a.in, (int64_t)a.B * a.C * a.H * a.W, (int64_t)b * a.C * a.H * a.W);
        const uint32_t cstride = (uint32_t)(a.H * a.W * 4);
        const int row_items = a.nchunks * 4 * nq;
        const int nitems = (g0 + sh + kG) * row_items;  // <= kPreItems * kNT (host check)
        const int need = Lb + T - 1;
        floatx4 xv[kPreItems][8];
#pragma unroll
        for (int k = 0; k < kPreItems; ++k) {
            const int it = k * kNT + tid;
            const int cg = it & 3;
            int r = it >> 2;
            const int q4 = r % nq;
            r /= nq;
            const int ch = r % a.nchunks;
            const int i = r / a.nchunks - sh;        // strip input row
            const int hin = ohA - P.iph + i;
            const int c0 = ch * 32 + cg * 8, win = ic0 + q4 * 4;
            const bool ok = it < nitems && (unsigned)i < (unsigned)need &&
                            (unsigned)hin < (unsigned)a.H && c0 < a.C && (unsigned)win < (unsigned)a.W;
            const uint32_t vo = ok ? (uint32_t)((c0 * a.H * a.W + hin * a.W + win) * 4) : kBufOOB;
#pragma unroll
            for (int j = 0; j < 8; ++j) xv[k][j] = buf_load4s(src, vo, j * cstride);
        }
#pragma unroll
        for (int k = 0; k < kPreW; ++k) {
            const int i = k * kNT + tid;
            if (i < n16)
                *reinterpret_cast<half8*>(wl + (i >> 8) * 2048 + ring_off((i & 255) >> 2, i & 3)) = wv[k];
        }
#pragma unroll
        for (int k = 0; k < kPreItems; ++k) {
            const int it = k * kNT + tid;
            const int cg = it & 3;
            int r = it >> 2;
            const int q4 = r % nq;
            r /= nq;
            const int ch = r % a.nchunks;
            const int i = r / a.nchunks - sh;
            if (it < nitems && (unsigned)i < (unsigned)need) {
                half_t* dst = ring + (i % a.NR) * a.nchunks * plane + ch * plane + q4 * 128;
                const int sw = q4 & 1;  // odd quads write their pixel pairs swapped
#pragma unroll
                for (int jj = 0; jj < 4; ++jj) {
                    float col[8];
#pragma unroll
                    for (int j = 0; j < 8; ++j) col[j] = sw ? xv[k][j][jj ^ 1] : xv[k][j][jj];
                    *reinterpret_cast<half8*>(dst + ring_off(4 * q4 + (jj ^ sw), cg) - 4 * q4 * 32) =
                        pack8(col);
                }
            }
        }
    }

    if (wave < 2 * kG) {
        // ---- consumers: one half output row per step ----
        const int kc = lane >> 4;                // k chunk of this lane's fragments
        // Weight fragment offsets (tap 0, chunk 0). The 64 x 32 weight slice
        // of a tap uses the ring's pixel layout (filter f in place of pixel p),
        // which serves this 16-row x 2-chunk read pattern without bank
        // conflicts (the GEMM tile swizzle lds_off<32> would cost 2x here);
        // filter group fg sits 512*fg halves further.
        int wrow[4];
#pragma unroll
        for (int fg = 0; fg < 4; ++fg) wrow[fg] = ring_off(lane & 15, kc) + 512 * fg;
        const int nqt = a.nchunks * taps;
        // Output: buffer resource over this image's [F, Hout, Wout] block;
        // lanes outside the tile get kBufOOB and their stores are dropped.
        const rsrc_t dst_img = make_rsrc_in(a.out, (int64_t)a.B * a.F * a.Hout * a.Wout, (int64_t)b * a.F * a.Hout * a.Wout);
        const int hw = a.Hout * a.Wout;
        const int fl = ftile * 64 + (lane & 15);  // filter of this lane (+ fg*16)
        // Fused epilogue (the bias and ReLU of a Conv2D layer): bias of each of
        // this lane's 4 filters, and the mask image (written when ReLU asks
        // for it, at the output's offsets: mask = out > 0, which is v > 0).
        const bool mask_on = EPI == kEpiBiasRelu && a.epi.mask;
        float bv[4];
#pragma unroll
        for (int fg = 0; fg < 4; ++fg)
            bv[fg] = a.epi.bias && fl + fg * 16 < a.F ? a.epi.bias[fl + fg * 16] : 0.f;
        const rsrc_t mask_img =
            make_rsrc_in(mask_on ? a.epi.mask : a.out, (int64_t)a.B * a.F * a.Hout * a.Wout, (int64_t)b * a.F * a.Hout * a.Wout);
        auto finish = [&](floatx4_t v, int fg) {
            if constexpr (EPI != kEpiNone) {
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const float t = v[j] + bv[fg];
                    v[j] = EPI == kEpiBiasRelu ? (t > 0.f ? t : 0.f) : t;
                }
            }
            return v;
        };
        auto mask_of = [](floatx4_t v) {
            floatx4_t m;
#pragma unroll
            for (int j = 0; j < 4; ++j) m[j] = v[j] > 0.f ? 1.f : 0.f;
            return m;
        };
        const int px0 = (wave / kG) * PXG * 16;   // first pixel of this wave's half row
        // Pixel fragment offsets within a ring plane per column tap (UC == 3).
        int poff[UC == 3 ? 3 : 1][PXG];
        if constexpr (UC == 3) {
#pragma unroll
            for (int u = 0; u < 3; ++u)
#pragma unroll
                for (int pg = 0; pg < PXG; ++pg)
                    poff[u][pg] = ring_off(px0 + pg * 16 + (lane & 15) + u + coff, kc);
        }
        // UC == 3: a step's results wait in res (byte offsets roff, kBufOOB:
        // none) and are stored between the MFMA blocks of the next step, so
        // the output stores overlap the MFMAs instead of stalling the wave
        // at the end of every step while the memory pipe drains.
        floatx4_t res[UC == 3 ? PXG : 1][4];
        uint32_t roff[UC == 3 ? PXG : 1][4];
        bool pending = false;
#define SEERA_STREAM_FLUSH(PG, FG0)                                                         \
    _Pragma("unroll") for (int fg = (FG0); fg < (FG0) + 2; ++fg) {                          \
        __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(uintx4_t, res[PG][fg]),   \
                                               dst_img, roff[PG][fg], 0, 0);                \
        if (mask_on)                                                                        \
            __builtin_amdgcn_raw_buffer_store_b128(                                         \
                __builtin_bit_cast(uintx4_t, mask_of(res[PG][fg])), mask_img, roff[PG][fg], \
                0, 0);                                                                      \
    }
        for (int s = 0; s < nsteps; ++s) {
            __syncthreads();  // the rows of step s are in the ring
            const int o = s * kG + wave % kG - sh;  // output row of this wave (strip-relative)
            if (o < 0 || o >= Lb || px0 >= a.WC) {
                if constexpr (UC == 3) {
                    if (pending) {
#pragma unroll
                        for (int pg = 0; pg < PXG; ++pg) { SEERA_STREAM_FLUSH(pg, 0) SEERA_STREAM_FLUSH(pg, 2) }
                        pending = false;
                    }
                }
                continue;
            }
            // acc[pg][fg]: pixels of group pg (rows) x filters of group fg
            // (columns); lane holds pixels 4*(lane/16) + r at filter lane%16.
            floatx4_t acc[PXG][4];
#pragma unroll
            for (int pg = 0; pg < PXG; ++pg)
#pragma unroll
                for (int fg = 0; fg < 4; ++fg) acc[pg][fg] = floatx4_t{0.f, 0.f, 0.f, 0.f};
            const int slot0 = o % a.NR;
            // (ch, t, u) of the next fragment set to read
            int ch = 0, t = 0, u = 0;
            half8 fa[2][4], fb[2][PXG];
#define SEERA_STREAM_READ(BUF)                                                              \
    {                                                                                       \
        const half_t* w = wl + (ch * taps + t * U + u) * 2048;                              \
        int slot = slot0 + t;                                                               \
        if (slot >= a.NR) slot -= a.NR;                                                     \
        const half_t* rp = ring + (slot * a.nchunks + ch) * plane;                          \
        _Pragma("unroll") for (int fg = 0; fg < 4; ++fg) fa[BUF][fg] =                      \
            *reinterpret_cast<const half8*>(w + wrow[fg]);                                  \
        _Pragma("unroll") for (int pg = 0; pg < PXG; ++pg) fb[BUF][pg] =                    \
            *reinterpret_cast<const half8*>(rp + ring_off(px0 + pg * 16 + (lane & 15) + u + coff, kc)); \
        if (++u == U) {                                                                     \
            u = 0;                                                                          \
            if (++t == T) {                                                                 \
                t = 0;                                                                      \
                if (ch + 1 < a.nchunks) ++ch; /* past the end: re-reads, never used */      \
            }                                                                               \
        }                                                                                   \
    }
#define SEERA_STREAM_MMA(BUF)                                                               \
    _Pragma("unroll") for (int pg = 0; pg < PXG; ++pg)                                      \
        _Pragma("unroll") for (int fg = 0; fg < 4; ++fg)                                    \
            acc[pg][fg] = mfma16x16x32(fb[BUF][pg], fa[BUF][fg], acc[pg][fg]);
            if constexpr (UC == 3) {
                // Three column taps known at compile time: the sets of one
                // (chunk, row tap) pair use fragment buffers 0, 1, 2 and reads
                // run two sets ahead of the MFMAs (one set ahead leaves the
                // MFMAs waiting on LDS latency with 8 waves reading). Pixel
                // offsets per tap are per-lane constants, weight offsets are
                // immediates off one base per pair.
                const int nct = a.nchunks * T;
                int ct_t = 0, ct_ch = 0;  // (row tap, chunk) of the pair being read
#define SEERA_STREAM_READ3(T_, CH_, U_, BUF)                                                \
    {                                                                                       \
        const half_t* w = wl + ((CH_) * T + (T_)) * 6144 + (U_) * 2048;                     \
        int slot = slot0 + (T_);                                                            \
        if (slot >= a.NR) slot -= a.NR;                                                     \
        const half_t* rp = ring + (slot * a.nchunks + (CH_)) * plane;                       \
        _Pragma("unroll") for (int pg = 0; pg < PXG; ++pg) fb3[BUF][pg] =                   \
            *reinterpret_cast<const half8*>(rp + poff[U_][pg]);                             \
        _Pragma("unroll") for (int fg = 0; fg < 4; ++fg) fa3[BUF][fg] =                     \
            *reinterpret_cast<const half8*>(w + wrow[fg]);                                  \
    }
#define SEERA_STREAM_MMA3(BUF)                                                              \
    _Pragma("unroll") for (int pg = 0; pg < PXG; ++pg)                                      \
        _Pragma("unroll") for (int fg = 0; fg < 4; ++fg)                                    \
            acc[pg][fg] = mfma16x16x32(fb3[BUF][pg], fa3[BUF][fg], acc[pg][fg]);
                half8 fa3[3][4], fb3[3][PXG];
                SEERA_STREAM_READ3(0, 0, 0, 0)
                SEERA_STREAM_READ3(0, 0, 1, 1)
                for (int ct = 0; ct < nct; ++ct) {
                    SEERA_STREAM_READ3(ct_t, ct_ch, 2, 2)
                    // the next pair (the last one again past the end)
                    if (ct + 1 < nct) {
                        if (++ct_t == T) { ct_t = 0; ++ct_ch; }
                    }
                    SEERA_STREAM_MMA3(0)
                    // the previous step's results: pixel group ct (ct < PXG)
                    if (pending && ct < PXG) {
                        if (ct == 0) { SEERA_STREAM_FLUSH(0, 0) }
                        if (PXG > 1 && ct == 1) { SEERA_STREAM_FLUSH(PXG - 1, 0) }
                    }
                    SEERA_STREAM_READ3(ct_t, ct_ch, 0, 0)
                    SEERA_STREAM_MMA3(1)
                    if (pending && ct < PXG) {
                        if (ct == 0) { SEERA_STREAM_FLUSH(0, 2) }
                        if (PXG > 1 && ct == 1) { SEERA_STREAM_FLUSH(PXG - 1, 2) }
                    }
                    SEERA_STREAM_READ3(ct_t, ct_ch, 1, 1)
                    SEERA_STREAM_MMA3(2)
                }
                if (pending && PXG > 1 && nct < 2) {
                    SEERA_STREAM_FLUSH(PXG - 1, 0)
                    SEERA_STREAM_FLUSH(PXG - 1, 2)
                }
#undef SEERA_STREAM_READ3
#undef SEERA_STREAM_MMA3
            } else {
                // Reads run one fragment set ahead of the MFMAs and are issued
                // unconditionally, so every MFMA waits only for its own set.
                SEERA_STREAM_READ(0)
                for (int q = 0; q < nqt; q += 2) {
                    SEERA_STREAM_READ(1)
                    SEERA_STREAM_MMA(0)
                    SEERA_STREAM_READ(0)
                    if (q + 1 < nqt) { SEERA_STREAM_MMA(1) }
                }
            }
#undef SEERA_STREAM_READ
#undef SEERA_STREAM_MMA
            // 4 consecutive output pixels per lane (the host guarantees output
            // rows contiguous and 16-byte aligned).
            const int orow = (ohA + o) * a.Wout;
#pragma unroll
            for (int pg = 0; pg < PXG; ++pg) {
                const int px = px0 + pg * 16 + 4 * kc;  // first of this lane's 4 pixels
                const bool pok = px < a.WC && ow0 + px < P.Wo;
#pragma unroll
                for (int fg = 0; fg < 4; ++fg) {
                    const int f = fl + fg * 16;
                    const uint32_t off =
                        pok && f < a.F ? (uint32_t)((f * hw + orow + ow0 + px) * 4) : kBufOOB;
                    if constexpr (UC == 3) {
                        res[pg][fg] = finish(acc[pg][fg], fg);
                        roff[pg][fg] = off;
                    } else {
                        const floatx4_t v = finish(acc[pg][fg], fg);
                        __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(uintx4_t, v),
                                                               dst_img, off, 0, 0);
                        if (mask_on)
                            __builtin_amdgcn_raw_buffer_store_b128(
                                __builtin_bit_cast(uintx4_t, mask_of(v)), mask_img, off, 0, 0);
                    }
                }
            }
            pending = UC == 3;
        }
        if constexpr (UC == 3) {
            if (pending) {
#pragma unroll
                for (int pg = 0; pg < PXG; ++pg) { SEERA_STREAM_FLUSH(pg, 0) SEERA_STREAM_FLUSH(pg, 2) }
            }
        }
#undef SEERA_STREAM_FLUSH
        return;
    }

    // ---- producers: input rows into the ring, one step ahead ----
    // Item k of this thread (it = ptid + k*kProd) is (row of the group,
    // 32-channel chunk, 8-channel group cg, column quad q4), cg fastest; the
    // same items recur every step, only the group's first row changes. Buffer
    // resource over this image: out-of-image rows and columns and rows outside
    // the strip read as 0 (the host checks that one image spans less than
    // kMaxTileSpanBytes and that C is a multiple of 8, so an item's 8 channels
    // are all in range or all out).
    const int ptid = tid - kCons;
    const rsrc_t src = make_rsrc_in(a.in, (int64_t)a.B * a.C * a.H * a.W, (int64_t)b * a.C * a.H * a.W);
    const uint32_t cstride = (uint32_t)(a.H * a.W * 4);
    const int row_items = a.nchunks * 4 * nq;    // items per input row
    const int need = Lb + T - 1;                 // strip-relative input rows used
    const int hin0 = ohA - P.iph;                // image row of strip input row 0
    int prow[kItems];                            // row within the group (kG: none)
    uint32_t pcol[kItems];                       // byte offset of (c0, row 0, win); kBufOOB: none
    int pdst[kItems];                            // ring offset (halves) of (chunk, pixel 4*q4)
    int pcg[kItems];                             // 8-channel group
    int prq[kItems];                             // (2*q4) & 3: chunk rotation of pixels 4*q4, 4*q4+1
#pragma unroll
    for (int k = 0; k < kItems; ++k) {
        const int it = ptid + k * kProd;
        const int cg = it & 3;
        int r = it >> 2;
        const int q4 = r % nq;
        r /= nq;
        const int ch = r % a.nchunks;
        prow[k] = it < kG * row_items ? r / a.nchunks : kG;
        const int c0 = ch * 32 + cg * 8, win = ic0 + q4 * 4;
        pcol[k] = c0 < a.C && (unsigned)win < (unsigned)a.W ? (uint32_t)((c0 * a.H * a.W + win) * 4)
                                                             : kBufOOB;
        pdst[k] = ch * plane + q4 * 128;
        pcg[k] = cg;
        prq[k] = (2 * q4) & 3;
    }
    floatx4 v[kItems][8];  // one step's items: 8 channels x 4 columns each

    // Issue the loads of the rows [I0, I0 + NROWS) that this thread's items cover.
#define SEERA_STREAM_LOAD(V, I0, NROWS)                                                     \
    {                                                                                       \
        _Pragma("unroll") for (int k = 0; k < kItems; ++k) {                                \
            const int i = (I0) + prow[k];                                                   \
            const int hin = hin0 + i;                                                       \
            const bool ok = prow[k] < (NROWS) && (unsigned)i < (unsigned)need &&            \
                            (unsigned)hin < (unsigned)a.H && pcol[k] != kBufOOB;            \
            const uint32_t vo = ok ? pcol[k] + (uint32_t)(hin * a.W * 4) : kBufOOB;         \
            _Pragma("unroll") for (int j = 0; j < 8; ++j)                                   \
                V[k][j] = buf_load4s(src, vo, j * cstride);                                 \
        }                                                                                   \
    }
    // Round the loaded items to fp16 and write them into their ring slots.
#define SEERA_STREAM_STORE(V, I0, NROWS)                                                    \
    {                                                                                       \
        _Pragma("unroll") for (int k = 0; k < kItems; ++k) {                                \
            const int i = (I0) + prow[k];                                                   \
            if (prow[k] < (NROWS) && (unsigned)i < (unsigned)need) {                        \
                half_t* dst = ring + (i % a.NR) * a.nchunks * plane + pdst[k];              \
                const int sw = prq[k] >> 1; /* odd quads: pixel pairs swapped */            \
                _Pragma("unroll") for (int jj = 0; jj < 4; ++jj) {                          \
                    float col[8];                                                           \
                    _Pragma("unroll") for (int j = 0; j < 8; ++j)                           \
                        col[j] = sw ? V[k][j][jj ^ 1] : V[k][j][jj];                        \
                    /* = ring_off(4*q4 + q, cg) relative to pixel 4*q4 */                   \
                    const int q = jj ^ sw;                                                  \
                    *reinterpret_cast<half8*>(dst + q * 32 +                                \
                                              ((pcg[k] ^ ((prq[k] + (q >> 1)) & 3)) << 3)) = \
                        pack8(col);                                                         \
                }                                                                           \
            }                                                                               \
        }                                                                                   \
    }
    __syncthreads();  // releases step 0 (the prologue wrote its rows)
    // Group 1 is requested after the release: issued before it, these loads
    // wait behind every block's prologue traffic and hold step 0 back.
    SEERA_STREAM_LOAD(v, g0 + kG, kG)
    for (int s = 0; s + 1 < nsteps; ++s) {
        // Ring slots of group s+1 held the rows only step s-1 read.
        SEERA_STREAM_STORE(v, g0 + (s + 1) * kG, kG)
        SEERA_STREAM_LOAD(v, g0 + (s + 2) * kG, kG)
        __syncthreads();  // releases step s+1
    }
#undef SEERA_STREAM_LOAD
#undef SEERA_STREAM_STORE
}

template <int PXG, int UC, int EPI>
hipError_t launch_epi(const StreamArgs& a, int nftiles, hipStream_t st) {
    auto kern = stream_conv_kernel<PXG, UC, EPI>;
    hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(kern),
                                       hipFuncAttributeMaxDynamicSharedMemorySize,
                                       (int)a.lds_bytes);
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL(kern, dim3(a.nblocks, nftiles), dim3(kNT), (size_t)a.lds_bytes, st, a);
    return hipGetLastError();
}

// The epilogue as a compile-time choice: its arithmetic then sits between the
// last MFMAs of a step and the barrier with no selects or branches.
template <int PXG, int UC>
hipError_t launch_pxg(const StreamArgs& a, int nftiles, hipStream_t st) {
    if (a.epi.act == kActRelu) return launch_epi<PXG, UC, kEpiBiasRelu>(a, nftiles, st);
    if (a.epi.bias) return launch_epi<PXG, UC, kEpiBias>(a, nftiles, st);
    return launch_epi<PXG, UC, kEpiNone>(a, nftiles, st);
}

}  // namespace

int stream_conv(const BandConvArgs& band, hipStream_t st, bool* used) {
    *used = false;
    SEERA_TRY(split_conv(band, st, used));
    if (*used) return SEERA_OK;
    if (band.ish != 1 || band.isw != 1 || band.nphase < 1) return SEERA_OK;
    StreamArgs a{};
    a.in = band.in; a.wk = band.wk; a.out = band.out; a.epi = band.epi;
    a.B = band.B; a.C = band.C; a.H = band.H; a.W = band.W;
    a.F = band.F; a.Hout = band.Hout; a.Wout = band.Wout;
    a.osh = band.osh; a.osw = band.osw;
    a.nchunks = band.nchunks;
    a.nphase = band.nphase;
    int max_t = 1, max_u = 1, max_taps = 1, max_wo = 0, max_ho = 0;
    for (int z = 0; z < a.nphase; ++z) {
        a.ph[z] = band.ph[z];
        max_t = std::max(max_t, a.ph[z].T);
        max_u = std::max(max_u, a.ph[z].U);
        max_taps = std::max(max_taps, a.ph[z].T * a.ph[z].U);
        max_wo = std::max(max_wo, a.ph[z].Wo);
        max_ho = std::max(max_ho, a.ph[z].Ho);
    }
    if (max_ho == 0 || max_wo == 0 || max_t - 1 > kG) return SEERA_OK;
    const int ncb = (max_wo + 63) / 64;
    a.WC = (((max_wo + ncb - 1) / ncb) + 3) & ~3;
    a.BC4 = (a.WC + max_u - 1 + 3 + 3) & ~3;
    a.NR = 2 * kG + max_t - 1;
    a.wl_halves = a.nchunks * max_taps * 2048;
    a.lds_bytes = (int64_t)a.wl_halves * 2 + (int64_t)a.NR * a.nchunks * a.BC4 * 64 + kTailPad;
    if (a.lds_bytes > kBandMaxLds) return SEERA_OK;
    if ((int64_t)a.C * a.H * a.W * 4 > kMaxTileSpanBytes || a.C % 8 != 0 ||
        (int64_t)a.F * a.Hout * a.Wout * 4 > kMaxTileSpanBytes)
        return SEERA_OK;
    // Output rows must be contiguous and 16-byte aligned (float4 stores).
    if (a.osw != 1 || a.osh != 1 || a.Wout % 4 != 0 || (reinterpret_cast<uintptr_t>(a.out) & 15) != 0)
        return SEERA_OK;
    for (int z = 0; z < a.nphase; ++z)
        if (a.ph[z].opw != 0 || a.ph[z].oph != 0) return SEERA_OK;
    if (kG * a.nchunks * a.BC4 > kProd * kItems) return SEERA_OK;  // items per step
    // prologue: weight pieces and the first T-1+kG rows' items per thread
    if (a.nchunks * max_taps * 256 > kPreW * kNT ||
        (max_t - 1 + kG) * a.nchunks * a.BC4 > kPreItems * kNT)
        return SEERA_OK;
    // Strip length: fewest rounds of one block per CU, each costing about
    // (steps + 1.5) step times (the prologue fetches the first rows unhidden).
    const int ncu = device_cus();
    const int nftiles = band.nftiles;
    int best_l = 0;
    double best_cost = 1e30;
    for (int L = kG; L < max_ho + kG; L += kG) {
        int64_t blocks = 0;
        for (int z = 0; z < a.nphase; ++z)
            blocks += (int64_t)a.B * ((a.ph[z].Ho + L - 1) / L) * ((a.ph[z].Wo + a.WC - 1) / a.WC);
        blocks *= nftiles;
        const double cost = (double)((blocks + ncu - 1) / ncu) * ((L + kG - 1) / kG + 1.5);
        if (cost < best_cost) { best_cost = cost; best_l = L; }
    }
    a.L = best_l;
    int blocks = 0;
    for (int z = 0; z < a.nphase; ++z) {
        BandPhase& p = a.ph[z];
        p.nrb = (p.Ho + a.L - 1) / a.L;
        p.ncb = (p.Wo + a.WC - 1) / a.WC;
        p.block0 = blocks;
        blocks += a.B * p.nrb * p.ncb;
    }
    a.nblocks = blocks;
    if (a.nblocks == 0 || nftiles == 0) { *used = true; return SEERA_OK; }
    const int pxg = ((a.WC + 15) / 16 + 1) / 2;  // pixel groups per consumer wave
    hipError_t e;
    bool u3 = true;
    for (int z = 0; z < a.nphase; ++z) u3 = u3 && a.ph[z].U == 3;
    if (u3)
        e = pxg == 1 ? launch_pxg<1, 3>(a, nftiles, st) : launch_pxg<2, 3>(a, nftiles, st);
    else
        e = pxg == 1 ? launch_pxg<1, 0>(a, nftiles, st) : launch_pxg<2, 0>(a, nftiles, st);
    if (e != hipSuccess) return fail_hip(e, "stream conv launch");
    *used = true;
    return SEERA_OK;
}

}  // namespace seera
