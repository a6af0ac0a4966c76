// conv_stride2.hip -- 4x4 convolution at stride 2, padding 1, by row
// streaming: the dX pass of a 4x4 stride-2 transposed convolution
// (upsampling.cu:128-197, 337-346) and the forward of a 4x4 stride-2
// convolution (convolution.cu:15-101, 367-389):
//   out[b, f, oh, ow] = sum_{c, r < 4, s < 4} W[f, c, r, s] * in[b, c, 2*oh - 1 + r, 2*ow - 1 + s]
// (zero outside the input).
//
// The ring holds each input row split by column parity: plane E has the even
// columns (pixel m = column 2m), plane O the odd ones (pixel m = column
// 2m + 1), fp16, channel-last. Output column ow then reads O pixels ow - 1
// and ow (taps s = 0, 2) and E pixels ow and ow + 1 (taps s = 1, 3): four
// unit-stride frames instead of a stride-2 gather.
//
// A block owns one image, a strip of L output rows, up to 32 output columns
// and 64 filters:
//   * 4 consumer waves, one per 16-filter group. A wave keeps its weight
//     fragments (C/32 chunks x 16 taps, fp16) in registers for the whole strip;
//     a step computes 2 output rows x 32 columns x 16 filters with
//     v_mfma_f32_16x16x32_f16 (16 pixels x 32 channels of the ring as A, the
//     register weights as B); every input row of the step (6: 2*2 new + 2
//     shared with the previous step) is read once per (chunk, frame) and
//     serves the one or two output rows whose taps reach it.
//   * 4 producer waves write the 4 input rows of the next step into the ring
//     and issue the loads of the step after it.
// HBM sees each input element once per 64-filter tile (plus 2 halo rows per
// strip) and each output element once.
#include "conv_band.h"
#include "mfma_core.h"

namespace seera {
namespace {

typedef float floatx4_t __attribute__((ext_vector_type(4)));
typedef uint32_t uintx4_t __attribute__((ext_vector_type(4)));

__device__ __forceinline__ floatx4_t mfma16x16x32(half8 a, half8 b, floatx4_t c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}

// Ring plane layout (as conv_stream.hip): pixel p holds 32 channels as four
// 16-byte chunks, the chunk order rotated by (p >> 1) & 3. On odd column
// quads the producers write the two pixels of a plane in swapped order, so the
// 8 lanes of a ds_write_b128 group (4 channel groups of two adjacent quads)
// hit 8 distinct 16-byte slots of a 128-byte window.
__device__ __forceinline__ int ring_off(int p, int chunk) {
    return p * 32 + ((chunk ^ ((p >> 1) & 3)) << 3);
}

constexpr int kRows = 2;          // output rows per step
constexpr int kIn = 2 * kRows;    // new input rows per step
constexpr int kCons = 4 * 64;     // consumer threads
constexpr int kProd = 256;        // producer threads
constexpr int kNT = kCons + kProd;
constexpr int kItems = 3;         // input items per producer thread per step
constexpr int kPreItems = 4;      // input items per producer thread, prologue
constexpr int kWC = 32;           // output columns per block
constexpr int kBC = 36;           // ring pixels per parity plane (kWC + 4, whole quads)
constexpr int kNR = 2 * kIn + 2;  // ring rows
constexpr int kTailPad = 1024;

struct Stride2Args {
    const float* in;     // [B, C, H, W] fp32
    const half_t* wk;    // fragment-order fp16 weights (prep_stride2_weights)
    float* out;          // [B, F, Ho, Wo] fp32
    int B, C, H, W, F, Ho, Wo;
    int L;               // output rows per strip
    int nstrips, ncb;    // strips and column tiles per image
    int64_t lds_bytes;
};

// Weight fragments in the order the consumer waves load them: for filter
// tile ft (64 filters) and filter group g (16): [chunk][r][s] blocks of 64
// lanes x 8 halves, lane l holding W[ft*64 + g*16 + l%16, chunk*32 + 8*(l/16)
// + j, r, s] (0 past F and C).
__global__ void prep_stride2_weights(const float* __restrict__ W, half_t* __restrict__ wk, int F,
                                     int C, int nchunks, int total_lanes) {
    const int gi = blockIdx.x * blockDim.x + threadIdx.x;  // (fragment, lane)
    if (gi >= total_lanes) return;
    const int lane = gi & 63;
    int fr = gi >> 6;
    const int tap = fr & 15;
    fr >>= 4;
    const int ch = fr % nchunks;
    const int grp = fr / nchunks;  // ft*4 + g
    const int f = grp * 16 + (lane & 15);
    const int k0 = ch * 32 + 8 * (lane >> 4);
    float v[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        const int k = k0 + j;
        v[j] = f < F && k < C ? W[((int64_t)f * C + k) * 16 + tap] : 0.f;
    }
    *reinterpret_cast<half8*>(wk + (int64_t)gi * 8) = pack8(v);
}

template <int NCH>
__global__ __launch_bounds__(kNT) void stride2_conv_kernel(const Stride2Args a) {
    extern __shared__ __attribute__((aligned(16))) half_t ring[];
    int local = blockIdx.x;
    const int cb = local % a.ncb;
    local /= a.ncb;
    const int strip = local % a.nstrips;
    const int b = local / a.nstrips;
    const int ftile = blockIdx.y;
    const int oh0 = strip * a.L;                  // first output row of the strip
    const int Lb = min(a.L, a.Ho - oh0);          // output rows of this strip
    const int nsteps = (Lb + kRows - 1) / kRows;
    const int ow0 = cb * kWC;
    // Ring pixel p of a parity plane is input column 2*(ow0 - 2 + p) (E) or
    // 2*(ow0 - 2 + p) + 1 (O); quad q4 of the producers covers input columns
    // c0 + 4*q4 .. +3 with c0 = 2*ow0 - 4 (E pixels 2*q4, 2*q4+1 and O pixels
    // 2*q4, 2*q4+1).
    const int c0 = 2 * ow0 - 4;
    constexpr int plane = kBC * 32;               // halves per (row, parity, chunk) plane
    constexpr int rowh = 2 * NCH * plane;         // halves per ring row
    // Strip input row i is image row 2*oh0 - 1 + i and sits in ring slot
    // i % kNR; step s reads rows 4s .. 4s+5; group g >= 1 (written during
    // step g-1) is rows 4g+2 .. 4g+5, the prologue writes rows 0..5.
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const rsrc_t src = make_rsrc_in(a.in, (int64_t)a.B * a.C * a.H * a.W, (int64_t)b * a.C * a.H * a.W);
    const uint32_t cstride = (uint32_t)(a.H * a.W * 4);
    constexpr int nq = kBC / 2;                   // column quads per input row
    constexpr int row_items = NCH * 4 * nq;       // items per input row
    const int need = 2 * Lb + 2;                  // strip input rows used
    const int hin0 = 2 * oh0 - 1;                 // image row of strip input row 0

    if (wave < 4) {
        // ---------------- consumers ----------------
        half8 wv[NCH][4][4];  // [chunk][r][s]
        {
            const half8* wsrc = reinterpret_cast<const half8*>(a.wk) +
                                (int64_t)(ftile * 4 + wave) * (16 * NCH) * 64 + lane;
#pragma unroll
            for (int ch = 0; ch < NCH; ++ch)
#pragma unroll
                for (int t = 0; t < 16; ++t) wv[ch][t >> 2][t & 3] = wsrc[(ch * 16 + t) * 64];
        }
        const int kc = lane >> 4;
        const int f = ftile * 64 + wave * 16 + (lane & 15);
        const rsrc_t dst_img = make_rsrc_in(a.out, (int64_t)a.B * a.F * a.Ho * a.Wo, (int64_t)b * a.F * a.Ho * a.Wo);
        const int hw = a.Ho * a.Wo;
        // Frames: tap s = 0: O pixel x+1, s = 1: E x+2, s = 2: O x+2, s = 3: E x+3
        // (x = output column - ow0); [s][pixel group] offsets within a row.
        int foff[4][2];
#pragma unroll
        for (int s = 0; s < 4; ++s)
#pragma unroll
            for (int pg = 0; pg < 2; ++pg) {
                const int par = (s & 1) ? 0 : 1;  // 0: E plane, 1: O plane
                const int p = pg * 16 + (lane & 15) + 1 + ((s + 1) >> 1);
                foff[s][pg] = par * NCH * plane + ring_off(p, kc);
            }

        for (int s = 0; s < nsteps; ++s) {
            __syncthreads();  // the rows of step s are in the ring
            floatx4_t acc[kRows][2];
#pragma unroll
            for (int r = 0; r < kRows; ++r)
#pragma unroll
                for (int pg = 0; pg < 2; ++pg) acc[r][pg] = floatx4_t{0.f, 0.f, 0.f, 0.f};
            // Input row j of the step (strip row 4s + j) is tap row r = j of
            // output row 2s and r = j - 2 of output row 2s + 1.
            half8 fb[2][4][2];
#define SEERA_S2_READ(Q, BUF)                                                                \
    {                                                                                        \
        const half_t* rp = ring + ((4 * s + (Q) % 6) % kNR) * rowh + ((Q) / 6) * plane;      \
        _Pragma("unroll") for (int t = 0; t < 4; ++t)                                        \
            _Pragma("unroll") for (int pg = 0; pg < 2; ++pg)                                 \
                fb[BUF][t][pg] = *reinterpret_cast<const half8*>(rp + foff[t][pg]);          \
    }
            SEERA_S2_READ(0, 0)
#pragma unroll
            for (int q = 0; q < NCH * 6; ++q) {
                if (q + 1 < NCH * 6) SEERA_S2_READ(q + 1, (q + 1) & 1)
                const int ch = q / 6, j = q % 6;
#pragma unroll
                for (int t = 0; t < 4; ++t)
#pragma unroll
                    for (int r = 0; r < kRows; ++r) {
                        const int kr = j - 2 * r;
                        if (kr < 0 || kr > 3) continue;
#pragma unroll
                        for (int pg = 0; pg < 2; ++pg)
                            acc[r][pg] = mfma16x16x32(fb[q & 1][t][pg], wv[ch][kr][t], acc[r][pg]);
                    }
            }
#undef SEERA_S2_READ
            // Lane: output columns x..x+3 (x = ow0 + pg*16 + 4*kc) of filter f.
#pragma unroll
            for (int r = 0; r < kRows; ++r) {
                const int o = s * kRows + r;
                const int orow = (oh0 + o) * a.Wo;
#pragma unroll
                for (int pg = 0; pg < 2; ++pg) {
                    const int x = ow0 + pg * 16 + 4 * kc;
                    const bool ok = o < Lb && x < a.Wo && f < a.F;
                    const uint32_t off = ok ? (uint32_t)((f * hw + orow + x) * 4) : kBufOOB;
                    __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(uintx4_t, acc[r][pg]),
                                                           dst_img, off, 0, 0);
                }
            }
        }
        return;
    }

    // ---------------- producers ----------------
    // Item (row of the group, chunk, 8-channel group cg, column quad q4), cg
    // fastest: 8 channels x 4 columns, written as 2 E and 2 O pixels.
    const int ptid = tid - kCons;
#define SEERA_S2_ITEM_WRITE(V, I, CH, CG, Q4)                                                \
    {                                                                                        \
        half_t* dst = ring + ((I) % kNR) * rowh + (CH) * plane;                              \
        const int sw = ((Q4) & 1) << 1;  /* odd quads: the two pixels of a plane swapped */  \
        _Pragma("unroll") for (int jj = 0; jj < 4; ++jj) {                                   \
            float col[8];                                                                    \
            _Pragma("unroll") for (int j = 0; j < 8; ++j) col[j] = sw ? V[j][jj ^ 2] : V[j][jj]; \
            /* column c0 + 4*q4 + q: parity q & 1, pixel 2*q4 + q/2 */                       \
            const int q = jj ^ sw;                                                           \
            *reinterpret_cast<half8*>(dst + (q & 1) * NCH * plane +                          \
                                      ring_off(2 * (Q4) + (q >> 1), (CG))) = pack8(col);     \
        }                                                                                    \
    }
    {
        // Prologue: strip rows 0..5.
        const int nitems = (kIn + 2) * row_items;  // <= kPreItems * kProd (host check)
        floatx4 xv[kPreItems][8];
#pragma unroll
        for (int k = 0; k < kPreItems; ++k) {
            const int it = k * kProd + ptid;
            const int cg = it & 3;
            int r = it >> 2;
            const int q4 = r % nq;
            r /= nq;
            const int ch = r % NCH;
            const int i = r / NCH;
            const int hin = hin0 + i;
            const int cc = ch * 32 + cg * 8, win = c0 + q4 * 4;
            const bool ok = it < nitems && i < need && (unsigned)hin < (unsigned)a.H &&
                            cc < a.C && (unsigned)win < (unsigned)a.W;
            const uint32_t vo = ok ? (uint32_t)((cc * a.H * a.W + hin * a.W + win) * 4) : kBufOOB;
#pragma unroll
            for (int j = 0; j < 8; ++j) xv[k][j] = buf_load4s(src, vo, j * cstride);
        }
#pragma unroll
        for (int k = 0; k < kPreItems; ++k) {
            const int it = k * kProd + ptid;
            const int cg = it & 3;
            int r = it >> 2;
            const int q4 = r % nq;
            r /= nq;
            const int ch = r % NCH;
            const int i = r / NCH;
            if (it < nitems && i < need) SEERA_S2_ITEM_WRITE(xv[k], i, ch, cg, q4)
        }
    }
    int prow[kItems], pch[kItems], pcg[kItems], pq4[kItems];
    uint32_t pcol[kItems];
#pragma unroll
    for (int k = 0; k < kItems; ++k) {
        const int it = ptid + k * kProd;
        const int cg = it & 3;
        int r = it >> 2;
        const int q4 = r % nq;
        r /= nq;
        const int ch = r % NCH;
        prow[k] = it < kIn * row_items ? r / NCH : kIn;
        const int cc = ch * 32 + cg * 8, win = c0 + q4 * 4;
        pcol[k] = cc < a.C && (unsigned)win < (unsigned)a.W ? (uint32_t)((cc * a.H * a.W + win) * 4)
                                                             : kBufOOB;
        pch[k] = ch;
        pcg[k] = cg;
        pq4[k] = q4;
    }
    // The rows of group g are requested during step g-2 and written during
    // step g-1 (before the barrier that releases step g).
    floatx4 v[kItems][8];
#define SEERA_S2_LOAD(G)                                                                     \
    {                                                                                        \
        _Pragma("unroll") for (int k = 0; k < kItems; ++k) {                                 \
            const int i = 2 + (G) * kIn + prow[k];                                           \
            const int hin = hin0 + i;                                                        \
            const bool ok = prow[k] < kIn && i < need && (unsigned)hin < (unsigned)a.H &&    \
                            pcol[k] != kBufOOB;                                              \
            const uint32_t vo = ok ? pcol[k] + (uint32_t)(hin * a.W * 4) : kBufOOB;          \
            _Pragma("unroll") for (int j = 0; j < 8; ++j) v[k][j] = buf_load4s(src, vo, j * cstride); \
        }                                                                                    \
    }
#define SEERA_S2_STORE(G)                                                                    \
    {                                                                                        \
        _Pragma("unroll") for (int k = 0; k < kItems; ++k) {                                 \
            const int i = 2 + (G) * kIn + prow[k];                                           \
            if (prow[k] < kIn && i < need) SEERA_S2_ITEM_WRITE(v[k], i, pch[k], pcg[k], pq4[k]) \
        }                                                                                    \
    }
    __syncthreads();  // releases step 0 (the prologue wrote its rows)
    SEERA_S2_LOAD(1)
    for (int g = 1; g < nsteps; ++g) {
        // Ring slots of group g held rows that only step g-2 read.
        SEERA_S2_STORE(g)
        SEERA_S2_LOAD(g + 1)
        __syncthreads();  // releases step g
    }
#undef SEERA_S2_LOAD
#undef SEERA_S2_STORE
#undef SEERA_S2_ITEM_WRITE
}

template <int NCH>
hipError_t launch_nch(const Stride2Args& a, int nblocks, int nftiles, hipStream_t st) {
    auto kern = stride2_conv_kernel<NCH>;
    hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(kern),
                                       hipFuncAttributeMaxDynamicSharedMemorySize,
                                       (int)a.lds_bytes);
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL(kern, dim3(nblocks, nftiles), dim3(kNT), (size_t)a.lds_bytes, st, a);
    return hipGetLastError();
}

}  // namespace

int stride2_conv(const float* in, const float* Wt, float* out, int B, int C, int H, int W, int F,
                 hipStream_t st, bool* used) {
    *used = false;
    if (B <= 0 || F <= 0 || C <= 0 || C % 32 != 0 || C > 64 || W % 4 != 0) return SEERA_OK;
    if ((reinterpret_cast<uintptr_t>(in) & 15) != 0 || (reinterpret_cast<uintptr_t>(out) & 15) != 0)
        return SEERA_OK;
    Stride2Args a{};
    a.in = in; a.out = out;
    a.B = B; a.C = C; a.H = H; a.W = W; a.F = F;
    a.Ho = (H + 2 - 4) / 2 + 1;
    a.Wo = (W + 2 - 4) / 2 + 1;
    if (a.Ho <= 0 || a.Wo <= 0 || a.Wo % 4 != 0) return SEERA_OK;
    if ((int64_t)C * H * W * 4 >= kMaxTileSpanBytes || (int64_t)F * a.Ho * a.Wo * 4 >= kMaxTileSpanBytes)
        return SEERA_OK;
    const int nch = C / 32;
    a.ncb = (a.Wo + kWC - 1) / kWC;
    a.lds_bytes = (int64_t)kNR * 2 * nch * kBC * 64 + kTailPad;
    if (a.lds_bytes > kBandMaxLds) return SEERA_OK;
    const int row_items = nch * 4 * (kBC / 2);
    if (kIn * row_items > kProd * kItems || (kIn + 2) * row_items > kPreItems * kProd)
        return SEERA_OK;
    const int nftiles = (F + 63) / 64;
    // Strip length: fewest rounds of one block per CU, each costing about
    // (steps + 1.5) step times (the prologue fetches the weights and the first
    // rows unhidden).
    const int ncu = device_cus();
    int best_l = kRows;
    double best_cost = 1e30;
    for (int L = kRows; L < a.Ho + kRows; L += kRows) {
        const int64_t blocks = (int64_t)B * ((a.Ho + L - 1) / L) * a.ncb * nftiles;
        const double cost = (double)((blocks + ncu - 1) / ncu) * ((L + kRows - 1) / kRows + 1.5);
        if (cost < best_cost) { best_cost = cost; best_l = L; }
    }
    a.L = best_l;
    a.nstrips = (a.Ho + a.L - 1) / a.L;
    const int64_t nblocks = (int64_t)B * a.nstrips * a.ncb;
    if (nblocks > 0x7fffffff) return SEERA_OK;
    const int64_t lanes = (int64_t)nftiles * 4 * nch * 16 * 64;
    if (lanes > 0x7fffffff) return SEERA_OK;
    void* ws = nullptr;
    SEERA_TRY(workspace(sizeof(half_t) * (size_t)lanes * 8, &ws, st));
    a.wk = static_cast<const half_t*>(ws);
    hipLaunchKernelGGL(prep_stride2_weights, dim3((unsigned)((lanes + 255) / 256)), dim3(256), 0, st,
                       Wt, static_cast<half_t*>(ws), F, C, nch, (int)lanes);
    SEERA_HIP_TRY(hipGetLastError());
    const hipError_t e = nch == 1 ? launch_nch<1>(a, (int)nblocks, nftiles, st)
                                  : launch_nch<2>(a, (int)nblocks, nftiles, st);
    if (e != hipSuccess) return fail_hip(e, "stride2 conv launch");
    *used = true;
    return SEERA_OK;
}

}  // namespace seera
