// conv_phase2.hip -- stride-2 transposed convolution (and the dX pass of a
// stride-2 convolution) with all four stride phases in one block.
//
// The launch computes, for row phase a and column phase c of the output
// (out row 2*oh + a, out column 2*ow + c),
//   out[b, f, 2*oh + a, 2*ow + c] =
//     sum_{k < C, t < T[a], u < U[c]} Wk_{a,c}[f, t, u, k] * in[b, k, oh + t - iph[a], ow + u - ipw[c]]
// (upsampling.cu:15-126, 376-401 for the transposed forward; convolution.cu:
// 144-265, 401-429 for a stride-2 convolution's dX), with T, U <= 2.
//
// A block owns one image, a strip of L phase rows, up to 32 phase columns and
// 32 output channels, and streams the input rows once:
//   * 4 consumer waves, one per (row phase a, 16-filter half). A wave keeps
//     every weight fragment it needs (2 column phases x C/32 chunks x 2 x 2
//     taps, fp16) in registers for the whole strip and in each step computes
//     2 phase rows x 32 phase columns x 16 filters x both column phases from
//     the ring: v_mfma_f32_16x16x32_f16 with 16 pixels x 32 channels of the
//     ring as A and the register weights as B. A lane then holds 4
//     consecutive phase columns of one filter for each column phase, which
//     interleave into 8 consecutive output floats: two 16-byte stores.
//   * 4 producer waves write the 2 input rows of the next step into the ring
//     (fp16, channel-last) and issue the loads of the step after it; they also
//     store the outputs: the consumer waves write each step's results into an
//     LDS staging tile, and during the next step but one the producers take
//     them out (counting themselves out through an LDS counter the consumers
//     wait on before they overwrite the tile) and store whole runs of four
//     output rows of a filter plane. Measured on config 5 with the consumers
//     storing their results themselves: 6.8 us of the 25 us forward were those
//     stores (the matrix waves stall on store back-pressure).
// Every input pixel frame at column offset d = u - ipw[c] is read from LDS
// once per tap row and serves both column phases where their offsets meet.
// HBM sees each input element once per 32-filter tile (plus halo rows) and
// each output element once.
#include <limits.h>

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
// 16-byte chunks, the chunk order rotated by (p >> 1) & 3. Producers write an
// item's four pixels in pairs swapped on odd column quads: the 8 lanes of a
// ds_write_b128 group (4 channel groups of two adjacent quads) then hit 8
// distinct 16-byte slots of a 128-byte window (in quad order the two quads'
// pixels sit 256 bytes apart, on the same 4 slots).
__device__ __forceinline__ int ring_off(int p, int chunk) {
    return p * 32 + ((chunk ^ ((p >> 1) & 3)) << 3);
}

constexpr int kRows = 2;          // phase rows per step
constexpr int kCons = 4 * 64;     // consumer threads
constexpr int kProd = 256;        // producer threads
constexpr int kNT = kCons + kProd;
constexpr int kItems = 2;         // input items per producer thread per step
constexpr int kPreItems = 3;      // input items per producer thread, prologue
constexpr int kWC = 32;           // phase columns per block
constexpr int kND = 3;            // column offsets d read per tap row
constexpr int kTailPad = 1024;
// Output staging tile: fp32 [4 output rows][32 filters][8 phase-column quads
// x 2 column phases], 16 slots of 16 bytes per (row, filter): slot 2*pq + c
// holds phase columns 4pq .. 4pq + 3 of column phase c (an accumulator as the
// MFMAs leave it), stored at slot (2*pq + c) ^ (f & 15) so that the
// consumers' writes (8 lanes: 8 filters at one slot) and the producers'
// reads (a slot pair of one filter) hit distinct 16-byte slots.
constexpr int kStageBytes = 4 * 32 * 16 * 16;
constexpr int kStageItems = 4;    // staged slot pairs per producer thread (4 x 32 x 8 / 256)
static_assert(kStageItems * 256 >= 4 * 32 * 8, "the producers cover the staging tile");
__device__ __forceinline__ int stage_off(int r, int f, int slot) {
    return ((r * 32 + f) * 16 + (slot ^ (f & 15))) * 4;
}

struct Phase2Args {
    const float* in;     // [B, C, H, W] fp32
    const half_t* wk;    // fragment-order fp16 weights (prep_phase2_weights)
    float* out;          // [B, F, Hout, Wout] fp32
    int B, C, H, W, F, Hout, Wout;
    int nchunks;         // C / 32
    int T[2], iph[2];    // row phase a: input row oh + t - iph[a], t < T[a]
    int U[2], ipw[2];    // column phase c: input column ow + u - ipw[c], u < U[c]
    int emin, ne;        // input row offsets used: [emin, emin + ne)
    int dmin;            // input column offsets read: [dmin, dmin + kND)
    int Hp, Wp;          // phase grid: Hout / 2 x Wout / 2
    int L;               // phase rows per strip
    int nstrips, ncb;    // strips and column tiles per image
    int BC4;             // ring pixels per plane
    int NR;              // ring rows
    int64_t lds_bytes;
    int64_t stage_off;   // byte offset of the staging tile (and its counter after it)
};

// Weight fragments in the order the consumer waves load them: for filter
// tile ft (32 filters), filter half h, row phase a: [c][chunk][t][u] blocks
// of 64 lanes x 8 halves, lane l holding filter ft*32 + h*16 + l%16 and
// channels chunk*32 + 8*(l/16) + j. Tap (t, u) of phase (a, c) is kernel
// element (r0h[a] + 2*(T[a]-1-t), r0w[c] + 2*(U[c]-1-u)) of W [C, F, R, S];
// taps past T[a] / U[c], filters >= F and channels >= C are 0.
struct Phase2Prep {
    int T[2], U[2], r0h[2], r0w[2];
};

__global__ void prep_phase2_weights(const float* __restrict__ W, half_t* __restrict__ wk, int C,
                                    int F, int R, int S, int nchunks, int total_lanes,
                                    const Phase2Prep pp) {
    const int gi = blockIdx.x * blockDim.x + threadIdx.x;  // (fragment, lane)
    if (gi >= total_lanes) return;
    const int lane = gi & 63;
    int fr = gi >> 6;
    const int u = fr & 1, t = (fr >> 1) & 1;
    fr >>= 2;
    const int ch = fr % nchunks;
    fr /= nchunks;
    const int c = fr & 1, a = (fr >> 1) & 1, h = (fr >> 2) & 1, ft = fr >> 3;
    const int f = ft * 32 + h * 16 + (lane & 15);
    const int k0 = ch * 32 + 8 * (lane >> 4);
    const bool tap_ok = t < pp.T[a] && u < pp.U[c] && f < F;
    const int r = pp.r0h[a] + 2 * (pp.T[a] - 1 - t), s = pp.r0w[c] + 2 * (pp.U[c] - 1 - u);
    float v[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        const int k = k0 + j;
        v[j] = tap_ok && k < C ? W[(((int64_t)k * F + f) * R + r) * S + s] : 0.f;
    }
    *reinterpret_cast<half8*>(wk + (int64_t)gi * 8) = pack8(v);
}

template <int NCH>
__global__ __launch_bounds__(kNT) void phase2_conv_kernel(const Phase2Args a) {
    extern __shared__ __attribute__((aligned(16))) half_t ring[];
    float* const stg = reinterpret_cast<float*>(reinterpret_cast<char*>(ring) + a.stage_off);
    int* const stg_cnt = reinterpret_cast<int*>(stg + kStageBytes / 4);
    int local = blockIdx.x;
    const int cb = local % a.ncb;
    local /= a.ncb;
    const int strip = local % a.nstrips;
    const int b = local / a.nstrips;
    const int ftile = blockIdx.y;
    const int oh0 = strip * a.L;                  // first phase row of the strip
    const int Lb = min(a.L, a.Hp - oh0);          // phase rows of this strip
    const int nsteps = (Lb + kRows - 1) / kRows;
    const int ow0 = cb * kWC;
    const int icr = ow0 + a.dmin;                 // input column of ring pixel coff
    const int ic0 = icr >= 0 ? (icr & ~3) : -((-icr + 3) & ~3);
    const int coff = icr - ic0;                   // 0..3
    const int nq = a.BC4 >> 2;
    const int plane = a.BC4 * 32;                 // halves per (ring row, chunk) plane
    // Strip input row i is image row oh0 + emin + i and sits in ring slot
    // i % NR; group g (written during step g-1) starts at row g0 + g*kRows,
    // after ne-1 halo rows.
    const int g0 = a.ne - 1;
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const rsrc_t src = make_rsrc_in(a.in, (int64_t)a.B * a.C * a.H * a.W, (int64_t)b * a.C * a.H * a.W);
    const uint32_t cstride = (uint32_t)(a.H * a.W * 4);
    const int row_items = NCH * 4 * nq;           // items per input row
    const int need = Lb + a.ne - 1;               // strip input rows used
    const int hin0 = oh0 + a.emin;                // image row of strip input row 0

    // ---- prologue: the producers request the first ne-1+kRows input rows
    // and write them to the ring; the consumers request their weights (chunk
    // by chunk, in the order the MFMAs use them), so the first MFMAs wait
    // only for the first chunk's ----
    half8 wv[2][NCH][2][2];
    const int ra = wave >> 1, fh = wave & 1;      // consumer: row phase, filter half
    if (wave < 4) {
        const half8* wsrc = reinterpret_cast<const half8*>(a.wk) +
                            (int64_t)((ftile * 2 + fh) * 2 + ra) * (8 * NCH) * 64 + lane;
#pragma unroll
        for (int ch = 0; ch < NCH; ++ch)
#pragma unroll
            for (int t = 0; t < 2; ++t)
#pragma unroll
                for (int c = 0; c < 2; ++c)
#pragma unroll
                    for (int u = 0; u < 2; ++u)
                        wv[c][ch][t][u] = wsrc[(((c * NCH + ch) * 2 + t) * 2 + u) * 64];
    } else {
        const int ptid = tid - kCons;
        if (ptid == 0) *stg_cnt = 0;  // read by the consumers only after step 0's barrier
        const int nitems = (g0 + kRows) * row_items;  // <= kPreItems * kProd (host check)
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
            const int c0 = ch * 32 + cg * 8, win = ic0 + q4 * 4;
            const bool ok = it < nitems && i < need && (unsigned)hin < (unsigned)a.H &&
                            c0 < a.C && (unsigned)win < (unsigned)a.W;
            const uint32_t vo = ok ? (uint32_t)((c0 * a.H * a.W + hin * a.W + win) * 4) : kBufOOB;
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
            if (it < nitems && i < need) {
                half_t* dst = ring + (i % a.NR) * NCH * plane + ch * plane;
                const int sw = q4 & 1;  // odd quads write their pixel pairs swapped
#pragma unroll
                for (int jj = 0; jj < 4; ++jj) {
                    float col[8];
#pragma unroll
                    for (int j = 0; j < 8; ++j) col[j] = sw ? xv[k][j][jj ^ 1] : xv[k][j][jj];
                    *reinterpret_cast<half8*>(dst + ring_off(4 * q4 + (jj ^ sw), cg)) = pack8(col);
                }
            }
        }
    }

    if (wave < 4) {
        // ---- consumers ----
        // Column tap u of phase 0 reads frame u (input column ow + dmin + u),
        // of phase 1 frame u + 1 (ipw[0] = ipw[1] + 1); every (row, chunk, row
        // tap) set is 3 frames x 2 pixel groups read once, then 8 MFMAs: tap
        // u = 0 of every (pixel group, phase), then u = 1, so dependent
        // accumulations sit four MFMAs apart. The reads of the next set are
        // issued before the MFMAs of this one.
        constexpr int ND = kND;
        constexpr int NQ = kRows * NCH * 2;
        const int kc = lane >> 4;
        const int iph = a.iph[ra];
        int poff[ND][2];
#pragma unroll
        for (int di = 0; di < ND; ++di)
#pragma unroll
            for (int pg = 0; pg < 2; ++pg) poff[di][pg] = ring_off(pg * 16 + (lane & 15) + di + coff, kc);

        for (int s = 0; s < nsteps; ++s) {
            __syncthreads();  // the rows of step s are in the ring
            // Ring slot of strip input row s*kRows + j - iph - emin (j = row + tap).
            const int base = s * kRows - iph - a.emin;  // >= 0
            int sl[3];
#pragma unroll
            for (int j = 0; j < 3; ++j) sl[j] = (base + j) % a.NR;
            floatx4_t acc[kRows][2][2];  // [row][pixel group][column phase]
#pragma unroll
            for (int r = 0; r < kRows; ++r)
#pragma unroll
                for (int pg = 0; pg < 2; ++pg)
#pragma unroll
                    for (int c = 0; c < 2; ++c) acc[r][pg][c] = floatx4_t{0.f, 0.f, 0.f, 0.f};
            half8 fb[2][ND][2];
#define SEERA_P2_READ(Q, BUF)                                                                \
    {                                                                                        \
        const int r_ = (Q) / (NCH * 2), ch_ = ((Q) / 2) % NCH, t_ = (Q) % 2;                 \
        const half_t* rp = ring + (sl[r_ + t_] * NCH + ch_) * plane;                         \
        _Pragma("unroll") for (int di = 0; di < ND; ++di)                                    \
            _Pragma("unroll") for (int pg = 0; pg < 2; ++pg)                                 \
                fb[BUF][di][pg] = *reinterpret_cast<const half8*>(rp + poff[di][pg]);        \
    }
            SEERA_P2_READ(0, 0)
#pragma unroll
            for (int q = 0; q < NQ; ++q) {
                if (q + 1 < NQ) SEERA_P2_READ(q + 1, (q + 1) & 1)
                const int r = q / (NCH * 2), ch = (q / 2) % NCH, t = q % 2;
#pragma unroll
                for (int u = 0; u < 2; ++u)
#pragma unroll
                    for (int pg = 0; pg < 2; ++pg)
#pragma unroll
                        for (int c = 0; c < 2; ++c)
                            acc[r][pg][c] = mfma16x16x32(fb[q & 1][u + c][pg],
                                                         wv[c][ch][t][u], acc[r][pg][c]);
            }
#undef SEERA_P2_READ
            // Lane: phase columns pc..pc+3 (phase quad 4*pg + kc) of filter f
            // for each column phase, staged as they are once the producers
            // have taken step s-1 out of the tile.
            while (__hip_atomic_load(stg_cnt, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP) < 4 * s)
                __builtin_amdgcn_s_sleep(1);
            const int fl = fh * 16 + (lane & 15);
#pragma unroll
            for (int r = 0; r < kRows; ++r)
#pragma unroll
                for (int pg = 0; pg < 2; ++pg)
#pragma unroll
                    for (int c = 0; c < 2; ++c)
                        *reinterpret_cast<floatx4_t*>(stg + stage_off(2 * r + ra, fl, 2 * (4 * pg + kc) + c)) =
                            acc[r][pg][c];
        }
        __syncthreads();  // the last step's results are staged
        return;
    }

    // ---- producers: input rows into the ring, one step ahead ----
    // Item k of this thread (it = ptid + k*kProd) is (row of the group,
    // chunk, 8-channel group cg, column quad q4), cg fastest; the same items
    // recur every step, only the group's first row changes.
    const int ptid = tid - kCons;
    int prow[kItems];
    uint32_t pcol[kItems];
    int pdst[kItems];
    int pcg[kItems];
    int pq4[kItems];
#pragma unroll
    for (int k = 0; k < kItems; ++k) {
        const int it = ptid + k * kProd;
        const int cg = it & 3;
        int r = it >> 2;
        const int q4 = r % nq;
        r /= nq;
        const int ch = r % NCH;
        prow[k] = it < kRows * row_items ? r / NCH : kRows;
        const int c0 = ch * 32 + cg * 8, win = ic0 + q4 * 4;
        pcol[k] = c0 < a.C && (unsigned)win < (unsigned)a.W ? (uint32_t)((c0 * a.H * a.W + win) * 4)
                                                             : kBufOOB;
        pdst[k] = ch * plane + q4 * 128;
        pcg[k] = cg;
        pq4[k] = q4;
    }
    // The rows of group g are requested during step g-2 and written during
    // step g-1 (before the barrier that releases step g).
    floatx4 v0[kItems][8];
#define SEERA_P2_LOAD(V, G)                                                                  \
    {                                                                                        \
        _Pragma("unroll") for (int k = 0; k < kItems; ++k) {                                 \
            const int i = g0 + (G) * kRows + prow[k];                                        \
            const int hin = hin0 + i;                                                        \
            const bool ok = prow[k] < kRows && i < need && (unsigned)hin < (unsigned)a.H &&  \
                            pcol[k] != kBufOOB;                                              \
            const uint32_t vo = ok ? pcol[k] + (uint32_t)(hin * a.W * 4) : kBufOOB;          \
            _Pragma("unroll") for (int j = 0; j < 8; ++j) V[k][j] = buf_load4s(src, vo, j * cstride); \
        }                                                                                    \
    }
#define SEERA_P2_STORE(V, G)                                                                 \
    {                                                                                        \
        _Pragma("unroll") for (int k = 0; k < kItems; ++k) {                                 \
            const int i = g0 + (G) * kRows + prow[k];                                        \
            if (prow[k] < kRows && i < need) {                                               \
                half_t* dst = ring + (i % a.NR) * NCH * plane + pdst[k];                     \
                const int sw = pq4[k] & 1;                                                   \
                _Pragma("unroll") for (int jj = 0; jj < 4; ++jj) {                           \
                    float col[8];                                                            \
                    _Pragma("unroll") for (int j = 0; j < 8; ++j)                            \
                        col[j] = sw ? V[k][j][jj ^ 1] : V[k][j][jj];                         \
                    /* = ring_off(4*q4 + q, cg) relative to pixel 4*q4 */                    \
                    const int q = jj ^ sw, p = 4 * pq4[k] + q;                               \
                    *reinterpret_cast<half8*>(dst + q * 32 + ((pcg[k] ^ ((p >> 1) & 3)) << 3)) = \
                        pack8(col);                                                          \
                }                                                                            \
            }                                                                                \
        }                                                                                    \
    }
    // Staged outputs: item k of this thread is (k * 256 + ptid) = (f * 4 +
    // row) * npq + pq, phase quads fastest (four consecutive output rows of a
    // filter plane are contiguous in HBM when the block spans the row): the
    // two column phases of phase columns 4pq .. 4pq + 3 interleave into output
    // columns 8pq .. 8pq + 7. Each item is read and stored in turn (8
    // registers at a time); the producers count themselves out of the tile
    // after their last read, at the start of a step whose consumers need the
    // tile only at its end.
    const int npq = min(2 * kWC, a.Wout - 2 * ow0) >> 3;
    const int nst_items = 4 * 32 * npq;
    const rsrc_t dst_img = make_rsrc_in(a.out, (int64_t)a.B * a.F * a.Hout * a.Wout, (int64_t)b * a.F * a.Hout * a.Wout);
    auto flush = [&](int st) {  // phase rows 2st, 2st + 1: output rows 4st .. 4st + 3
#pragma unroll
        for (int k = 0; k < kStageItems; ++k) {
            const int idx = k * kProd + ptid;
            const int pq = idx % npq, fr = idx / npq, fl = fr >> 2, orow = fr & 3;
            const int f = ftile * 32 + fl;
            if (idx < nst_items) {
                const float* base = stg + (orow * 32 + fl) * 64;
                const int s0 = (2 * pq) ^ (fl & 15);  // column phase 0; phase 1 is s0 ^ 1
                const floatx4_t e = *reinterpret_cast<const floatx4_t*>(base + s0 * 4);
                const floatx4_t o = *reinterpret_cast<const floatx4_t*>(base + (s0 ^ 1) * 4);
                const bool ok = f < a.F && kRows * st + (orow >> 1) < Lb;
                const uint32_t off = ok ? (uint32_t)(((f * a.Hout + 2 * oh0 + 4 * st + orow) * a.Wout +
                                                      2 * ow0 + 8 * pq) * 4) : kBufOOB;
                const floatx4_t lo = {e[0], o[0], e[1], o[1]}, hi = {e[2], o[2], e[3], o[3]};
                __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(uintx4_t, lo), dst_img, off, 0, 0);
                __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(uintx4_t, hi), dst_img,
                                                       ok ? off + 16u : kBufOOB, 0, 0);
            }
        }
        __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0): every read has returned
        if (lane == 0) __hip_atomic_fetch_add(stg_cnt, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
    };
    __syncthreads();  // releases step 0 (the prologue wrote its rows)
    SEERA_P2_LOAD(v0, 1)
    for (int g = 1; g < nsteps; ++g) {
        if (g >= 2) flush(g - 2);  // step g-2's results
        // Ring slots of group g held rows that only step g-2 read.
        SEERA_P2_STORE(v0, g)
        SEERA_P2_LOAD(v0, g + 1)
        __syncthreads();  // releases step g
    }
    if (nsteps >= 2) flush(nsteps - 2);
    __syncthreads();  // the last step's results are staged
    flush(nsteps - 1);
    __builtin_amdgcn_s_waitcnt(0);
#undef SEERA_P2_LOAD
#undef SEERA_P2_STORE
}

template <int NCH>
hipError_t launch_nch(const Phase2Args& a, int nblocks, int nftiles, hipStream_t st) {
    auto kern = phase2_conv_kernel<NCH>;
    hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(kern),
                                       hipFuncAttributeMaxDynamicSharedMemorySize,
                                       (int)a.lds_bytes);
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL(kern, dim3(nblocks, nftiles), dim3(kNT), (size_t)a.lds_bytes, st, a);
    return hipGetLastError();
}

}  // namespace

int phase2_conv(const float* in, const float* Wt, float* out, int B, int C, int H, int W, int F,
                int Hout, int Wout, int R, int S, const int T[2], const int iph[2],
                const int r0h[2], const int U[2], const int ipw[2], const int r0w[2],
                hipStream_t st, bool* used) {
    *used = false;
    if (C <= 0 || C % 32 != 0 || C > 128 || F <= 0 || B <= 0) return SEERA_OK;
    if (Hout % 2 != 0 || Wout % 8 != 0 || Hout == 0) return SEERA_OK;
    if ((reinterpret_cast<uintptr_t>(in) & 15) != 0 || (reinterpret_cast<uintptr_t>(out) & 15) != 0 ||
        W % 4 != 0)
        return SEERA_OK;
    // 2 x 2 taps per phase (a 4x4 kernel at stride 2), column phase 1 reading
    // one input column right of phase 0 (ipw[0] = ipw[1] + 1: padding 1 is the
    // one padding that meets the width conditions above and below).
    for (int z = 0; z < 2; ++z)
        if (T[z] != 2 || U[z] != 2) return SEERA_OK;
    if (ipw[0] - ipw[1] != 1) return SEERA_OK;
    if ((int64_t)C * H * W * 4 >= kMaxTileSpanBytes || (int64_t)F * Hout * Wout * 4 >= kMaxTileSpanBytes)
        return SEERA_OK;
    Phase2Args a{};
    a.in = in; a.out = out;
    a.B = B; a.C = C; a.H = H; a.W = W; a.F = F; a.Hout = Hout; a.Wout = Wout;
    a.nchunks = C / 32;
    int emax = INT_MIN, dmax = INT_MIN;
    a.emin = INT_MAX;
    a.dmin = INT_MAX;
    for (int z = 0; z < 2; ++z) {
        a.T[z] = T[z]; a.iph[z] = iph[z]; a.U[z] = U[z]; a.ipw[z] = ipw[z];
        a.emin = std::min(a.emin, -iph[z]);
        emax = std::max(emax, T[z] - 1 - iph[z]);
        a.dmin = std::min(a.dmin, -ipw[z]);
        dmax = std::max(dmax, U[z] - 1 - ipw[z]);
    }
    a.ne = emax - a.emin + 1;
    if (a.ne > 3 || dmax - a.dmin + 1 > kND) return SEERA_OK;
    a.Hp = Hout / 2;
    a.Wp = Wout / 2;
    a.ncb = (a.Wp + kWC - 1) / kWC;
    a.BC4 = (kWC + kND - 1 + 3 + 3) & ~3;
    a.NR = 2 * kRows + a.ne - 1;
    a.stage_off = (int64_t)a.NR * a.nchunks * a.BC4 * 64 + kTailPad;
    a.lds_bytes = a.stage_off + kStageBytes + 16;
    if (a.lds_bytes > kBandMaxLds) return SEERA_OK;
    const int row_items = a.nchunks * 4 * (a.BC4 / 4);
    if (kRows * row_items > kProd * kItems || (a.ne - 1 + kRows) * row_items > kPreItems * kProd)
        return SEERA_OK;
    const int nftiles = (F + 31) / 32;
    // Strip length: fewest rounds of one block per CU, each costing about
    // (steps + 1.5) step times (the prologue fetches the weights and the first
    // rows unhidden).
    const int ncu = device_cus();
    int best_l = kRows;
    double best_cost = 1e30;
    for (int L = kRows; L < a.Hp + kRows; L += kRows) {
        const int64_t blocks = (int64_t)B * ((a.Hp + L - 1) / L) * a.ncb * nftiles;
        const double cost = (double)((blocks + ncu - 1) / ncu) * ((L + kRows - 1) / kRows + 1.5);
        if (cost < best_cost) { best_cost = cost; best_l = L; }
    }
    a.L = best_l;
    a.nstrips = (a.Hp + a.L - 1) / a.L;
    const int64_t nblocks = (int64_t)B * a.nstrips * a.ncb;
    if (nblocks > 0x7fffffff) return SEERA_OK;
    // Weights: nftiles x 2 halves x 2 row phases x 2 column phases x chunks x 4 taps fragments.
    const int64_t nfrag = (int64_t)nftiles * 8 * a.nchunks * 4;
    const int64_t lanes = nfrag * 64;
    if (lanes > 0x7fffffff) return SEERA_OK;
    void* ws = nullptr;
    SEERA_TRY(workspace(sizeof(half_t) * (size_t)lanes * 8, &ws, st));
    a.wk = static_cast<const half_t*>(ws);
    Phase2Prep pp{};
    for (int z = 0; z < 2; ++z) {
        pp.T[z] = T[z]; pp.U[z] = U[z]; pp.r0h[z] = r0h[z]; pp.r0w[z] = r0w[z];
    }
    hipLaunchKernelGGL(prep_phase2_weights, dim3((unsigned)((lanes + 255) / 256)), dim3(256), 0, st,
                       Wt, static_cast<half_t*>(ws), C, F, R, S, a.nchunks, (int)lanes, pp);
    SEERA_HIP_TRY(hipGetLastError());
    hipError_t e;
    switch (a.nchunks) {
        case 1: e = launch_nch<1>(a, (int)nblocks, nftiles, st); break;
        case 2: e = launch_nch<2>(a, (int)nblocks, nftiles, st); break;
        case 3: e = launch_nch<3>(a, (int)nblocks, nftiles, st); break;
        default: e = launch_nch<4>(a, (int)nblocks, nftiles, st); break;
    }
    if (e != hipSuccess) return fail_hip(e, "phase2 conv launch");
    *used = true;
    return SEERA_OK;
}

}  // namespace seera
