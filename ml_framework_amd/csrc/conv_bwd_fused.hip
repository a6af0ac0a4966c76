// conv_bwd_fused.hip -- Conv2D backward (dX, dW and optionally db) of a 3x3,
// stride 1, pad 1 layer of 64 -> 64 channels in one pass over dY.
//
// Both gradients read dY at the same place for an input position (h, w):
//   dX[b, c, h, w]  = sum_{f, r, s} W[f, c, r, s] * dY[b, f, h + 1 - r, w + 1 - s]
//   dW[f, c, r, s]  = sum_{b, h, w} dY[b, f, h + 1 - r, w + 1 - s] * X[b, c, h, w]
//   db[f]           = sum_{b, oh, ow} dY[b, f, oh, ow]
// (convolution.cu:144-265 dX, convolution.cu:268-366 and 431-452 dW,
// Seera_Engine.py:42-65 db). A block owns one image and a strip of L rows of
// X / dX, and walks it two rows per step:
//   * 4 producer waves stream the dY rows the step adds (rows h-1 .. h+2 of
//     the step's X rows h, h+1) and the step's two X rows into two rings of
//     fp16 channel-last pixels (loaded two steps ahead, rounded on the way in);
//   * 8 consumer waves each compute a quarter of the step's dX tile
//     (v_mfma_f32_16x16x32_f16: 16 pixels x 32 filters of the dY ring as A,
//     the flipped weights, resident in LDS, as B), store it, then accumulate
//     their 32-filter x 16-channel x 9-tap slice of dW with 32 pixels of dY as
//     A and of X as B. Those fragments want pixels along K, which the
//     channel-last rings hold across lanes: ds_read_b64_tr_b16 transposes
//     them on the way out of LDS.
// HBM sees dY once (plus two halo rows per strip), X once and dX once. Each
// block writes its 64 x 576 dW partial (and 64 db partials); wgrad_reduce
// (conv_band.hip) adds them in a fixed order.
#include "conv_band.h"
#include "mfma_core.h"

namespace seera {
namespace {

typedef float floatx4_t __attribute__((ext_vector_type(4)));
typedef uint32_t uintx4_t __attribute__((ext_vector_type(4)));
typedef _Float16 half4 __attribute__((ext_vector_type(4)));
// The transposed-read builtin's operand type: 4 x __fp16 in LDS.
typedef __fp16 fp16x4_t __attribute__((__vector_size__(4 * sizeof(__fp16))));
typedef __attribute__((address_space(3))) fp16x4_t lds_fp16x4;

__device__ __forceinline__ floatx4_t mfma16x16x32(half8 a, half8 b, floatx4_t c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}

constexpr int kG = 2;              // X / dX rows per step
constexpr int kCons = 512;         // 8 consumer waves
constexpr int kProd = 256;         // 4 producer waves
constexpr int kNT = kCons + kProd;
constexpr int kNRY = 2 * kG + 2;   // dY ring rows: the step's kG + 2, the next step's kG
constexpr int kNRX = 2 * kG;       // X ring rows: the step's kG, the next step's kG
constexpr int kTaps = 9;
constexpr int kWHalves = 2 * kTaps * 2048;  // flipped weights: 2 filter chunks x 9 taps x 64 x 32
constexpr int kItems = 2;          // row items per producer thread per step
constexpr int kYPad = 4;           // dY ring pixel = column + 4
constexpr int kXPad = 8;           // X ring pixel = column + 8

// Weights: the layout of the row-streaming forward kernel (64 rows x four
// 16-byte chunks per tap, chunk order rotated by (row >> 1) & 3).
__device__ __forceinline__ int w_off(int row, int chunk) {
    return row * 32 + ((chunk ^ ((row >> 1) & 3)) << 3);
}

// Rings: pixel p of a (row, 32-channel plane) holds its 32 channels as four
// 16-byte chunks in the order chunk ^ ((p >> 1) & 3), the layout of the
// row-streaming forward kernel's ring. Measured on gfx950, a ds_read_b128 is
// conflict-free when every 8 consecutive lanes hit 8 distinct 16-byte slots
// of a 128-byte window, as is a ds_write_b128; the transposed 64-bit reads
// when each 32-lane half covers the 64 banks once. Here:
//   * dX A fragments (16 consecutive pixels at one chunk per 16 lanes): any 8
//     consecutive pixels differ in p mod 8, which fixes both the pixel's half
//     of the window and its chunk rotation;
//   * dW fragments (transposed reads of 16 channels = 32 bytes per pixel, 8
//     consecutive pixels per half-wave): pixels p and p + 4 share a 64-byte
//     column and differ in rotation bit 1, so they take its two halves;
//   * producer writes (two column quads x 4 chunks per 8 lanes): odd quads
//     write their pixel pairs swapped, so the two pixels of a write differ in
//     bit 0.
__device__ __forceinline__ int ring_off(int p, int chunk) {
    return p * 32 + ((chunk ^ ((p >> 1) & 3)) << 3);
}

__device__ __forceinline__ half4 read_tr(const half_t* p) {
    return __builtin_bit_cast(half4, __builtin_amdgcn_ds_read_tr16_b64_v4f16((lds_fp16x4*)(p)));
}
__device__ __forceinline__ half8 cat8(half4 a, half4 b) {
    return __builtin_shufflevector(a, b, 0, 1, 2, 3, 4, 5, 6, 7);
}

struct FusedArgs {
    const float* dy;    // [B, 64, H, W]
    const float* x;     // [B, 64, H, W]
    const float* w;     // [64 f, 64 c, 3, 3] conv weights (16-byte aligned)
    float* dx;          // [B, 64, H, W]
    float* part;        // [nsplit][64 f][576]: column (r*3 + s)*64 + c
    float* dbpart;      // [nsplit][64] (nullptr: no bias gradient)
    int B, H, W;
    int L, nstrip, nsplit;
    int BCY, BCX;       // ring pixels per (row, plane)
    int ncol, Wt;       // column tiles per row, columns per tile (W > 56: tiles of <= 56)
    int QW;             // X column quads per tile row (Wt / 4)
    int HQ;             // dY halo quads on each side of a tile (1 with column tiles, else 0)
    int64_t lds_bytes;
    int wbuild_once;    // the rings hold both weight chunks' fp16 copies at once
};

// The flipped weights in LDS: wl[(chunk * 9 + t*3 + u) * 2048 + w_off(c, k / 8)
// + k % 8] = W[32*chunk + k, c, 2 - t, 2 - u] in fp16, the 3x3 transposed
// convolution dX = conv(dY, flip(W)^T). Every block builds them in its
// prologue from the fp32 weights (L2-resident after the first blocks), one
// 32-filter chunk at a time, through a natural-order fp16 copy of the chunk
// in the ring area.
constexpr int kWLoads = 64 * 576 / 4 / kNT;     // float4 weight loads per thread (12)
constexpr int kPieces = kTaps * 4 * 64 / kNT;   // 16-byte pieces per thread per chunk (3)
static_assert(kWLoads * kNT * 4 == 64 * 576 && kPieces * kNT == kTaps * 4 * 64,
              "the weight build divides evenly over the block");

template <int NKB>
__global__ __launch_bounds__(kNT) void fused_bwd_kernel(const FusedArgs a) {
    extern __shared__ __attribute__((aligned(16))) half_t smem[];
    const int split = blockIdx.x;
    const int ct = split % a.ncol, bs = split / a.ncol;
    const int b = bs / a.nstrip, strip = bs - b * a.nstrip;
    const int c0 = ct * a.Wt;                  // first column of the tile
    const int h0 = strip * a.L;
    const int Lb = min(a.L, a.H - h0);         // X / dX rows of this strip
    const int nsteps = (Lb + kG - 1) / kG;
    const int PY = a.BCY * 32, PX = a.BCX * 32;  // halves per (row, plane)
    half_t* const wl = smem;
    half_t* const ry = smem + kWHalves;        // [kNRY][2 planes][BCY px][32 ch]
    half_t* const rx = ry + kNRY * 2 * PY;     // [kNRX][2 planes][BCX px][32 ch]
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const bool producer = wave >= kCons / 64;
    const int ptid = tid - kCons;
    const int HW = a.H * a.W;
    const uint32_t cstride = (uint32_t)(HW * 4);
    const int64_t total = (int64_t)a.B * 64 * HW;
    const rsrc_t ysrc = make_rsrc_in(a.dy, total, (int64_t)b * 64 * HW);
    const rsrc_t xsrc = make_rsrc_in(a.x, total, (int64_t)b * 64 * HW);
    // Items (8 channels x 4 columns) per row: X rows hold the tile's QW
    // quads, dY rows HQ more quads of halo on either side.
    const int QY = a.QW + 2 * a.HQ;
    const int row_items_x = 8 * a.QW, row_items_y = 8 * QY;
    const bool db_on = a.dbpart != nullptr;

    // Item `it` of a group of rows (nq quads per row, hq of them halo on the
    // left): (row rr, plane, 8-channel group cg, column quad q4), cg fastest;
    // quad q4 holds columns c0 + 4*(q4 - hq) .. + 3 (zeros outside the image).
    // Its 8 loads (one float4 per channel) and its ring offset for pixel
    // 4*(q4 - hq) + pad.
    auto item_load = [&](rsrc_t src, int nq, int hq, int it, int img_row, bool ok, floatx4 (&v)[8]) {
        const int cg = it & 3, q4 = (it >> 2) % nq, plane = (it >> 2) / nq;
        const int col = c0 + 4 * (q4 - hq);
        const uint32_t vo = ok && (unsigned)img_row < (unsigned)a.H && (unsigned)col < (unsigned)a.W
            ? (uint32_t)((((plane * 32 + cg * 8) * a.H + img_row) * a.W + col) * 4) : kBufOOB;
#pragma unroll
        for (int j = 0; j < 8; ++j) v[j] = buf_load4s(src, vo, j * cstride);
    };
    auto item_store = [&](half_t* ring_row, int P, int pad, int nq, int hq, int it, const floatx4 (&v)[8]) {
        const int cg = it & 3, q4 = (it >> 2) % nq, plane = (it >> 2) / nq;
        half_t* dst = ring_row + plane * P;
        const int sw = q4 & 1;  // odd quads write their pixel pairs swapped
#pragma unroll
        for (int jj = 0; jj < 4; ++jj) {
            float col[8];
#pragma unroll
            for (int j = 0; j < 8; ++j) col[j] = sw ? v[j][jj ^ 1] : v[j][jj];
            *reinterpret_cast<half8*>(dst + ring_off(4 * (q4 - hq) + pad + (jj ^ sw), cg)) = pack8(col);
        }
    };
    // A dY item's quad is the tile's own (not halo): only those enter db.
    auto own_y = [&](int it) {
        const int q4 = ((it % row_items_y) >> 2) % QY;
        return q4 >= a.HQ && q4 < a.QW + a.HQ;
    };
    // Bias gradient: the producers sum each dY item of the strip's own rows
    // (dY rows h0 .. h0 + Lb - 1) per channel, in fp32 before rounding.
    auto item_sum = [&](const floatx4 (&v)[8], float (&sum)[8]) {
#pragma unroll
        for (int j = 0; j < 8; ++j) sum[j] += (v[j][0] + v[j][1]) + (v[j][2] + v[j][3]);
    };
    float dsum[8];  // producers: per-channel sums of their dY items (prologue and loop)
#pragma unroll
    for (int j = 0; j < 8; ++j) dsum[j] = 0.f;

    // ---- prologue: dY rows [h0 - 1, h0 + 3) (strip rows j = 0..3) by the
    // producers, X rows [h0, h0 + 2) by the consumers (requested first: they
    // come from HBM), then the weights, built in LDS while the rows arrive;
    // the ring pixels outside the image (never written by the producers) are
    // zeroed ----
    {
        floatx4 pv[2][8];
        // producers ptid < 2*row_items_y: dY items it = ptid + 2*row_items_y*k
        // of rows 0..3, the channels of their loop item (so one set of bias
        // sums serves both); consumers tid < 2*row_items_x: X item tid of rows 0, 1
        const bool pro = tid < kCons ? tid < 2 * row_items_x : ptid < 2 * row_items_y;
#pragma unroll
        for (int k = 0; k < 2; ++k) {
            const int ri = producer ? row_items_y : row_items_x;
            const int it = (producer ? ptid : tid) + k * 2 * ri;
            const int rr = it / ri;
            if (producer) item_load(ysrc, QY, a.HQ, it % ri, h0 - 1 + rr, pro && rr <= Lb + 1, pv[k]);
            else if (k == 0) item_load(xsrc, a.QW, 0, it % ri, h0 + rr, pro && rr < Lb, pv[k]);
        }
        // The flipped weights, per 32-filter chunk: the fp32 rows of its
        // filters (float4 i = k * kNT + tid of the chunk's 18432 floats; both
        // chunks requested at once), their natural-order fp16 copy (filter fl
        // of the chunk, channel c, tap r*3 + s at half fl*576 + c*9 + r*3 +
        // s), then piece (tap, k quad kq, c), c fastest, gathers its 8
        // filters (a 32-lane half reads 32 distinct banks: 18-byte pixel
        // stride) and writes them as one 16-byte chunk (8 consecutive c on 8
        // distinct slots). When the rings hold both chunks' copies, one
        // barrier serves both; otherwise the chunks take turns.
        floatx4 wf[kWLoads];
#pragma unroll
        for (int k = 0; k < kWLoads; ++k) wf[k] = *reinterpret_cast<const floatx4*>(a.w + 4 * (k * kNT + tid));
        half_t* const stg = ry;
        auto put = [&](int k, half_t* base) {
            half4 h;
#pragma unroll
            for (int q = 0; q < 4; ++q) h[q] = to_half(wf[k][q]);
            *reinterpret_cast<half4*>(base + 4 * ((k % (kWLoads / 2)) * kNT + tid)) = h;
        };
        auto gather = [&](int ch, const half_t* base) {
#pragma unroll
            for (int m = 0; m < kPieces; ++m) {
                const int pc = m * kNT + tid;
                const int c = pc & 63, kq = (pc >> 6) & 3, tap = pc >> 8;
                const half_t* src = base + 8 * kq * 576 + c * 9 + (kTaps - 1 - tap);
                half8 h;
#pragma unroll
                for (int j = 0; j < 8; ++j) h[j] = src[j * 576];
                *reinterpret_cast<half8*>(wl + (ch * kTaps + tap) * 2048 + w_off(c, kq)) = h;
            }
        };
        if (a.wbuild_once) {
#pragma unroll
            for (int k = 0; k < kWLoads; ++k) put(k, stg + (k / (kWLoads / 2)) * 32 * 576);
            __syncthreads();
            gather(0, stg);
            gather(1, stg + 32 * 576);
        } else {
#pragma unroll
            for (int ch = 0; ch < 2; ++ch) {
                if (ch) __syncthreads();  // chunk 0's pieces are read
#pragma unroll
                for (int k = 0; k < kWLoads / 2; ++k) put(ch * (kWLoads / 2) + k, stg);
                __syncthreads();
                gather(ch, stg);
            }
        }
        __syncthreads();  // the staging copy is read: the rings may be written
        // pixels no item writes: dY ring [0, ylo) and [ylo + 4*QY, BCY), X
        // ring [0, kXPad) and [kXPad + Wt, BCX), of every (row, plane), 4
        // chunks each (ylo = kYPad - 4*HQ)
        const half8 z8 = {0, 0, 0, 0, 0, 0, 0, 0};
        const int ylo = kYPad - 4 * a.HQ;
        const int nyp = a.BCY - 4 * QY, nxp = a.BCX - a.Wt;
        const int nzy = kNRY * 2 * nyp * 4, nz = nzy + kNRX * 2 * nxp * 4;
        for (int i = tid; i < nz; i += kNT) {
            const bool y = i < nzy;
            const int iz = y ? i : i - nzy, np = y ? nyp : nxp;
            const int lo = y ? ylo : kXPad, span = y ? 4 * QY : a.Wt;
            const int rest = iz >> 2, pp = rest % np, rp = rest / np;
            const int px = pp < lo ? pp : span + pp;
            *reinterpret_cast<half8*>((y ? ry + rp * PY : rx + rp * PX) + px * 32 + (iz & 3) * 8) = z8;
        }
#pragma unroll
        for (int k = 0; k < 2; ++k) {
            const int ri = producer ? row_items_y : row_items_x;
            const int it = (producer ? ptid : tid) + k * 2 * ri;
            const int rr = it / ri;
            if (producer) {
                if (pro) {
                    item_store(ry + rr * 2 * PY, PY, kYPad, QY, a.HQ, it % ri, pv[k]);
                    if (db_on && rr >= 1 && rr <= Lb && own_y(it)) item_sum(pv[k], dsum);
                }
            } else if (k == 0 && pro) {
                item_store(rx + rr * 2 * PX, PX, kXPad, a.QW, 0, it % ri, pv[k]);
            }
        }
    }

    if (!producer) {
        // ---- consumers ----
        const int G = lane >> 4, e = (lane >> 2) & 3, q = lane & 3;
        // dW role: filters 32*fh + 16*fg + (0..15) (fg = 0, 1) x channels 16*cw + (0..15).
        const int fh = wave & 1, cw = wave >> 1;
        // Transposed-read offsets (halves) within a ring plane for K block 0
        // (block kb adds kb * 1024: the rotation repeats every 8 pixels).
        // Lane (G, e, q) addresses pixel 4G + e + 16*rd of the block and
        // channels 4q .. 4q + 3 of its 16-channel half; read rd hands lane l
        // those 4 pixels of channel l % 16, so MFMA K slot 8G + j holds pixel
        // 4G + (j & 3) + 16*(j >> 2) of the block, for dY and X alike.
        // (read 1 is 16 pixels = 512 halves further, same rotation)
        int oy[2];  // [fg]: dY ring pixel pd = 4G + e (dY column pd - 4)
        int ox[3];  // [s]:  X ring pixel pd + 3 + s (X column pd - 5 + s)
        {
            const int pd = 4 * G + e;
#pragma unroll
            for (int fg = 0; fg < 2; ++fg) oy[fg] = ring_off(pd, 2 * fg + (q >> 1)) + 4 * (q & 1);
#pragma unroll
            for (int s = 0; s < 3; ++s)
                ox[s] = ring_off(pd + 3 + s, 2 * (cw & 1) + (q >> 1)) + 4 * (q & 1);
        }
        // dX role: row dr of the step, pixel groups 2*pxh + pg (16 pixels
        // each) x channel groups 2*chh + cs (16 channels each), with
        // v_mfma_f32_16x16x32_f16: the A fragment lane holds pixel lane % 16,
        // the B fragment lane channel lane % 16, each 8 consecutive filters
        // (16-byte chunk kc = lane / 16 of a 32-filter plane).
        const int dr = wave >> 2, pxh = (wave >> 1) & 1, chh = wave & 1;
        const int kc = lane >> 4;
        int oa[3];  // [u]: A fragment offset of pixel group 0 within a dY plane
                    // (group 1 sits 16 pixels = 512 halves further, same rotation)
#pragma unroll
        for (int u = 0; u < 3; ++u) oa[u] = ring_off(32 * pxh + (lane & 15) + u + kYPad - 1, kc);
        const int ob = w_off(lane & 15, kc) + 512 * 2 * chh;  // + 512 * cs
        const rsrc_t dxdst = make_rsrc_in(a.dx, total, (int64_t)b * 64 * HW);

        floatx4_t acc[2][3][3];
#pragma unroll
        for (int fg = 0; fg < 2; ++fg)
#pragma unroll
            for (int r = 0; r < 3; ++r)
#pragma unroll
                for (int s = 0; s < 3; ++s) acc[fg][r][s] = floatx4_t{0.f, 0.f, 0.f, 0.f};

        for (int st = 0; st < nsteps; ++st) {
            __syncthreads();  // the rows of step st are in the rings
            const int i0 = st * kG;  // strip-relative X row of the step's first row
            // The two consumer waves of a SIMD (w and w + 4) run the dX and dW
            // halves of the step in opposite order, so that one's LDS waits in
            // the dX half (one read per MFMA) fall under the other's dW MFMAs.
            auto dx_half = [&]() {
            // ---- dX: row i0 + dr, 32 pixels x 32 channels ----
                floatx4_t ad[2][2];
#pragma unroll
                for (int pg = 0; pg < 2; ++pg)
#pragma unroll
                    for (int cs = 0; cs < 2; ++cs) ad[pg][cs] = floatx4_t{0.f, 0.f, 0.f, 0.f};
                // Three fragment sets in flight: with one, every MFMA group
                // waits out a full LDS round trip.
                half8 fa[3][2], fb[3][2];  // [buf][pg], [buf][cs]
                // K slice kk = (plane, tap): 32 filters of one tap
                auto rd_set = [&](int kk, int buf) {
                    const int plane = kk / kTaps, tap = kk % kTaps, t = tap / 3, u = tap % 3;
                    const int slot = (i0 + dr + t) % kNRY;  // dY strip row j = i + t
                    const half_t* yp = ry + (slot * 2 + plane) * PY + oa[u];
                    const half_t* wp = wl + kk * 2048 + ob;
#pragma unroll
                    for (int pg = 0; pg < 2; ++pg)
                        fa[buf][pg] = *reinterpret_cast<const half8*>(yp + 512 * pg);
#pragma unroll
                    for (int cs = 0; cs < 2; ++cs)
                        fb[buf][cs] = *reinterpret_cast<const half8*>(wp + 512 * cs);
                };
                rd_set(0, 0);
                rd_set(1, 1);
#pragma unroll
                for (int kk = 0; kk < 2 * kTaps; ++kk) {
                    if (kk + 2 < 2 * kTaps) rd_set(kk + 2, (kk + 2) % 3);
#pragma unroll
                    for (int pg = 0; pg < 2; ++pg)
#pragma unroll
                        for (int cs = 0; cs < 2; ++cs)
                            ad[pg][cs] = mfma16x16x32(fa[kk % 3][pg], fb[kk % 3][cs], ad[pg][cs]);
                    // (keeps each chunk's reads ahead of the previous chunks'
                    // MFMAs; left free, the scheduler sinks them to their use)
                    __builtin_amdgcn_sched_barrier(0);
                }
                // lane holds pixels 4*kc + (0..3) of group pg at channel lane % 16
                const int i = i0 + dr;
                if (i < Lb) {
                    const int orow = (h0 + i) * a.W + c0;
#pragma unroll
                    for (int pg = 0; pg < 2; ++pg) {
                        const int px = 32 * pxh + 16 * pg + 4 * kc;
#pragma unroll
                        for (int cs = 0; cs < 2; ++cs) {
                            const int c = 16 * (2 * chh + cs) + (lane & 15);
                            const uint32_t off = px < a.Wt && c0 + px < a.W
                                ? (uint32_t)((c * HW + orow + px) * 4) : kBufOOB;
                            __builtin_amdgcn_raw_buffer_store_b128(
                                __builtin_bit_cast(uintx4_t, ad[pg][cs]), dxdst, off, 0, 0);
                        }
                    }
                }
            };
            auto dw_half = [&]() {
            // ---- dW: X rows i0, i0 + 1 against dY rows j = i0 .. i0 + 3 ----
            // One (K block, X row) pair at a time, its three column shifts of X
            // against the three dY rows it meets (unrolled, the next pair's
            // fragments are hoisted and the consumers spill).
#pragma unroll 1
            for (int q2 = 0; q2 < 2 * NKB; ++q2) {
                const int kb = q2 >> 1, ii = q2 & 1;
                const half_t* xp = rx + (((i0 + ii) % kNRX) * 2 + (cw >> 1)) * PX + kb * 1024;
                half8 xb[3];
#pragma unroll
                for (int s = 0; s < 3; ++s)
                    xb[s] = cat8(read_tr(xp + ox[s]), read_tr(xp + ox[s] + 512));
                half8 ya[2][2];  // [buf][fg]
                // tap r pairs X row i0 + ii with dY row j = i0 + ii + 2 - r
                auto rd_y = [&](int r, int buf) {
                    const half_t* yp = ry + (((i0 + ii + 2 - r) % kNRY) * 2 + fh) * PY + kb * 1024;
#pragma unroll
                    for (int fg = 0; fg < 2; ++fg)
                        ya[buf][fg] = cat8(read_tr(yp + oy[fg]), read_tr(yp + oy[fg] + 512));
                };
                rd_y(0, 0);
#pragma unroll
                for (int r = 0; r < 3; ++r) {
                    if (r + 1 < 3) rd_y(r + 1, (r + 1) & 1);
#pragma unroll
                    for (int s = 0; s < 3; ++s)
#pragma unroll
                        for (int fg = 0; fg < 2; ++fg)
                            acc[fg][r][s] = mfma16x16x32(ya[r & 1][fg], xb[s], acc[fg][r][s]);
                }
            }
            };
            // (sched_barrier: left free, the scheduler hoists the second
            // half's independent LDS reads into the first and spills)
            dx_half();
            dw_half();
        }
        // Partial: part[split][f][(r*3 + s)*64 + c]; lane holds filters
        // 4*(lane/16) + i of its 16 x 16 tile at channel lane % 16.
        float* const dst = a.part + (int64_t)split * 64 * 576;
#pragma unroll
        for (int fg = 0; fg < 2; ++fg)
#pragma unroll
            for (int r = 0; r < 3; ++r)
#pragma unroll
                for (int s = 0; s < 3; ++s) {
                    const int n = (r * 3 + s) * 64 + 16 * cw + (lane & 15);
#pragma unroll
                    for (int i = 0; i < 4; ++i)
                        dst[(32 * fh + 16 * fg + 4 * G + i) * 576 + n] = acc[fg][r][s][i];
                }
    } else {
        // ---- producers: the rows of step s + 1 into the rings during step s ----
        // Thread ptid moves dY item ptid (k = 0: strip row j = 2(s+1) + 2 +
        // rr) and X item ptid (k = 1: strip row i = 2(s+1) + rr) of the rows a
        // step adds, so each load's buffer resource is wave-uniform. Decoded
        // once: row rr (2: none), the byte offset of its 8 channels at column
        // 4*q4 in image row 0, its ring offset (halves, pixel 4*q4 + pad)
        // within a ring row, its 8-channel group and chunk rotation.
        floatx4 va[kItems][8], vb[kItems][8];  // two steps of items in flight
        // per item: the byte offset of its 8 channels at step 0's row
        // (pbase), that row (rbase; past every limit when the thread has no
        // item), and packed: ring offset (bits 0-23), channel group (24-25),
        // chunk rotation (26-27), row rr (28-29). Step sn reads row
        // rbase + 2*sn while that row is below the strip's last dY / X row
        // and inside the image (rlim, wave-uniform).
        int pbase[kItems], rbase[kItems], pmeta[kItems];
        constexpr bool pisy[kItems] = {true, false};
        const int W4 = a.W * 4;
        const int rlim[kItems] = {min(h0 + Lb + 1, a.H), min(h0 + Lb, a.H)};
#pragma unroll
        for (int k = 0; k < kItems; ++k) {
            const int it2 = ptid;
            const int ri = pisy[k] ? row_items_y : row_items_x, nq = pisy[k] ? QY : a.QW;
            const int hq = pisy[k] ? a.HQ : 0;
            const int rr = it2 < 2 * ri ? it2 / ri : 2;
            const int ir = it2 % ri;
            const int cg = ir & 3, q4 = (ir >> 2) % nq, plane = (ir >> 2) / nq;
            const int pad = (pisy[k] ? kYPad : kXPad) - 4 * hq;
            const int col = c0 + 4 * (q4 - hq);
            const bool cin = (unsigned)col < (unsigned)a.W;  // else: zeros, every step
            rbase[k] = rr < 2 && cin ? (pisy[k] ? h0 + 1 : h0) + rr : INT_MAX / 2;
            pbase[k] = (((plane * 32 + cg * 8) * a.H) * a.W + col) * 4 + (rbase[k] < a.H ? rbase[k] * W4 : 0);
            const bool own = !pisy[k] || (q4 >= hq && q4 < a.QW + hq);
            pmeta[k] = (plane * (pisy[k] ? PY : PX) + (4 * q4 + pad) * 32) | (cg << 24) |
                       (((2 * q4 + pad / 2) & 3) << 26) | (rr << 28) | (own ? 1 << 30 : 0);
        }
        auto load_item = [&](int sn, int k, floatx4 (&v)[8]) {
            const bool ok = rbase[k] + 2 * sn < rlim[k];
            const uint32_t vo = ok ? (uint32_t)(pbase[k] + 2 * sn * W4) : kBufOOB;
#pragma unroll
            for (int j = 0; j < 8; ++j) v[j] = buf_load4s(pisy[k] ? ysrc : xsrc, vo, j * cstride);
        };
        auto store_item = [&](int sn, int k, const floatx4 (&v)[8]) {
            {
                // dY strip row j = 2sn + 2 + rr up to the last step's window
                // (rows past Lb + 1 are zeros), X strip rows up to 2*nsteps
                // (rows past the strip are zeros)
                const int prr = (pmeta[k] >> 28) & 3, pcg = (pmeta[k] >> 24) & 3, prq = (pmeta[k] >> 26) & 3;
                const int r = 2 * sn + prr + (pisy[k] ? 2 : 0);
                if (prr < 2 && r < 2 * nsteps + (pisy[k] ? 2 : 0)) {
                    half_t* dst = (pisy[k] ? ry + (r % kNRY) * 2 * PY : rx + (r % kNRX) * 2 * PX) +
                                  (pmeta[k] & 0xFFFFFF);
                    const int sw = prq >> 1;  // odd quads: pixel pairs swapped
#pragma unroll
                    for (int jj = 0; jj < 4; ++jj) {
                        float col[8];
#pragma unroll
                        for (int j = 0; j < 8; ++j) col[j] = sw ? v[j][jj ^ 1] : v[j][jj];
                        const int q = jj ^ sw;  // = ring_off(4*q4 + pad + q, cg) - pdst
                        *reinterpret_cast<half8*>(dst + q * 32 + ((pcg ^ ((prq + (q >> 1)) & 3)) << 3)) =
                            pack8(col);
                    }
                    if (db_on && pisy[k] && r <= Lb && ((pmeta[k] >> 30) & 1)) item_sum(v, dsum);
                }
            }
        };
        __syncthreads();  // releases step 0 (the prologue wrote its rows)
        // Step s+2's rows are requested before step s+1's are written, item
        // by item, so each load has a whole step to arrive (the two register
        // sets alternate; loads past the last step read nothing).
        auto step = [&](int sn, floatx4 (&vs)[kItems][8], floatx4 (&vl)[kItems][8]) {
#pragma unroll
            for (int k = 0; k < kItems; ++k) {
                load_item(sn + 1, k, vl[k]);
                // (left free, the scheduler sinks the loads below the stores)
                __builtin_amdgcn_sched_barrier(0);
                store_item(sn, k, vs[k]);  // its ring slots held rows only step sn-2 read
            }
        };
#pragma unroll
        for (int k = 0; k < kItems; ++k) load_item(1, k, va[k]);
        for (int s = 0; s + 1 < nsteps; s += 2) {
            step(s + 1, va, vb);
            __syncthreads();  // releases step s+1
            if (s + 2 >= nsteps) break;
            step(s + 2, vb, va);
            __syncthreads();  // releases step s+2
        }
    }
    if (db_on) {
        // The producers' sums meet in LDS once every consumer is past its
        // last ring read: thread ptid < 2*row_items_y holds the sums of in-row
        // item ptid % row_items_y over its rows (rr = ptid / row_items_y, + 2
        // per step, and the prologue's rows 1..3).
        __syncthreads();
        // (the producer index is rebuilt from the wave and lane ids rather
        // than kept live through the loop, where every register is taken)
        const int ptid = wave * 64 + (int)__builtin_amdgcn_mbcnt_hi(~0u, __builtin_amdgcn_mbcnt_lo(~0u, 0u)) - kCons;
        floatx4* const red = reinterpret_cast<floatx4*>(smem);
        if (producer && ptid < 2 * row_items_y) {
            red[2 * ptid] = floatx4{dsum[0], dsum[1], dsum[2], dsum[3]};
            red[2 * ptid + 1] = floatx4{dsum[4], dsum[5], dsum[6], dsum[7]};
        }
        __syncthreads();
        if (producer && ptid < 64) {
            // filter f = 32*plane + 8*cg + j: items (rr, plane, cg, q4) in order
            const int f = ptid, plane = f >> 5, cg = (f >> 3) & 3, j = f & 7;
            const float* redf = reinterpret_cast<const float*>(smem);
            float sum = 0.f;
            for (int rr = 0; rr < 2; ++rr)
                for (int q4 = 0; q4 < QY; ++q4) {
                    const int slot = rr * row_items_y + (plane * QY + q4) * 4 + cg;
                    sum += redf[slot * 8 + j];
                }
            a.dbpart[(int64_t)split * 64 + f] = sum;
        }
    }
}

}  // namespace

int fused_conv_bwd(const float* dY, const float* Wconv, const float* X, float* dX, float* dW,
                   float* db, int B, int C, int H, int W, int F, int R, int S, int sh, int sw,
                   int ph, int pw, hipStream_t st, bool* used) {
    *used = false;
    if (C != 64 || F != 64 || R != 3 || S != 3 || sh != 1 || sw != 1 || ph != 1 || pw != 1)
        return SEERA_OK;
    if (B < 1 || H < 1 || W < 4 || W % 4 != 0) return SEERA_OK;
    if (((reinterpret_cast<uintptr_t>(dY) | reinterpret_cast<uintptr_t>(X) |
          reinterpret_cast<uintptr_t>(dX) | reinterpret_cast<uintptr_t>(Wconv)) & 15) != 0)
        return SEERA_OK;
    if ((int64_t)64 * H * W * 4 > kMaxTileSpanBytes) return SEERA_OK;
    FusedArgs a{};
    a.dy = dY; a.x = X; a.dx = dX; a.w = Wconv;
    a.B = B; a.H = H; a.W = W;
    // Rows wider than 56 run as column tiles of at most 56: each tile's dY
    // rows carry one quad of halo on either side (the dX of its edge columns
    // reads one dY column past them; dW pairs the tile's own X columns with
    // them), and db counts only the tile's own dY columns.
    a.ncol = (W + 55) / 56;
    a.Wt = ((W + a.ncol - 1) / a.ncol + 3) & ~3;
    a.HQ = a.ncol > 1 ? 1 : 0;
    a.QW = a.Wt / 4;
    const int QY = a.QW + 2 * a.HQ;
    if (2 * 8 * QY > kProd || 2 * 8 * a.QW > kCons) return SEERA_OK;  // items per row pair
    // K blocks of 32 dY pixels cover ring pixels [0, 32*nkb), i.e. columns
    // [-4, 32*nkb - 4) of the tile; the dX fragments reach ring pixel Wt + 4.
    const int nkb = (a.Wt + 5 + 31) / 32;
    a.BCY = 32 * nkb;
    a.BCX = 32 * nkb + kXPad;
    if (a.BCY < kYPad - 4 * a.HQ + 4 * QY) return SEERA_OK;  // the halo quad must fit the ring
    a.lds_bytes = (int64_t)kWHalves * 2 + (int64_t)kNRY * 2 * a.BCY * 64 + (int64_t)kNRX * 2 * a.BCX * 64;
    if (a.lds_bytes > kBandMaxLds) return SEERA_OK;
    // the db reduction reuses the rings: 2 rows of items x 8 floats; the
    // weight build stages one chunk (18432 halves) there
    if ((int64_t)2 * 8 * QY * 32 > a.lds_bytes) return SEERA_OK;
    const int64_t ring_halves = (int64_t)kNRY * 2 * a.BCY * 32 + (int64_t)kNRX * 2 * a.BCX * 32;
    if (ring_halves < 32 * 576) return SEERA_OK;
    a.wbuild_once = ring_halves >= 64 * 576;
    // Strip length: fewest rounds of one block per CU, each about (steps + 2)
    // step times.
    const int ncu = device_cus();
    double best = 1e30;
    for (int L = kG; L < H + kG; L += kG) {
        const int64_t blocks = (int64_t)B * ((H + L - 1) / L) * a.ncol;
        const double cost = (double)((blocks + ncu - 1) / ncu) * ((L + kG - 1) / kG + 2);
        if (cost < best) { best = cost; a.L = L; }
    }
    a.nstrip = (H + a.L - 1) / a.L;
    if ((int64_t)B * a.nstrip * a.ncol > 0x7fffffff) return SEERA_OK;
    a.nsplit = B * a.nstrip * a.ncol;
    const size_t part_n = (size_t)a.nsplit * 64 * 576, db_n = db ? (size_t)a.nsplit * 64 : 0;
    void* ws = nullptr;
    SEERA_TRY(workspace(sizeof(float) * (part_n + db_n), &ws, st));
    a.part = static_cast<float*>(ws);
    a.dbpart = db ? a.part + part_n : nullptr;
    const void* k = nkb == 1 ? reinterpret_cast<const void*>(fused_bwd_kernel<1>)
                             : reinterpret_cast<const void*>(fused_bwd_kernel<2>);
    SEERA_HIP_TRY(hipFuncSetAttribute(k, hipFuncAttributeMaxDynamicSharedMemorySize, (int)a.lds_bytes));
    void* args[] = {&a};
    SEERA_HIP_TRY(hipLaunchKernel(k, dim3(a.nsplit), dim3(kNT), args, (size_t)a.lds_bytes, st));
    SEERA_TRY(reduce_wgrad_partials(a.part, dW, 64, 64, 3, 3, 64, 1, 1, a.nsplit, st, a.dbpart, db));
    *used = true;
    return SEERA_OK;
}

}  // namespace seera
