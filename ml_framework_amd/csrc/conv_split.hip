// conv_split.hip -- 3x3, stride 1, pad 1 convolution of 64 input channels
// (the Conv2D forward of such a layer, and its dX through flipped weights) by
// row streaming with three wave roles, so that no matrix-core wave ever
// touches global memory:
//   out[b, f, oh, ow] = sum_{c, t, u} Wk[f, t, u, c] * in[b, c, oh + t - 1, ow + u - 1]
// (convolution.cu:15-101 forward; convolution.cu:144-265 dX).
//
// Inputs of more than 64 channels (a multiple of 64) run as one launch per
// 64-channel slice, each after the first adding its sums to the output it
// finds (the fused epilogue on the last one).
//
// A block owns one image, a strip of L output rows, up to 56 columns (rows
// wider than that run as column tiles, each ring row holding the tile's
// columns and one quad of halo on either side) and 64 filters, and walks the
// strip two output rows per step. One wave of each role per SIMD:
//   * 4 consumer waves: wave w computes half w&1 (32 pixels) of output row
//     w>>1 of the step for all 64 filters (v_mfma_f32_16x16x32_f16, 16 pixels
//     x 32 channels of the ring as A, the LDS-resident weights as B; the 18
//     fragment sets of a step fully unrolled, read three sets ahead) and
//     writes the fp32 results into an LDS staging tile;
//   * 4 producer waves: the two input rows a step adds, requested two steps
//     ahead (two register sets), rounded to fp16 and written channel-last
//     into a ring of 6 rows;
//   * 4 storer waves: during step s they take step s-1's results out of the
//     staging tile, count themselves out of it (an LDS counter the consumers
//     wait on before they overwrite it), apply the fused epilogue (bias, ReLU,
//     mask) and store them: each store instruction covers whole runs of two
//     output rows of a filter plane.
// Measured on the Conv2D config-4 forward with the single-role-pair stream
// kernel: without its output stores the kernel ran 12 us shorter, without its
// input loads 8.5 us, and with 44 % fewer LDS reads no shorter: the matrix
// waves were held by their own stores' back-pressure, which this layout
// takes off them.
#include <type_traits>

#include "conv_band.h"
#include "mfma_core.h"

namespace seera {
namespace {

typedef float floatx4_t __attribute__((ext_vector_type(4)));
typedef uint32_t uintx4_t __attribute__((ext_vector_type(4)));

__device__ __forceinline__ floatx4_t mfma16x16x32(half8 a, half8 b, floatx4_t c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}

// f(integral_constant<int, I>) for I = B .. E-1, in order.
template <int B, int E, class F>
__device__ __forceinline__ void static_for(F&& f) {
    if constexpr (B < E) {
        f(std::integral_constant<int, B>{});
        static_for<B + 1, E>(f);
    }
}

// Ring / weight layout of the row-streaming kernels (conv_stream.hip): pixel
// (or filter) p holds its 32 channels as four 16-byte chunks in the order
// chunk ^ ((p >> 1) & 3).
__device__ __forceinline__ int ring_off(int p, int chunk) {
    return p * 32 + ((chunk ^ ((p >> 1) & 3)) << 3);
}

// Staging tile: fp32 [2 rows][64 filters][16 column quads], quad q of filter
// f at slot q ^ (f & 15), so that both the consumers' 16-byte writes (8 lanes:
// 8 filters at one quad) and the storers' reads (8 lanes: 8 quads of a
// filter) hit 8 distinct 16-byte slots of a 128-byte window.
__device__ __forceinline__ int stage_off(int r, int f, int q) {
    return ((r * 64 + f) * 16 + (q ^ (f & 15))) * 4;
}

constexpr int kWaves = 4;                  // waves per role
constexpr int kNT = 3 * kWaves * 64;       // consumers, producers, storers
constexpr int kNRing = 6;                  // ring rows: a step's 4, the next step's 2
constexpr int kWPieces = 2 * 9 * 256;      // 16-byte weight pieces (2 chunks x 9 taps x 64 x 4)
constexpr int kPreW = kWPieces / kNT;      // per thread (6)
constexpr int kStageBytes = 2 * 64 * 16 * 16;
constexpr int kStoreItems = 7;             // staged float4s per storer thread (2 x 64 x 14 / 256)
static_assert(kPreW * kNT == kWPieces, "the weight pieces divide evenly over the block");

struct SplitArgs {
    const float* in;     // 64 input channels of image b at in + b * in_bstride ([64, H, W] fp32)
    int64_t in_bstride;  // floats per input image (C * H * W)
    const half_t* wk;    // prepared fp16 weights (conv_band.hip layout) of those 64 channels
    int64_t wk_fstride;  // halves per 64-filter tile of wk
    float* out;          // [B, F, H, W] fp32
    int B, H, W, F;
    int L, nstrip;       // output rows per strip, strips per image
    int ncol, Wt;        // column tiles per row, columns per tile (W > 56: tiles of <= 56)
    int nq;              // ring column quads per row (W/4 + 2)
    int nqo;             // output column quads per row (W/4)
    ConvEpi epi;
};

constexpr int kEpiNone = 0, kEpiBias = 1, kEpiBiasRelu = 2;

// ACC: out += this launch's sums (a later 64-channel pass of a wider input;
// the epilogue, if any, applies to the total).
template <int EPI, bool ACC>
__global__ __launch_bounds__(kNT) void split_conv_kernel(const SplitArgs a) {
    extern __shared__ __attribute__((aligned(16))) half_t smem[];
    const int ct = blockIdx.x % a.ncol, bs = blockIdx.x / a.ncol;
    const int strip = bs % a.nstrip, b = bs / a.nstrip;
    const int c0 = ct * a.Wt;                  // first column of the tile
    const int ftile = blockIdx.y;
    const int ohA = strip * a.L;
    const int Lb = min(a.L, a.H - ohA);        // output rows of this strip
    const int nsteps = (Lb + 1) / 2;
    const int need = Lb + 2;                   // strip input rows (row i = image row ohA - 1 + i)
    const int BC4 = 4 * a.nq;
    const int plane = BC4 * 32;                // halves per (ring row, 32-channel plane)
    half_t* const wl = smem;
    half_t* const ring = smem + kWPieces * 8;
    float* const stg = reinterpret_cast<float*>(ring + kNRing * 2 * plane);
    int* const stg_cnt = reinterpret_cast<int*>(stg + kStageBytes / 4);
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int HW = a.H * a.W;
    const rsrc_t src = make_rsrc_in(a.in, (int64_t)(a.B - 1) * a.in_bstride + 64 * HW, (int64_t)b * a.in_bstride);
    const uint32_t cstride = (uint32_t)(HW * 4);
    const int row_items = 8 * a.nq;            // (plane, 8-channel group, column quad) per row

    // Item it of a group of rows: (row rr, plane ch, group cg, quad q4), cg
    // fastest; loads of its 8 channels x 4 columns (zeros outside the image)
    // and their fp16 write into ring slot (first row + rr) % 6.
    auto item_load = [&](int it, int i0, bool on, floatx4 (&v)[8]) {
        const int cg = it & 3, q4 = (it >> 2) % a.nq, ch = (it >> 2) / a.nq % 2;
        const int rr = it / row_items, i = i0 + rr, hin = ohA - 1 + i, win = c0 + 4 * q4 - 4;
        const bool ok = on && (unsigned)hin < (unsigned)a.H && (unsigned)win < (unsigned)a.W;
        const uint32_t vo = ok ? (uint32_t)((((ch * 32 + cg * 8) * a.H + hin) * a.W + win) * 4) : kBufOOB;
#pragma unroll
        for (int j = 0; j < 8; ++j) v[j] = buf_load4s(src, vo, j * cstride);
    };
    auto item_store = [&](int it, int i0, const floatx4 (&v)[8]) {
        const int cg = it & 3, q4 = (it >> 2) % a.nq, ch = (it >> 2) / a.nq % 2;
        const int i = i0 + it / row_items;
        half_t* dst = ring + ((i % kNRing) * 2 + ch) * plane;
        const int sw = q4 & 1;  // odd quads write their pixel pairs swapped (conflict-free b128)
#pragma unroll
        for (int jj = 0; jj < 4; ++jj) {
            float col[8];
#pragma unroll
            for (int j = 0; j < 8; ++j) col[j] = sw ? v[j][jj ^ 1] : v[j][jj];
            *reinterpret_cast<half8*>(dst + ring_off(4 * q4 + (jj ^ sw), cg)) = pack8(col);
        }
    };

    // ---- prologue, by all waves: the weights and strip input rows 0..3 ----
    {
        const half_t* wsrc = a.wk + (int64_t)ftile * a.wk_fstride;
        half8 wv[kPreW];
#pragma unroll
        for (int k = 0; k < kPreW; ++k) wv[k] = *reinterpret_cast<const half8*>(wsrc + (int64_t)(k * kNT + tid) * 8);
        floatx4 xv[8];
        const bool pro = tid < 4 * row_items;
        item_load(tid, 0, pro && tid / row_items < need, xv);
#pragma unroll
        for (int k = 0; k < kPreW; ++k) {
            const int i = k * kNT + tid;
            *reinterpret_cast<half8*>(wl + (i >> 8) * 2048 + ring_off((i & 255) >> 2, i & 3)) = wv[k];
        }
        if (pro && tid / row_items < need) item_store(tid, 0, xv);
        if (tid == 0) *stg_cnt = 0;
    }
    __syncthreads();  // B0: step 0's rows and the weights are in LDS

    if (wave < kWaves) {
        // ---- consumers ----
        const int dr = wave >> 1, px0 = 32 * (wave & 1), kc = lane >> 4;
        int poff[3][2];
#pragma unroll
        for (int u = 0; u < 3; ++u)
#pragma unroll
            for (int pg = 0; pg < 2; ++pg) poff[u][pg] = ring_off(px0 + 16 * pg + (lane & 15) + u + 3, kc);
        const int wrow = ring_off(lane & 15, kc);
        for (int s = 0; s < nsteps; ++s) {
            floatx4_t acc[2][4];
#pragma unroll
            for (int pg = 0; pg < 2; ++pg)
#pragma unroll
                for (int fg = 0; fg < 4; ++fg) acc[pg][fg] = floatx4_t{0.f, 0.f, 0.f, 0.f};
            const int o = 2 * s + dr;  // strip output row; its tap-t input row is o + t
            // set q = (ch * 3 + t) * 3 + u, in fragment buffer q & 3
            half8 fa[4][4], fb[4][2];
#define SEERA_SPLIT_READ(Q)                                                                 \
    {                                                                                       \
        constexpr int ch_ = (Q) / 9, t_ = ((Q) / 3) % 3, u_ = (Q) % 3, b_ = (Q) & 3;        \
        const half_t* w = wl + ((ch_ * 3 + t_) * 3 + u_) * 2048 + wrow;                     \
        const half_t* rp = ring + (((o + t_) % kNRing) * 2 + ch_) * plane;                  \
        _Pragma("unroll") for (int pg = 0; pg < 2; ++pg) fb[b_][pg] =                       \
            *reinterpret_cast<const half8*>(rp + poff[u_][pg]);                             \
        _Pragma("unroll") for (int fg = 0; fg < 4; ++fg) fa[b_][fg] =                       \
            *reinterpret_cast<const half8*>(w + 512 * fg);                                  \
    }
            SEERA_SPLIT_READ(0)
            SEERA_SPLIT_READ(1)
            SEERA_SPLIT_READ(2)
            static_for<0, 18>([&](auto qc) {
                constexpr int q = decltype(qc)::value;
                if constexpr (q + 3 < 18) SEERA_SPLIT_READ(q + 3)
#pragma unroll
                for (int pg = 0; pg < 2; ++pg)
#pragma unroll
                    for (int fg = 0; fg < 4; ++fg)
                        acc[pg][fg] = mfma16x16x32(fb[q & 3][pg], fa[q & 3][fg], acc[pg][fg]);
                __builtin_amdgcn_sched_barrier(0);
            });
#undef SEERA_SPLIT_READ
            // The storers have taken step s-1's results out of the staging
            // tile once all four counted themselves out (4 per step).
            while (__hip_atomic_load(stg_cnt, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP) < 4 * s)
                __builtin_amdgcn_s_sleep(1);
            // lane: pixels 4*(lane/16) + r of group pg at filter 16*fg + lane%16
#pragma unroll
            for (int pg = 0; pg < 2; ++pg)
#pragma unroll
                for (int fg = 0; fg < 4; ++fg)
                    *reinterpret_cast<floatx4_t*>(stg + stage_off(dr, 16 * fg + (lane & 15),
                                                                  (px0 >> 2) + 4 * pg + kc)) = acc[pg][fg];
            __syncthreads();  // B(s+1)
        }
        return;
    }

    if (wave < 2 * kWaves) {
        // ---- producers: step k's two new rows are strip input rows 2k+2,
        // 2k+3, requested during step k-2 and written during step k-1 ----
        const int ptid = tid - kWaves * 64;
        const bool has = ptid < 2 * row_items;
        floatx4 va[8], vb[8];
        auto rows_of = [](int k) { return 2 * k + 2; };
        item_load(ptid, rows_of(1), has && 1 < nsteps && ptid / row_items + rows_of(1) < need, va);
        item_load(ptid, rows_of(2), has && 2 < nsteps && ptid / row_items + rows_of(2) < need, vb);
        for (int s = 0; s < nsteps; s += 2) {
            // step s: write step s+1's rows (va), then request step s+3's into va
            if (has && s + 1 < nsteps && ptid / row_items + rows_of(s + 1) < need)
                item_store(ptid, rows_of(s + 1), va);
            item_load(ptid, rows_of(s + 3), has && s + 3 < nsteps && ptid / row_items + rows_of(s + 3) < need, va);
            __syncthreads();  // B(s+1)
            if (s + 1 >= nsteps) break;
            if (has && s + 2 < nsteps && ptid / row_items + rows_of(s + 2) < need)
                item_store(ptid, rows_of(s + 2), vb);
            item_load(ptid, rows_of(s + 4), has && s + 4 < nsteps && ptid / row_items + rows_of(s + 4) < need, vb);
            __syncthreads();  // B(s+2)
        }
        __builtin_amdgcn_s_waitcnt(0);  // loads past the last step read nothing; drain them
        return;
    }

    // ---- storers: during step s (s >= 1) the results of step s-1; after the
    // last barrier those of the last step ----
    const int stid = tid - 2 * kWaves * 64;
    const int nitems = 2 * 64 * a.nqo;
    const int64_t out_n = (int64_t)a.B * a.F * HW, out_o = (int64_t)b * a.F * HW;
    const rsrc_t dst_img = make_rsrc_in(a.out, out_n, out_o);
    const rsrc_t mask_img = make_rsrc_in(EPI == kEpiBiasRelu && a.epi.mask ? a.epi.mask : a.out, out_n, out_o);
    const bool mask_on = EPI == kEpiBiasRelu && a.epi.mask;
    // item k: index (k * 256 + stid) = (f * 2 + r) * nqo + q, quads fastest:
    // two output rows of a filter plane are contiguous in HBM
    int sf[kStoreItems], sr[kStoreItems], sq[kStoreItems];
    float sbias[kStoreItems];
#pragma unroll
    for (int k = 0; k < kStoreItems; ++k) {
        const int idx = k * 256 + stid;
        const int q = idx % a.nqo, fr = idx / a.nqo;
        sf[k] = idx < nitems ? fr >> 1 : -1;
        sr[k] = fr & 1;
        sq[k] = q;
        const int fg = ftile * 64 + (fr >> 1);
        sbias[k] = EPI != kEpiNone && a.epi.bias && sf[k] >= 0 && fg < a.F ? a.epi.bias[fg] : 0.f;
    }
    // Output offset of item k of step st (kBufOOB past the strip or tile).
    auto item_off = [&](int st, int k) {
        const int o = 2 * st + sr[k], f = ftile * 64 + sf[k];
        return o < Lb && f < a.F && c0 + 4 * sq[k] < a.W
            ? (uint32_t)(((f * a.H + ohA + o) * a.W + c0 + 4 * sq[k]) * 4) : kBufOOB;
    };
    // ACC: the output's current values of the items of the next step to
    // store, requested a step ahead (loads issued after a store of the same
    // buffer would otherwise each wait out the store before them).
    floatx4_t old[kStoreItems];
    auto load_old = [&](int st) {
#pragma unroll
        for (int k = 0; k < kStoreItems; ++k)
            old[k] = __builtin_bit_cast(floatx4_t, __builtin_amdgcn_raw_buffer_load_b128(
                         dst_img, sf[k] >= 0 ? item_off(st, k) : kBufOOB, 0, 0));
    };
    if constexpr (ACC) load_old(0);
    for (int s = 0; s <= nsteps; ++s) {
        if (s > 0) {
            const int st = s - 1;  // the staged step
            floatx4_t v[kStoreItems];
#pragma unroll
            for (int k = 0; k < kStoreItems; ++k)
                if (sf[k] >= 0) v[k] = *reinterpret_cast<const floatx4_t*>(stg + stage_off(sr[k], sf[k], sq[k]));
            // every read of this wave has returned: the tile may be overwritten
            __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0)
            if (lane == 0) __hip_atomic_fetch_add(stg_cnt, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
#pragma unroll
            for (int k = 0; k < kStoreItems; ++k) {
                if (sf[k] < 0) continue;
                const uint32_t off = item_off(st, k);
                floatx4_t x = v[k];
                if constexpr (ACC) x += old[k];
                if constexpr (EPI != kEpiNone) {
#pragma unroll
                    for (int j = 0; j < 4; ++j) {
                        const float t = x[j] + sbias[k];
                        x[j] = EPI == kEpiBiasRelu ? (t > 0.f ? t : 0.f) : t;
                    }
                }
                __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(uintx4_t, x), dst_img, off, 0, 0);
                if (mask_on) {
                    floatx4_t m;
#pragma unroll
                    for (int j = 0; j < 4; ++j) m[j] = x[j] > 0.f ? 1.f : 0.f;
                    __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(uintx4_t, m), mask_img, off, 0, 0);
                }
            }
            if constexpr (ACC)
                if (st + 1 < nsteps) load_old(st + 1);
        }
        if (s < nsteps) __syncthreads();  // B(s+1)
    }
}

template <int EPI, bool ACC>
hipError_t launch(const SplitArgs& a, int nblocks, int nftiles, int lds, hipStream_t st) {
    auto kern = split_conv_kernel<EPI, ACC>;
    hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(kern),
                                       hipFuncAttributeMaxDynamicSharedMemorySize, lds);
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL(kern, dim3(nblocks, nftiles), dim3(kNT), (size_t)lds, st, a);
    return hipGetLastError();
}

}  // namespace

int split_conv(const BandConvArgs& band, hipStream_t st, bool* used) {
    *used = false;
    // Inputs of 64k channels run as k launches over 64-channel slices, each
    // after the first adding its sums to the output.
    if (band.nphase != 1 || band.C < 64 || band.C % 64 != 0 || band.nchunks != band.C / 32 ||
        band.ish != 1 || band.isw != 1 || band.osh != 1 || band.osw != 1)
        return SEERA_OK;
    const BandPhase& P = band.ph[0];
    if (P.T != 3 || P.U != 3 || P.iph != 1 || P.ipw != 1 || P.oph != 0 || P.opw != 0 || P.woff != 0)
        return SEERA_OK;
    if (band.Hout != band.H || band.Wout != band.W || P.Ho != band.H || P.Wo != band.W) return SEERA_OK;
    if (band.W < 4 || band.W % 4 != 0 || band.H < 1 || band.B < 1) return SEERA_OK;
    if ((reinterpret_cast<uintptr_t>(band.out) & 15) != 0 || (reinterpret_cast<uintptr_t>(band.in) & 15) != 0)
        return SEERA_OK;
    if ((int64_t)64 * band.H * band.W * 4 > kMaxTileSpanBytes ||
        (int64_t)band.F * band.H * band.W * 4 > kMaxTileSpanBytes)
        return SEERA_OK;
    // Each further slice reads and rewrites the output once more: against the
    // band kernel, measured faster up to 4 (slice, filter tile) launches on
    // rows of 56 or more (16x128x112^2 -> 128: 160 -> 114 us; 64x128x56^2 ->
    // 128: 150 -> 109) or with one filter tile (32x192x28^2 -> 64: 46 -> 36),
    // slower on 28-column rows with two filter tiles (45 -> 52) and at 256
    // channels and filters (137 -> 185 at 28^2, 73 -> 91 at 56^2).
    const int npass = band.C / 64;
    if (npass > 1 && !(npass * band.nftiles <= 4 && (band.W >= 56 || band.nftiles == 1)))
        return SEERA_OK;
    SplitArgs a{};
    a.in = band.in; a.wk = band.wk; a.out = band.out; a.epi = band.epi;
    a.in_bstride = (int64_t)band.C * band.H * band.W;
    a.wk_fstride = (int64_t)band.nchunks * 9 * 2048;
    a.B = band.B; a.H = band.H; a.W = band.W; a.F = band.F;
    // Rows wider than 56 run as column tiles of at most 56 (the ring holds a
    // tile's columns plus a quad of halo on each side).
    a.ncol = (band.W + 55) / 56;
    a.Wt = ((band.W + a.ncol - 1) / a.ncol + 3) & ~3;
    a.nq = a.Wt / 4 + 2;
    a.nqo = a.Wt / 4;
    if (2 * 8 * a.nq > 256 || 4 * 8 * a.nq > kNT || 2 * 64 * a.nqo > kStoreItems * 256) return SEERA_OK;
    const int lds = kWPieces * 16 + kNRing * 2 * (4 * a.nq) * 64 + kStageBytes + 16;
    if (lds > kBandMaxLds) return SEERA_OK;
    // Strip length (even): fewest rounds of one block per CU, each about
    // (steps + 1.5) step times.
    const int ncu = device_cus();
    double best = 1e30;
    for (int L = 2; L < a.H + 2; L += 2) {
        const int64_t blocks = (int64_t)a.B * ((a.H + L - 1) / L) * a.ncol * band.nftiles;
        const double cost = (double)((blocks + ncu - 1) / ncu) * ((L + 1) / 2 + 1.5);
        if (cost < best) { best = cost; a.L = L; }
    }
    a.nstrip = (a.H + a.L - 1) / a.L;
    const int64_t nblocks = (int64_t)a.B * a.nstrip * a.ncol;
    if (nblocks > 0x7fffffff || band.nftiles > 65535) return SEERA_OK;
    const ConvEpi epi = band.epi;
    for (int pass = 0; pass < npass; ++pass) {
        SplitArgs q = a;
        q.in = band.in + (int64_t)pass * 64 * band.H * band.W;
        q.wk = band.wk + (int64_t)pass * 2 * 9 * 2048;  // chunks 2*pass, 2*pass + 1 of each tile
        q.epi = pass + 1 == npass ? epi : ConvEpi{};   // the epilogue on the total only
        const bool acc = pass > 0;
        hipError_t e;
        if (q.epi.act == kActRelu)
            e = acc ? launch<kEpiBiasRelu, true>(q, (int)nblocks, band.nftiles, lds, st)
                    : launch<kEpiBiasRelu, false>(q, (int)nblocks, band.nftiles, lds, st);
        else if (q.epi.bias)
            e = acc ? launch<kEpiBias, true>(q, (int)nblocks, band.nftiles, lds, st)
                    : launch<kEpiBias, false>(q, (int)nblocks, band.nftiles, lds, st);
        else
            e = acc ? launch<kEpiNone, true>(q, (int)nblocks, band.nftiles, lds, st)
                    : launch<kEpiNone, false>(q, (int)nblocks, band.nftiles, lds, st);
        if (e != hipSuccess) return fail_hip(e, "split conv launch");
    }
    *used = true;
    return SEERA_OK;
}

}  // namespace seera
