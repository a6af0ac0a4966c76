// igemm.h -- the generic fp16-MFMA tile kernel.
//
// A "problem" type P describes one (implicit) GEMM  C[M,N] = sum_k A(m,k) B(n,k):
//   P::template SA<ROWS, BK, NT>   stager type for the A tile (ROWS = BM)
//   P::template SB<ROWS, BK, NT>   stager type for the B tile (ROWS = BN)
//   p.init_a(sa, m0, tid)          once per block, before the K loop
//   p.init_b(sb, n0, tid)
//   p.load_a(sa, m0, k0, k1, tid)  fill the A stager for rows [m0, m0+BM)
//   p.load_b(sb, n0, k0, k1, tid)  fill the B stager for rows [n0, n0+BN)
//   p.store(m, n, z, v)            write one output element (m < M, n < N)
//   p.M, p.N, p.K, p.tiles_n, p.k_split, p.gm
// gridDim.x = tiles_m * tiles_n, gridDim.z = number of K splits.
//
// Pipeline (one barrier per BK slice, two LDS stages): the loads of slice t+1
// are issued from HBM into registers before the matrix cores start on slice t
// (held in LDS stage t&1); while the MFMAs of k-step kk run, the LDS fragments
// of k-step kk+1 are read; after the last MFMA of slice t the registers are
// rounded to fp16 and written to the other stage.
#pragma once

#include "mfma_core.h"

namespace seera {

template <int BM, int BN, int BK, int WM, int WN>
struct TileCfg {
    static constexpr int NT = WM * WN * 64;
    static constexpr int TM = BM / WM / 32;
    static constexpr int TN = BN / WN / 32;
    static constexpr int LDS_BYTES = 2 * (BM + BN) * BK * 2;
    static_assert(TM >= 1 && TN >= 1, "wave tile must hold one 32x32 MFMA tile");
    static_assert(BM % (WM * 32) == 0 && BN % (WN * 32) == 0, "tile/wave mismatch");
    static_assert(LDS_BYTES <= 160 * 1024, "LDS tile exceeds the 160 KB of a gfx950 CU");
};

template <int BM, int BN, int BK, int WM, int WN, class P>
__global__ __launch_bounds__(WM* WN * 64) void igemm_kernel(const P p) {
    using Cfg = TileCfg<BM, BN, BK, WM, WN>;
    constexpr int NT = Cfg::NT, TM = Cfg::TM, TN = Cfg::TN;
    extern __shared__ __attribute__((aligned(16))) half_t smem[];
    constexpr int STAGE = (BM + BN) * BK;  // halves per LDS stage (A then B)

    int tm, tn;
    tile_coords(blockIdx.x, gridDim.x, p.tiles_n, p.gm, tm, tn);
    const int m0 = tm * BM, n0 = tn * BN;
    const int kbeg = blockIdx.z * p.k_split;
    const int kend = min(p.K, kbeg + p.k_split);
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wm0 = (wave / WN) * (BM / WM), wn0 = (wave % WN) * (BN / WN);

    floatx16 acc[TM][TN];
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;

    typename P::template SA<BM, BK, NT> sa;
    typename P::template SB<BN, BK, NT> sb;
    const int nk = kend > kbeg ? (kend - kbeg + BK - 1) / BK : 0;
    if (nk > 0) {
        p.init_a(sa, m0, tid);
        p.init_b(sb, n0, tid);
        p.load_a(sa, m0, kbeg, kend, tid);
        p.load_b(sb, n0, kbeg, kend, tid);
        sa.store(smem, tid);
        sb.store(smem + BM * BK, tid);
        __syncthreads();
        for (int kt = 0; kt < nk; ++kt) {
            const int cur = kt & 1;
            const bool more = kt + 1 < nk;
            if (more) {
                const int k0 = kbeg + (kt + 1) * BK;
                p.load_a(sa, m0, k0, kend, tid);
                p.load_b(sb, n0, k0, kend, tid);
            }
            half_t* const now = smem + cur * STAGE;
            half_t* const next = smem + (cur ^ 1) * STAGE;
            mfma_slice<BK, TM, TN>(now, now + BM * BK, wm0, wn0, lane, acc);
            if (more) {
                sa.store(next, tid);
                sb.store(next + BM * BK, tid);
            }
            __syncthreads();
        }
    }

    const int z = blockIdx.z;
#pragma unroll
    for (int j = 0; j < TN; ++j) {
        const int n = n0 + wn0 + j * 32 + (lane & 31);
        if (n >= p.N) continue;
#pragma unroll
        for (int i = 0; i < TM; ++i)
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int m = m0 + wm0 + i * 32 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
                if (m < p.M) p.store(m, n, z, acc[i][j][r]);
            }
    }
}

// Host-side launch of igemm_kernel for problem `p` (p.tiles_n, p.k_split,
// p.gm must already be set; splits = number of K slices).
template <int BM, int BN, int BK, int WM, int WN, class P>
hipError_t launch_igemm(const P& p, int splits, hipStream_t stream) {
    using Cfg = TileCfg<BM, BN, BK, WM, WN>;
    const int tiles_m = (p.M + BM - 1) / BM;
    dim3 grid(tiles_m * p.tiles_n, 1, splits);
    auto kern = igemm_kernel<BM, BN, BK, WM, WN, P>;
    if (Cfg::LDS_BYTES > 65536) {
        hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(kern),
                                           hipFuncAttributeMaxDynamicSharedMemorySize,
                                           Cfg::LDS_BYTES);
        if (e != hipSuccess) return e;
    }
    hipLaunchKernelGGL(kern, grid, dim3(Cfg::NT), Cfg::LDS_BYTES, stream, p);
    return hipGetLastError();
}


// ---------------------------------------------------------------------------
// Warp-specialised variant for large tiles: CWM x CWN consumer waves run the
// MFMAs of K slice t from LDS stage t&1 while NPW producer waves round slice
// t+1 (loaded into their registers during slice t-1) to fp16 into stage
// (t+1)&1 and issue the global loads of slice t+2. One barrier per slice.
// With three waves per SIMD (two consumers, one producer) the fp32 loads and
// conversions overlap the matrix work instead of alternating with it.
// ---------------------------------------------------------------------------
template <int BM, int BN, int BK, int CWM, int CWN, int NPW>
struct WsCfg {
    static constexpr int NC = CWM * CWN * 64;    // consumer threads
    static constexpr int NP = NPW * 64;          // producer threads
    static constexpr int NT = NC + NP;
    static constexpr int TM = BM / CWM / 32;
    static constexpr int TN = BN / CWN / 32;
    static constexpr int LDS_BYTES = 2 * (BM + BN) * BK * 2;
    static_assert(TM >= 1 && TN >= 1, "wave tile must hold one 32x32 MFMA tile");
    static_assert(LDS_BYTES <= 160 * 1024, "LDS tile exceeds the 160 KB of a gfx950 CU");
};

template <int BM, int BN, int BK, int CWM, int CWN, int NPW, class P>
__global__ __launch_bounds__((CWM * CWN + NPW) * 64) void igemm_ws_kernel(const P p) {
    using Cfg = WsCfg<BM, BN, BK, CWM, CWN, NPW>;
    constexpr int TM = Cfg::TM, TN = Cfg::TN, NC = Cfg::NC, NP = Cfg::NP;
    extern __shared__ __attribute__((aligned(16))) half_t smem[];
    constexpr int STAGE = (BM + BN) * BK;

    int tm, tn;
    tile_coords(blockIdx.x, gridDim.x, p.tiles_n, p.gm, tm, tn);
    const int m0 = tm * BM, n0 = tn * BN;
    const int kbeg = blockIdx.z * p.k_split;
    const int kend = min(p.K, kbeg + p.k_split);
    const int nk = kend > kbeg ? (kend - kbeg + BK - 1) / BK : 0;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;

    if (tid < NC) {
        const int wm0 = (wave / CWN) * (BM / CWM), wn0 = (wave % CWN) * (BN / CWN);
        floatx16 acc[TM][TN];
#pragma unroll
        for (int i = 0; i < TM; ++i)
#pragma unroll
            for (int j = 0; j < TN; ++j)
#pragma unroll
                for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;
        for (int kt = 0; kt < nk; ++kt) {
            __syncthreads();  // slice kt is in stage kt&1
            const half_t* const now = smem + (kt & 1) * STAGE;
            mfma_slice<BK, TM, TN, false>(now, now + BM * BK, wm0, wn0, lane, acc);
        }
        const int z = blockIdx.z;
#pragma unroll
        for (int j = 0; j < TN; ++j) {
            const int n = n0 + wn0 + j * 32 + (lane & 31);
            if (n >= p.N) continue;
#pragma unroll
            for (int i = 0; i < TM; ++i)
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    const int m = m0 + wm0 + i * 32 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
                    if (m < p.M) p.store(m, n, z, acc[i][j][r]);
                }
        }
        return;
    }

    // Producer waves.
    if (nk == 0) return;
    const int ptid = tid - NC;
    typename P::template SA<BM, BK, NP> sa;
    typename P::template SB<BN, BK, NP> sb;
    p.init_a(sa, m0, ptid);
    p.init_b(sb, n0, ptid);
    p.load_a(sa, m0, kbeg, kend, ptid);
    p.load_b(sb, n0, kbeg, kend, ptid);
    sa.store(smem, ptid);
    sb.store(smem + BM * BK, ptid);
    if (nk > 1) {
        p.load_a(sa, m0, kbeg + BK, kend, ptid);
        p.load_b(sb, n0, kbeg + BK, kend, ptid);
    }
    __syncthreads();  // releases slice 0
    for (int kt = 0; kt + 1 < nk; ++kt) {
        half_t* const next = smem + ((kt + 1) & 1) * STAGE;
        sa.store(next, ptid);
        sb.store(next + BM * BK, ptid);
        if (kt + 2 < nk) {
            const int k0 = kbeg + (kt + 2) * BK;
            p.load_a(sa, m0, k0, kend, ptid);
            p.load_b(sb, n0, k0, kend, ptid);
        }
        __syncthreads();  // releases slice kt+1
    }
}

template <int BM, int BN, int BK, int CWM, int CWN, int NPW, class P>
hipError_t launch_igemm_ws(const P& p, int splits, hipStream_t stream) {
    using Cfg = WsCfg<BM, BN, BK, CWM, CWN, NPW>;
    const int tiles_m = (p.M + BM - 1) / BM;
    dim3 grid(tiles_m * p.tiles_n, 1, splits);
    auto kern = igemm_ws_kernel<BM, BN, BK, CWM, CWN, NPW, P>;
    if (Cfg::LDS_BYTES > 65536) {
        hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(kern),
                                           hipFuncAttributeMaxDynamicSharedMemorySize,
                                           Cfg::LDS_BYTES);
        if (e != hipSuccess) return e;
    }
    hipLaunchKernelGGL(kern, grid, dim3(Cfg::NT), Cfg::LDS_BYTES, stream, p);
    return hipGetLastError();
}

}  // namespace seera
