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
// A problem with `static constexpr bool kColSum = true` (the dB GEMM of a
// Dense layer with its bias gradient) also sums its B operand over K, per
// output column: its B stagers keep fp32 sums of the values they round into
// LDS (sb.colsum_begin(on), sb.cs[4] for the 4 columns SB::col0(tid) + q of
// a thread), the blocks of row tile 0 reduce them in a fixed order at the
// end (colsum_finish) and hand each column's sum of their K range to
// p.store_colsum(n, z, v). The pipelined kernel then loads zeros past the
// last slice instead of re-reading it, so that no slice is counted twice.
//
// Pipeline (one barrier per BK slice, two LDS stages): the loads of slice t+1
// are issued from HBM into registers before the matrix cores start on slice t
// (held in LDS stage t&1); while the MFMAs of k-step kk run, the LDS fragments
// of k-step kk+1 are read; after the last MFMA of slice t the registers are
// rounded to fp16 and written to the other stage.
#pragma once

#include <type_traits>

#include "mfma_core.h"

namespace seera {

template <class P, class = void>
struct has_colsum : std::false_type {};
template <class P>
struct has_colsum<P, std::void_t<decltype(P::kColSum)>> : std::bool_constant<P::kColSum> {};

// Problems that declare `static constexpr bool kStoreCol = true` take the 16
// accumulator rows of one output column at once (store_col): a fused
// epilogue can then read its per-column and per-element inputs before any
// output is written. Row r of the column is mrow + kAccRow[r], with mrow the
// lane's first row: each address is one per-lane base plus a wave-uniform
// row offset, so no per-row 64-bit offsets stay live beside the accumulators.
template <class P, class = void>
struct has_store_col : std::false_type {};
template <class P>
struct has_store_col<P, std::void_t<decltype(P::kStoreCol)>> : std::bool_constant<P::kStoreCol> {};

// Row of accumulator element r of a 32x32 MFMA tile, relative to the lane's
// first row mbase + 4*(lane/32).
__device__ __forceinline__ constexpr int acc_row(int r) { return 8 * (r >> 2) + (r & 3); }

// Writes accumulator tile column n of a wave: rows mbase + 8*(r/4) + 4*(lane/32)
// + r%4 of the 32x32 MFMA layout (rows >= M are skipped by the problem).
template <class P>
__device__ __forceinline__ void store_acc_col(const P& p, const floatx16& a, int mbase, int n, int z,
                                              int lane) {
    if constexpr (has_store_col<P>::value) {
        float v[16];
#pragma unroll
        for (int r = 0; r < 16; ++r) v[r] = a[r];
        p.store_col(n, z, mbase + 4 * (lane >> 5), v);
    } else {
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const int m = mbase + 4 * (lane >> 5) + acc_row(r);
            if (m < p.M) p.store(m, n, z, a[r]);
        }
    }
}

// End of a kColSum block of row tile 0 (every thread of the block calls it):
// holder threads (NH of them, each with the sums of columns col0 + q and a
// reduction slot in 0 .. NH/(ROWS/4) - 1 among the holders of that column
// group; slot -1: not a holder) put their sums in LDS, then the first ROWS
// threads add the slots in order.
template <int ROWS, int NH, class P>
__device__ __forceinline__ void colsum_finish(const P& p, const float (&cs)[4], int col0, int slot,
                                              int n0, int z, void* smem) {
    constexpr int CG = ROWS / 4, G = NH / CG;
    static_assert(NH % CG == 0, "each holder keeps one 4-column group");
    float* const red = reinterpret_cast<float*>(smem);
    __syncthreads();  // every LDS tile read is done
    if (slot >= 0) {
#pragma unroll
        for (int q = 0; q < 4; ++q) red[slot * ROWS + col0 + q] = cs[q];
    }
    __syncthreads();
    const int c = threadIdx.x;
    if (c < ROWS) {
        float t = 0.f;
        for (int g = 0; g < G; ++g) t += red[g * ROWS + c];
        p.store_colsum(n0 + c, z, t);
    }
}

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

    static_assert(!has_colsum<P>::value, "column sums run on the pipelined and warp-specialised kernels");
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
        for (int i = 0; i < TM; ++i) store_acc_col(p, acc[i][j], m0 + wm0 + i * 32, n, z, lane);
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
// Pipelined variant of igemm_kernel for problems with plain (branch-free)
// stagers: D register sets keep the loads of D K slices in flight instead of
// one. With one slice in flight every slice costs a full memory round trip
// (about 1.5 k cycles), which is what bounds the small tiles: a 64x64x32
// slice is 64 MFMA cycles. Slice s lives in set s % D; iteration kt runs the
// MFMAs of slice kt from LDS stage kt&1, rounds slice kt+1 from its set into
// the other stage and at once refills that set with slice kt+1+D. Loads past
// the last slice re-read it (never stored), so every iteration issues the
// same loads and the compiler's vmcnt waits stay exact.
// ---------------------------------------------------------------------------
// KG > 1 splits the block's K range over KG groups of WM x WN waves (each
// with its own LDS stages and register sets, contiguous parts of the range):
// more waves per CU keep more loads in flight for the small tiles, whose
// block count alone leaves one wave per SIMD. Group g > 0 hands its
// accumulators to group 0 through LDS at the end, added in group order.
template <int BM, int BN, int BK, int WM, int WN, int D, int KG>
struct PipeCfg {
    using Tile = TileCfg<BM, BN, BK, WM, WN>;
    static constexpr int NTG = Tile::NT;          // threads per group
    static constexpr int NT = NTG * KG;
    static constexpr int STAGE = (BM + BN) * BK;  // halves per LDS stage
    // groups 1 .. KG-1 hand over their accumulators at once, one slot each
    static constexpr int RED_BYTES = KG > 1 ? (KG - 1) * NTG * Tile::TM * Tile::TN * 16 * 4 : 0;
    static constexpr int LDS_BYTES =
        KG * Tile::LDS_BYTES > RED_BYTES ? KG * Tile::LDS_BYTES : RED_BYTES;
    static_assert(LDS_BYTES <= 160 * 1024, "LDS tile exceeds the 160 KB of a gfx950 CU");
};

// Body of igemm_pipe_kernel for block `bid` of `nblk` (split z) of problem p.
template <int BM, int BN, int BK, int WM, int WN, int D, int KG, class P>
__device__ __forceinline__ void pipe_body(const P& p, int bid, int nblk, int z_split,
                                          half_t* smem_all) {
    using Cfg = TileCfg<BM, BN, BK, WM, WN>;
    using PC = PipeCfg<BM, BN, BK, WM, WN, D, KG>;
    constexpr int NT = Cfg::NT, TM = Cfg::TM, TN = Cfg::TN;
    static_assert(D >= 2 && D % 2 == 0, "an even number of sets keeps the LDS stage of j fixed");
    constexpr int STAGE = PC::STAGE;

    int tm, tn;
    tile_coords(bid, nblk, p.tiles_n, p.gm, tm, tn);
    const int m0 = tm * BM, n0 = tn * BN;
    const int grp = KG > 1 ? __builtin_amdgcn_readfirstlane((int)threadIdx.x / NT) : 0;
    const int tid = (int)threadIdx.x - grp * NT, lane = tid & 63, wave = tid >> 6;
    half_t* const smem = smem_all + grp * 2 * STAGE;
    // this group's part of the block's K slices
    const int kb0 = z_split * p.k_split;
    const int kb1 = min(p.K, kb0 + p.k_split);
    const int nk_all = kb1 > kb0 ? (kb1 - kb0 + BK - 1) / BK : 0;
    const int per = (nk_all + KG - 1) / KG;
    const int kbeg = kb0 + grp * per * BK;
    const int kend = min(kb1, kbeg + per * BK);
    const int wm0 = (wave / WN) * (BM / WM), wn0 = (wave % WN) * (BN / WN);

    floatx16 acc[TM][TN];
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;

    const int nk = kend > kbeg ? (kend - kbeg + BK - 1) / BK : 0;
    // every group runs `per` iterations (the barriers are block-wide); a
    // group with fewer slices skips the MFMAs of the rest
    const int nit = KG > 1 ? per : nk;
    constexpr bool CS = has_colsum<P>::value;
    float csum[4] = {0.f, 0.f, 0.f, 0.f};
    if (nit > 0) {
        typename P::template SA<BM, BK, NT> sa[D];
        typename P::template SB<BN, BK, NT> sb[D];
        // (column sums: slices past the last load zeros, see the header; a
        // group without slices has kend <= kbeg: its loads all read 0)
        auto kof = [&](int s) { return kbeg + (CS ? s : min(s, max(nk - 1, 0))) * BK; };
#pragma unroll
        for (int d = 0; d < D; ++d) {
            p.init_a(sa[d], m0, tid);
            p.init_b(sb[d], n0, tid);
            if constexpr (CS) sb[d].colsum_begin(tm == 0);
        }
#pragma unroll
        for (int d = 0; d < D; ++d) {
            p.load_a(sa[d], m0, kof(d), kend, tid);
            p.load_b(sb[d], n0, kof(d), kend, tid);
        }
        sa[0].store(smem, tid);
        sb[0].store(smem + BM * BK, tid);
        p.load_a(sa[0], m0, kof(D), kend, tid);
        p.load_b(sb[0], n0, kof(D), kend, tid);
        __syncthreads();
        // Whole groups of D iterations, every store and load unconditional
        // (the MFMAs of iterations past the last slice are skipped): the loop
        // has one entry state, which keeps the waits exact across its back
        // edge.
        for (int kb = 0; kb < nit; kb += D) {
#pragma unroll
            for (int j = 0; j < D; ++j) {
                const int kt = kb + j;  // kb is a multiple of D (even): kt & 1 == j & 1
                const half_t* const now = smem + (j & 1) * STAGE;
                half_t* const next = smem + ((j + 1) & 1) * STAGE;
                if (kt < nk) mfma_slice<BK, TM, TN>(now, now + BM * BK, wm0, wn0, lane, acc);
                sa[(j + 1) % D].store(next, tid);
                sb[(j + 1) % D].store(next + BM * BK, tid);
                p.load_a(sa[(j + 1) % D], m0, kof(kt + 1 + D), kend, tid);
                p.load_b(sb[(j + 1) % D], n0, kof(kt + 1 + D), kend, tid);
                __syncthreads();
            }
        }
        // Drain the (unused) loads still in flight.
        __builtin_amdgcn_s_waitcnt(0);
        if constexpr (CS) {
#pragma unroll
            for (int d = 0; d < D; ++d)
#pragma unroll
                for (int q = 0; q < 4; ++q) csum[q] += sb[d].cs[q];
        }
    }
    if constexpr (CS) {
        // holders: every thread of every group (group g's slots follow g-1's)
        using SBT = typename P::template SB<BN, BK, NT>;
        constexpr int kSlots = NT / (BN / 4);
        if (tm == 0) {
            colsum_finish<BN, NT * KG>(p, csum, SBT::col0(tid), grp * kSlots + SBT::slot(tid), n0,
                                       z_split, smem_all);
            if constexpr (KG > 1) __syncthreads();  // the sums are read before LDS is reused
        }
    }
    if constexpr (KG > 1) {
        // groups 1.. write their accumulators into slots g-1 at once (the
        // stage reads of the last iteration ended at its barrier); group 0
        // adds them in group order
        float* const red = reinterpret_cast<float*>(smem_all);
        constexpr int kSlot = TM * TN * 16 * NT;
        if (grp != 0) {
            float* const mine = red + (grp - 1) * kSlot;
#pragma unroll
            for (int i = 0; i < TM; ++i)
#pragma unroll
                for (int j = 0; j < TN; ++j)
#pragma unroll
                    for (int r = 0; r < 16; ++r) mine[((i * TN + j) * 16 + r) * NT + tid] = acc[i][j][r];
        }
        __syncthreads();
        if (grp != 0) return;
#pragma unroll
        for (int g = 1; g < KG; ++g)
#pragma unroll
            for (int i = 0; i < TM; ++i)
#pragma unroll
                for (int j = 0; j < TN; ++j)
#pragma unroll
                    for (int r = 0; r < 16; ++r)
                        acc[i][j][r] += red[(g - 1) * kSlot + ((i * TN + j) * 16 + r) * NT + tid];
    }

    const int z = z_split;
#pragma unroll
    for (int j = 0; j < TN; ++j) {
        const int n = n0 + wn0 + j * 32 + (lane & 31);
        if (n >= p.N) continue;
#pragma unroll
        for (int i = 0; i < TM; ++i) store_acc_col(p, acc[i][j], m0 + wm0 + i * 32, n, z, lane);
    }
}

template <int BM, int BN, int BK, int WM, int WN, int D, int KG, class P>
__global__ __launch_bounds__(WM* WN * 64 * KG) void igemm_pipe_kernel(const P p) {
    extern __shared__ __attribute__((aligned(16))) half_t smem_all[];
    pipe_body<BM, BN, BK, WM, WN, D, KG>(p, blockIdx.x, gridDim.x, blockIdx.z, smem_all);
}

// Two problems of one tile shape in one launch (the dA and dB GEMMs of a
// layer's backward, which do not depend on each other): blocks [0, nb1) run
// p1's tiles, the rest p2's. Neither is split along K.
template <int BM, int BN, int BK, int WM, int WN, int D, int KG, class P1, class P2>
__global__ __launch_bounds__(WM* WN * 64 * KG) void igemm_pipe_pair_kernel(const P1 p1, const P2 p2,
                                                                          int nb1) {
    extern __shared__ __attribute__((aligned(16))) half_t smem_all[];
    if ((int)blockIdx.x < nb1)
        pipe_body<BM, BN, BK, WM, WN, D, KG>(p1, blockIdx.x, nb1, 0, smem_all);
    else
        pipe_body<BM, BN, BK, WM, WN, D, KG>(p2, (int)blockIdx.x - nb1, (int)gridDim.x - nb1, 0,
                                             smem_all);
}

template <int BM, int BN, int BK, int WM, int WN, int D, class P, int KG = 1>
hipError_t launch_igemm_pipe(const P& p, int splits, hipStream_t stream) {
    using PC = PipeCfg<BM, BN, BK, WM, WN, D, KG>;
    const int tiles_m = (p.M + BM - 1) / BM;
    dim3 grid(tiles_m * p.tiles_n, 1, splits);
    auto kern = igemm_pipe_kernel<BM, BN, BK, WM, WN, D, KG, P>;
    if (PC::LDS_BYTES > 65536) {
        hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(kern),
                                           hipFuncAttributeMaxDynamicSharedMemorySize,
                                           PC::LDS_BYTES);
        if (e != hipSuccess) return e;
    }
    hipLaunchKernelGGL(kern, grid, dim3(PC::NT), PC::LDS_BYTES, stream, p);
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

// Consumer side of the warp-specialised kernels: one barrier per slice, then
// the slice's MFMAs from LDS stage kt&1; finally the accumulators are stored.
template <int BM, int BN, int BK, int CWM, int CWN, class P>
__device__ __forceinline__ void ws_consume(const P& p, const half_t* smem, int m0, int n0, int nk,
                                           int wave, int lane) {
    constexpr int TM = BM / CWM / 32, TN = BN / CWN / 32;
    constexpr int STAGE = (BM + BN) * BK;
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
        for (int i = 0; i < TM; ++i) store_acc_col(p, acc[i][j], m0 + wm0 + i * 32, n, z, lane);
    }
}

template <int BM, int BN, int BK, int CWM, int CWN, int NPW, class P>
__global__ __launch_bounds__((CWM * CWN + NPW) * 64) void igemm_ws_kernel(const P p) {
    using Cfg = WsCfg<BM, BN, BK, CWM, CWN, NPW>;
    constexpr int NC = Cfg::NC, NP = Cfg::NP;
    extern __shared__ __attribute__((aligned(16))) half_t smem[];
    constexpr int STAGE = (BM + BN) * BK;

    int tm, tn;
    tile_coords(blockIdx.x, gridDim.x, p.tiles_n, p.gm, tm, tn);
    const int m0 = tm * BM, n0 = tn * BN;
    const int kbeg = blockIdx.z * p.k_split;
    const int kend = min(p.K, kbeg + p.k_split);
    const int nk = kend > kbeg ? (kend - kbeg + BK - 1) / BK : 0;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;

    constexpr bool CS = has_colsum<P>::value;
    if (tid < NC) {
        ws_consume<BM, BN, BK, CWM, CWN>(p, smem, m0, n0, nk, wave, lane);
        if constexpr (CS) {
            const float none[4] = {0.f, 0.f, 0.f, 0.f};
            if (tm == 0) colsum_finish<BN, NP>(p, none, 0, -1, n0, blockIdx.z, smem);
        }
        return;
    }

    // Producer waves.
    const int ptid = tid - NC;
    float csum[4] = {0.f, 0.f, 0.f, 0.f};
    if (nk > 0) {
    typename P::template SA<BM, BK, NP> sa;
    typename P::template SB<BN, BK, NP> sb;
    p.init_a(sa, m0, ptid);
    p.init_b(sb, n0, ptid);
    if constexpr (CS) sb.colsum_begin(tm == 0);
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
    if constexpr (CS) {
#pragma unroll
        for (int q = 0; q < 4; ++q) csum[q] = sb.cs[q];
    }
    }
    if constexpr (CS) {
        using SBT = typename P::template SB<BN, BK, NP>;
        if (tm == 0) colsum_finish<BN, NP>(p, csum, SBT::col0(ptid), SBT::slot(ptid), n0, blockIdx.z, smem);
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

// ---------------------------------------------------------------------------
// Warp-specialised kernel with streaming producers, for problems that supply
// streaming stagers (P::template WA / WB, p.ws_init_a / ws_init_b) and whose
// K range per split is a whole number of BK slices (checked by the host). Same
// consumers and the same LDS image as igemm_ws_kernel; the producers keep two
// K slices of loads in flight (register sets 0 and 1) and, part by part, round
// slice t+1 into LDS and at once reuse that part's registers for the loads of
// slice t+3. Loads past the last slice re-read it (never stored), so the load
// count per step is fixed and the compiler's vmcnt waits stay exact.
// ---------------------------------------------------------------------------
template <int BM, int BN, int BK, int CWM, int CWN, int NPW, class P>
__global__ __launch_bounds__((CWM * CWN + NPW) * 64) void igemm_ws2_kernel(const P p) {
    using Cfg = WsCfg<BM, BN, BK, CWM, CWN, NPW>;
    constexpr int NC = Cfg::NC, NP = Cfg::NP;
    extern __shared__ __attribute__((aligned(16))) half_t smem[];
    constexpr int STAGE = (BM + BN) * BK;

    int tm, tn;
    tile_coords(blockIdx.x, gridDim.x, p.tiles_n, p.gm, tm, tn);
    const int m0 = tm * BM, n0 = tn * BN;
    const int kbeg = blockIdx.z * p.k_split;
    const int kend = min(p.K, kbeg + p.k_split);
    const int nk = kend > kbeg ? (kend - kbeg + BK - 1) / BK : 0;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;

    constexpr bool CS = has_colsum<P>::value;
    if (tid < NC) {
        ws_consume<BM, BN, BK, CWM, CWN>(p, smem, m0, n0, nk, wave, lane);
        if constexpr (CS) {
            const float none[4] = {0.f, 0.f, 0.f, 0.f};
            if (tm == 0) colsum_finish<BN, NP>(p, none, 0, -1, n0, blockIdx.z, smem);
        }
        return;
    }

    const int ptid = tid - NC;
    float csum[4] = {0.f, 0.f, 0.f, 0.f};
    if (nk > 0) {
    using SA = typename P::template WA<BM, BK, NP>;
    using SB = typename P::template WB<BN, BK, NP>;
    SA sa;
    SB sb;
    p.ws_init_a(sa, m0, ptid);
    p.ws_init_b(sb, n0, ptid);
    if constexpr (CS) sb.colsum_begin(tm == 0);
    typename SA::Regs ra[2];
    typename SB::Regs rb[2];
    auto kof = [&](int s) { return kbeg + min(s, nk - 1) * BK; };

    // The sched barriers pin the issue order (A parts, then B parts, each
    // store followed by the loads that reuse its registers); the prologue
    // issues in the same order as the loop so that the waits stay exact.
#define SEERA_WS_FENCE() __builtin_amdgcn_sched_barrier(0)
#define SEERA_WS_LOADS(S, s)                                                   \
    do {                                                                       \
        const int k0_ = kof(s);                                                \
        const rsrc_t xa_ = sa.slice(k0_), xb_ = sb.slice(k0_);                 \
        _Pragma("unroll") for (int q = 0; q < SA::PARTS; ++q) {                \
            sa.load(ra[S], q, xa_);                                 \
            SEERA_WS_FENCE();                                                  \
        }                                                                      \
        _Pragma("unroll") for (int q = 0; q < SB::PARTS; ++q) {                \
            sb.load(rb[S], q, xb_);                                 \
            SEERA_WS_FENCE();                                                  \
        }                                                                      \
    } while (0)
    // Round slice s (register set S) into LDS stage s&1 and refill set S with
    // slice s+2.
#define SEERA_WS_STEP(S, s)                                                    \
    do {                                                                       \
        half_t* const st_ = smem + ((s) & 1) * STAGE;                          \
        const int k0_ = kof((s) + 2);                                          \
        const rsrc_t xa_ = sa.slice(k0_), xb_ = sb.slice(k0_);                 \
        _Pragma("unroll") for (int q = 0; q < SA::PARTS; ++q) {                \
            SEERA_WS_FENCE();                                                  \
            sa.store(ra[S], q, st_, ptid);                                     \
            SEERA_WS_FENCE();                                                  \
            sa.load(ra[S], q, xa_);                                 \
        }                                                                      \
        _Pragma("unroll") for (int q = 0; q < SB::PARTS; ++q) {                \
            SEERA_WS_FENCE();                                                  \
            sb.store(rb[S], q, st_ + BM * BK, ptid);                           \
            SEERA_WS_FENCE();                                                  \
            sb.load(rb[S], q, xb_);                                 \
        }                                                                      \
        SEERA_WS_FENCE();                                                      \
    } while (0)

    SEERA_WS_FENCE();
    SEERA_WS_LOADS(0, 0);
    SEERA_WS_LOADS(1, 1);
    SEERA_WS_STEP(0, 0);
    __syncthreads();  // releases slice 0
    int s = 1;
    for (; s + 1 < nk; s += 2) {
        SEERA_WS_STEP(1, s);
        __syncthreads();  // releases slice s
        SEERA_WS_STEP(0, s + 1);
        __syncthreads();  // releases slice s+1
    }
    if (s < nk) {
        SEERA_WS_STEP(1, s);
        __syncthreads();
    }
#undef SEERA_WS_STEP
#undef SEERA_WS_LOADS
#undef SEERA_WS_FENCE
    // Drain the (unused) loads still in flight before the wave ends.
    __builtin_amdgcn_s_waitcnt(0);
    if constexpr (CS) {
#pragma unroll
        for (int q = 0; q < 4; ++q) csum[q] = sb.cs[q];
    }
    }
    if constexpr (CS) {
        using SBT = typename P::template WB<BN, BK, NP>;
        if (tm == 0) colsum_finish<BN, NP>(p, csum, SBT::col0(ptid), SBT::slot(ptid), n0, blockIdx.z, smem);
    }
}

template <int BM, int BN, int BK, int CWM, int CWN, int NPW, class P>
hipError_t launch_igemm_ws2(const P& p, int splits, hipStream_t stream) {
    using Cfg = WsCfg<BM, BN, BK, CWM, CWN, NPW>;
    const int tiles_m = (p.M + BM - 1) / BM;
    dim3 grid(tiles_m * p.tiles_n, 1, splits);
    auto kern = igemm_ws2_kernel<BM, BN, BK, CWM, CWN, NPW, P>;
    if (Cfg::LDS_BYTES > 65536) {
        hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(kern),
                                           hipFuncAttributeMaxDynamicSharedMemorySize,
                                           Cfg::LDS_BYTES);
        if (e != hipSuccess) return e;
    }
    hipLaunchKernelGGL(kern, grid, dim3(Cfg::NT), Cfg::LDS_BYTES, stream, p);
    return hipGetLastError();
}

// igemm_ws2_kernel with one producer register set: slice s is rounded into
// LDS and the same registers at once take the loads of slice s + 1 (one slice
// of loads in flight), which leaves the registers for 64-deep slices (half as
// many barriers per K as 32-deep ones).
template <int BM, int BN, int BK, int CWM, int CWN, int NPW, class P>
__global__ __launch_bounds__((CWM * CWN + NPW) * 64) void igemm_ws1_kernel(const P p) {
    using Cfg = WsCfg<BM, BN, BK, CWM, CWN, NPW>;
    constexpr int NC = Cfg::NC, NP = Cfg::NP;
    extern __shared__ __attribute__((aligned(16))) half_t smem[];
    constexpr int STAGE = (BM + BN) * BK;

    int tm, tn;
    tile_coords(blockIdx.x, gridDim.x, p.tiles_n, p.gm, tm, tn);
    const int m0 = tm * BM, n0 = tn * BN;
    const int kbeg = blockIdx.z * p.k_split;
    const int kend = min(p.K, kbeg + p.k_split);
    const int nk = kend > kbeg ? (kend - kbeg + BK - 1) / BK : 0;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;

    constexpr bool CS = has_colsum<P>::value;
    if (tid < NC) {
        ws_consume<BM, BN, BK, CWM, CWN>(p, smem, m0, n0, nk, wave, lane);
        if constexpr (CS) {
            const float none[4] = {0.f, 0.f, 0.f, 0.f};
            if (tm == 0) colsum_finish<BN, NP>(p, none, 0, -1, n0, blockIdx.z, smem);
        }
        return;
    }

    const int ptid = tid - NC;
    float csum[4] = {0.f, 0.f, 0.f, 0.f};
    if (nk > 0) {
    using SA = typename P::template WA<BM, BK, NP>;
    using SB = typename P::template WB<BN, BK, NP>;
    SA sa;
    SB sb;
    p.ws_init_a(sa, m0, ptid);
    p.ws_init_b(sb, n0, ptid);
    if constexpr (CS) sb.colsum_begin(tm == 0);
    typename SA::Regs ra;
    typename SB::Regs rb;
    auto kof = [&](int s) { return kbeg + min(s, nk - 1) * BK; };
#define SEERA_WS_FENCE() __builtin_amdgcn_sched_barrier(0)
    {
        const int k0_ = kof(0);
        const rsrc_t xa_ = sa.slice(k0_), xb_ = sb.slice(k0_);
#pragma unroll
        for (int q = 0; q < SA::PARTS; ++q) {
            sa.load(ra, q, xa_);
            SEERA_WS_FENCE();
        }
#pragma unroll
        for (int q = 0; q < SB::PARTS; ++q) {
            sb.load(rb, q, xb_);
            SEERA_WS_FENCE();
        }
    }
    for (int s = 0; s < nk; ++s) {
        half_t* const st_ = smem + (s & 1) * STAGE;
        const int k0_ = kof(s + 1);
        const rsrc_t xa_ = sa.slice(k0_), xb_ = sb.slice(k0_);
#pragma unroll
        for (int q = 0; q < SA::PARTS; ++q) {
            SEERA_WS_FENCE();
            sa.store(ra, q, st_, ptid);
            SEERA_WS_FENCE();
            sa.load(ra, q, xa_);
        }
#pragma unroll
        for (int q = 0; q < SB::PARTS; ++q) {
            SEERA_WS_FENCE();
            sb.store(rb, q, st_ + BM * BK, ptid);
            SEERA_WS_FENCE();
            sb.load(rb, q, xb_);
        }
        SEERA_WS_FENCE();
        __syncthreads();  // releases slice s
    }
#undef SEERA_WS_FENCE
    __builtin_amdgcn_s_waitcnt(0);
    if constexpr (CS) {
#pragma unroll
        for (int q = 0; q < 4; ++q) csum[q] = sb.cs[q];
    }
    }
    if constexpr (CS) {
        using SBT = typename P::template WB<BN, BK, NP>;
        if (tm == 0) colsum_finish<BN, NP>(p, csum, SBT::col0(ptid), SBT::slot(ptid), n0, blockIdx.z, smem);
    }
}

template <int BM, int BN, int BK, int CWM, int CWN, int NPW, class P>
hipError_t launch_igemm_ws1(const P& p, int splits, hipStream_t stream) {
    using Cfg = WsCfg<BM, BN, BK, CWM, CWN, NPW>;
    const int tiles_m = (p.M + BM - 1) / BM;
    dim3 grid(tiles_m * p.tiles_n, 1, splits);
    auto kern = igemm_ws1_kernel<BM, BN, BK, CWM, CWN, NPW, P>;
    hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(kern),
                                       hipFuncAttributeMaxDynamicSharedMemorySize, Cfg::LDS_BYTES);
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL(kern, grid, dim3(Cfg::NT), Cfg::LDS_BYTES, stream, p);
    return hipGetLastError();
}

}  // namespace seera
