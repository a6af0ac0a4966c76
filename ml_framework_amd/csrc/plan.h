// plan.h -- tile-shape choice, split-K and launch for igemm problems.
#pragma once

#include <algorithm>
#include <type_traits>

#include "igemm.h"
#include "runtime.h"

namespace seera {

// Block-tile shapes (BM x BN x BK, wave grid):
//   L   256x256x64 (or x32), warp-specialised: 4x2 consumer waves of 64x128
//       run the MFMAs while 4 producer waves load and round the next K slice
//   W   64x256x32,  1x4 waves of 64x64  few rows (conv output channels)
//   M   128x128x64 (or x32), 2x2 waves of 64x64 (warp-specialised with 4 (or
//       2) producer waves when the operands take streaming stagers)
//   S   64x64x32,   2x2 waves of 32x32  small / odd shapes, scalar loads
//   T   32x32x32,   one wave per K group  GEMMs whose 32x32 tiles fit one round
//       of the CUs (half the operand bytes per CU of a 64x64 tile)
enum class Tile { L, W, M, S, T };

struct Plan {
    Tile tile;
    int splits;
    int k_split;
    int groups = 1;  // wave groups over the K range of a 64x64 (1, 2) or 32x32 (1 .. 8) block
};

constexpr int kNumCUs = 256;
constexpr int kBK = 32;      // split-K slice granularity (slice ends are predicated, so it need
                             // not be a multiple of the tile BK; it is a multiple of 4 floats)
constexpr int kMaxBK = 32;   // deepest K slice of any tile (tile span checks)
constexpr int kPipeDepth = 2;  // K slices of loads in flight in igemm_pipe_kernel (4 measured no faster)
// K per block from which a 64x64 tile runs two groups of 4 waves over the
// halves of its K range (1024^3: 13.2 -> 11.1 us; four groups: 12.4 us). From
// 512 rather than 1024: 768^3 forward 10.3 -> 8.5 us (backward 19.3 -> 17.0),
// 896^3 11.7 -> 9.5, 1000^3 13.4 -> 12.1 (its backward 25.6 -> 26.3, the one
// case measured slower); the MLP's GEMMs, on 32x32 tiles, do not take it.
constexpr int kGroupSplitK = 512;
// Largest split-K count that 64x64 tiles replace by two wave groups in the
// block (no partials, no reduce launch): MLP cfg3 step 67.6 -> 58.5 us;
// replacing up to 8 splits: 59.3 us. Two groups, not one per split: four
// groups (1024 threads per block) ran 3-12 % slower on every shape measured
// (512x784x640 forward 9.9 against 8.8 us, 640x2048x640 17.2 against 15.8).
constexpr int kMaxGroupSplits = 4;

inline int tile_bm(Tile t) { return t == Tile::L ? 256 : t == Tile::M ? 128 : t == Tile::T ? 32 : 64; }
inline int tile_bn(Tile t) {
    return t == Tile::L || t == Tile::W ? 256 : t == Tile::M ? 128 : t == Tile::T ? 32 : 64;
}

// The cost of a split-K reduce launch in operand floats per CU (the bytes a
// CU streams in the time of a dependent small launch, about 4.5 us), against
// which a 32x32 plan's unsplit K range is weighed.
constexpr double kSplitReduceFloats = 100000.0;

inline int64_t tile_count(Tile t, int M, int N) {
    return (int64_t)((M + tile_bm(t) - 1) / tile_bm(t)) * ((N + tile_bn(t) - 1) / tile_bn(t));
}

// Padded work per CU (rounds of a full chip x tile area), weighted by how
// efficiently each tile shape feeds the matrix cores; lowest wins. The 64x256
// tile weighs a little more than 128x128: per K slice it stages 320 operand
// rows against 256, and on equal padded work (2048^3) 128x128 ran 13% faster.
inline Plan plan_tiles(int M, int N, int K, bool big_tiles, bool allow_split,
                       bool allow_groups = false, bool allow_t = true) {
    Tile cands[4] = {Tile::L, Tile::W, Tile::M, Tile::S};
    const double eff[4] = {1.0, 1.25, 1.2, 1.6};
    Plan best{Tile::S, 1, std::max(K, 1)};
    double best_cost = 1e300;
    for (int i = 0; i < 4; ++i) {
        const Tile t = cands[i];
        if (!big_tiles && t != Tile::S) continue;
        const int64_t tiles = tile_count(t, M, N);
        const double rounds = (double)((tiles + kNumCUs - 1) / kNumCUs);
        const double cost = rounds * tile_bm(t) * tile_bn(t) * eff[i];
        if (cost < best_cost) {
            best_cost = cost;
            best.tile = t;
        }
    }
    const int64_t tiles = tile_count(best.tile, M, N);
    if (allow_split && tiles < kNumCUs / 2 && K >= 8 * kBK) {
        int want = (int)std::min<int64_t>((kNumCUs + tiles - 1) / tiles, K / (4 * kBK));
        want = std::max(want, 1);
        int ks = (K + want - 1) / want;
        ks = (ks + kBK - 1) / kBK * kBK;
        best.splits = (K + ks - 1) / ks;
        best.k_split = ks;
    }
    if (allow_groups && allow_t && best.tile == Tile::S && tile_count(Tile::T, M, N) <= kNumCUs) {
        // A small GEMM is bound by the operand bytes each CU streams (and
        // their latency): 32x32 tiles in one round of the CUs halve them
        // against 64x64 ones, with the K range unsplit (no reduce launch);
        // wave groups over K keep several slices in flight.
        const double cost_s = 128.0 * (best.splits > 1 ? best.k_split : K) +
                              (best.splits > 1 ? kSplitReduceFloats : 0.0);
        if (64.0 * K < cost_s) {
            Plan t{Tile::T, 1, std::max(K, 1)};
            const int slices = (K + kBK - 1) / kBK;
            t.groups = slices >= 32 ? 8 : slices >= 16 ? 4 : slices >= 8 ? 2 : 1;
            return t;
        }
    }
    if (allow_groups && best.tile == Tile::S) {
        if (best.splits > 1 && best.splits <= kMaxGroupSplits) {
            best.groups = 2;
            best.splits = 1;
            best.k_split = std::max(K, 1);
        } else if (best.splits == 1 && K >= kGroupSplitK) {
            best.groups = 2;
        }
    }
    return best;
}

// Deterministic split-K reduction: C[m, n] = sum_z P[z][m][n] in z order;
// blocks from nb_c on add the column sums of a kColSum problem instead,
// out[n] = sum_z cs[z*N + n] (same launch).
// sum_z P[z * stride + i] in z order, 16 loads in flight (a loop of single
// loads waits a memory round trip per split: 58 us for 256 splits of 64x64).
__device__ __forceinline__ float split_sum(const float* __restrict__ P, int64_t stride, int splits,
                                           int64_t i) {
    constexpr int kU = 16;
    float s = 0.f;
    int z = 0;
    for (; z + kU <= splits; z += kU) {
        float v[kU];
#pragma unroll
        for (int u = 0; u < kU; ++u) v[u] = P[(z + u) * stride + i];
#pragma unroll
        for (int u = 0; u < kU; ++u) s += v[u];
    }
    for (; z < splits; ++z) s += P[z * stride + i];
    return s;
}

static __global__ void splitk_reduce(const float* __restrict__ P, float* __restrict__ C,
                                     int M, int N, int64_t ldc, int splits, int64_t stride,
                                     int nb_c, const float* __restrict__ cs,
                                     float* __restrict__ cs_out) {
    if ((int)blockIdx.x >= nb_c) {
        const int n = ((int)blockIdx.x - nb_c) * blockDim.x + threadIdx.x;
        if (n >= N) return;
        cs_out[n] = split_sum(cs, N, splits, n);
        return;
    }
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= (int64_t)M * N) return;
    C[(i / N) * ldc + i % N] = split_sum(P, stride, splits, i);
}

// Problems that declare `static constexpr bool kWsStream = true` supply
// streaming stagers and run the large tile on igemm_ws2_kernel.
template <class P, class = void>
struct ws_stream : std::false_type {};
template <class P>
struct ws_stream<P, std::void_t<decltype(P::kWsStream)>> : std::bool_constant<P::kWsStream> {};

// The same sum, then the fused forward epilogue (bias, activation, mask).
static __global__ void splitk_reduce_epi(const float* __restrict__ P, float* __restrict__ C,
                                         int M, int N, int64_t ldc, int splits, int64_t stride,
                                         const float* __restrict__ bias, float* __restrict__ mask,
                                         int act) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= (int64_t)M * N) return;
    const float s = split_sum(P, stride, splits, i);
    const int n = (int)(i % N);
    const int64_t o = (i / N) * ldc + n;
    epilogue(C + o, mask ? mask + o : nullptr, s, bias ? bias[n] : 0.f, act);
}

// Problems with a fused epilogue declare `static constexpr bool kEpi = true`.
template <class P, class = void>
struct has_epi : std::false_type {};
template <class P>
struct has_epi<P, std::void_t<decltype(P::kEpi)>> : std::bool_constant<P::kEpi> {};

// Problems whose stagers load without branches (a fixed load count per
// slice) declare `static constexpr bool kPipe = true` and run the smaller
// tiles on igemm_pipe_kernel (several K slices of loads in flight).
template <class P, class = void>
struct pipe_ok : std::false_type {};
template <class P>
struct pipe_ok<P, std::void_t<decltype(P::kPipe)>> : std::bool_constant<P::kPipe> {};

template <bool BIG, class P>
hipError_t launch_tile(const P& p, Tile t, int splits, int groups, hipStream_t st) {
    if (t == Tile::T && !pipe_ok<P>::value) return hipErrorInvalidValue;  // planned for pipe problems only
    if constexpr (ws_stream<P>::value) {
        // The 128x128 tile with warp-specialised producers: four producer
        // waves with one 64-deep slice in flight (2048^3 in 31 us) when K and
        // the splits are whole 64-deep slices, else two producer waves with
        // two 32-deep slices in flight (33 us; 44 us on the pipelined kernel
        // below). The 64x64 and 64x256 tiles gain nothing or spill with a
        // single producer wave, and keep the pipelined kernel.
        if (t == Tile::M && p.K % 64 == 0 && p.k_split % 64 == 0)
            return launch_igemm_ws1<128, 128, 64, 2, 2, 4>(p, splits, st);
        if (t == Tile::M && p.K % 32 == 0)
            return launch_igemm_ws2<128, 128, 32, 2, 2, 2>(p, splits, st);
    }
    if constexpr (pipe_ok<P>::value) {
        switch (t) {
            case Tile::W: return launch_igemm_pipe<64, 256, 32, 1, 4, kPipeDepth>(p, splits, st);
            case Tile::M: return launch_igemm_pipe<128, 128, 32, 2, 2, kPipeDepth>(p, splits, st);
            case Tile::S:
                // two groups of 4 waves over the halves of the block's K range
                if (groups >= 2) return launch_igemm_pipe<64, 64, 32, 2, 2, kPipeDepth, P, 2>(p, splits, st);
                return launch_igemm_pipe<64, 64, 32, 2, 2, kPipeDepth>(p, splits, st);
            case Tile::T:
                if (groups >= 8) return launch_igemm_pipe<32, 32, 32, 1, 1, kPipeDepth, P, 8>(p, splits, st);
                if (groups >= 4) return launch_igemm_pipe<32, 32, 32, 1, 1, kPipeDepth, P, 4>(p, splits, st);
                if (groups == 2) return launch_igemm_pipe<32, 32, 32, 1, 1, kPipeDepth, P, 2>(p, splits, st);
                return launch_igemm_pipe<32, 32, 32, 1, 1, kPipeDepth>(p, splits, st);
            default: break;
        }
    }
    if constexpr (BIG) {
        switch (t) {
            case Tile::L:
                if constexpr (ws_stream<P>::value) {
                    // Split sizes are multiples of kBK, so K % 32 == 0 makes
                    // every 32-deep slice of every split whole; 64-deep
                    // slices (half the barriers per K) need K and the split
                    // size to be multiples of 64.
                    static_assert(kBK % 32 == 0, "split-K granularity must be whole slices");
                    if (p.K % 64 == 0 && p.k_split % 64 == 0)
                        return launch_igemm_ws1<256, 256, 64, 4, 2, 4>(p, splits, st);
                    if (p.K % 32 == 0) return launch_igemm_ws2<256, 256, 32, 4, 2, 4>(p, splits, st);
                }
                return launch_igemm_ws<256, 256, 32, 4, 2, 4>(p, splits, st);
            case Tile::W:
                if constexpr (!pipe_ok<P>::value) return launch_igemm<64, 256, 32, 1, 4>(p, splits, st);
                break;
            case Tile::M:
                if constexpr (!pipe_ok<P>::value) return launch_igemm<128, 128, 32, 2, 2>(p, splits, st);
                break;
            default: break;
        }
    }
    // (problems with pipelined stagers never get here: their W, M and S tiles
    // returned above)
    if constexpr (pipe_ok<P>::value)
        return launch_igemm_pipe<64, 64, 32, 2, 2, kPipeDepth>(p, splits, st);
    else
        return launch_igemm<64, 64, 32, 2, 2>(p, splits, st);
}

// Runs problem `p` under plan `pl`. Problems that support split-K expose
// `C`, `ldc` and `split_stride` and a row-major store; `splittable` says so.
template <bool BIG, class P>
int run_plan(P p, const Plan& pl, hipStream_t st) {
    static_assert(!(has_epi<P>::value && has_colsum<P>::value),
                  "the split-K reduce with an epilogue carries no column sums");
    p.tiles_n = (p.N + tile_bn(pl.tile) - 1) / tile_bn(pl.tile);
    p.k_split = pl.splits > 1 ? pl.k_split : std::max(p.K, 1);
    p.gm = 4;
    // The 256x256 tile runs one block per CU: past one round of the CUs its
    // tiles go region by region (tile_coords).
    if (pl.tile == Tile::L && pl.splits == 1 && p.M % (16 * 256) == 0 && p.N % (16 * 256) == 0 &&
        tile_count(pl.tile, p.M, p.N) > kNumCUs)
        p.gm = kGmRegions;
    if (tile_count(pl.tile, p.M, p.N) > kMaxGridX)
        return fail(SEERA_ERR_INVALID_ARGUMENT, "grid too large (%d x %d)", p.M, p.N);
    float* final_c = p.C;
    const int64_t final_ld = p.ldc;
    float* final_cs = nullptr;
    if constexpr (has_colsum<P>::value) final_cs = p.colsum;
    if (pl.splits > 1) {
        // split-K partials of C, then (column sums) one row of N per split
        const size_t cn = (size_t)pl.splits * p.M * p.N;
        const size_t csn = has_colsum<P>::value ? (size_t)pl.splits * p.N : 0;
        void* ws = nullptr;
        SEERA_TRY(workspace(sizeof(float) * (cn + csn), &ws, st));
        p.C = static_cast<float*>(ws);
        p.ldc = p.N;
        p.split_stride = (int64_t)p.M * p.N;
        if constexpr (has_colsum<P>::value) p.colsum = p.C + cn;
    }
    hipError_t e = launch_tile<BIG>(p, pl.tile, pl.splits, pl.groups, st);
    if (e != hipSuccess) return fail_hip(e, "igemm launch");
    if (pl.splits > 1) {
        const int64_t n = (int64_t)p.M * p.N;
        if constexpr (has_epi<P>::value) {
            hipLaunchKernelGGL(splitk_reduce_epi, dim3((unsigned)((n + 255) / 256)), dim3(256), 0,
                               st, p.C, final_c, p.M, p.N, final_ld, pl.splits, p.split_stride,
                               p.bias, p.mask, p.act);
        } else {
            const int nb_c = (int)((n + 255) / 256);
            const float* cs = nullptr;
            int nb_cs = 0;
            if constexpr (has_colsum<P>::value) {
                cs = p.colsum;
                nb_cs = (p.N + 255) / 256;
            }
            hipLaunchKernelGGL(splitk_reduce, dim3((unsigned)(nb_c + nb_cs)), dim3(256), 0, st,
                               p.C, final_c, p.M, p.N, final_ld, pl.splits, p.split_stride, nb_c,
                               cs, final_cs);
        }
        SEERA_HIP_TRY(hipGetLastError());
    }
    return SEERA_OK;
}

template <int BM, int KG, class P1, class P2>
hipError_t launch_igemm_pipe_pair(const P1& p1, int nb1, const P2& p2, int nb2, hipStream_t st) {
    constexpr int WG = BM / 32;  // 2x2 waves of 32x32 on 64x64 tiles, one wave on 32x32
    using PC = PipeCfg<BM, BM, 32, WG, WG, kPipeDepth, KG>;
    auto kern = igemm_pipe_pair_kernel<BM, BM, 32, WG, WG, kPipeDepth, KG, P1, P2>;
    static_assert(PC::LDS_BYTES <= 65536, "the pair kernel's LDS fits the default limit");
    hipLaunchKernelGGL(kern, dim3((unsigned)(nb1 + nb2)), dim3(PC::NT), PC::LDS_BYTES, st, p1, p2,
                       nb1);
    return hipGetLastError();
}

// Both plans of a pair on one small tile (32x32 or 64x64), unsplit, together
// within one round of the CUs: the pair runs as one launch.
inline bool pair_fits(const Plan& pl1, int M1, int N1, const Plan& pl2, int M2, int N2) {
    return pl1.tile == pl2.tile && (pl1.tile == Tile::S || pl1.tile == Tile::T) && pl1.splits == 1 &&
           pl2.splits == 1 && tile_count(pl1.tile, M1, N1) + tile_count(pl2.tile, M2, N2) <= kNumCUs;
}

// Plans of two independent GEMMs (a backward's dA and dB). When their best
// plans do not pair and one of them is a 32x32 plan, both retry on 64x64
// tiles (one launch costs less than the smaller tile saves); returns whether
// the plans pair, and leaves each GEMM's own best plan when they do not.
inline bool pair_plans(int M1, int N1, int K1, int M2, int N2, int K2, Plan& pl1, Plan& pl2) {
    pl1 = plan_tiles(M1, N1, K1, true, true, true);
    pl2 = plan_tiles(M2, N2, K2, true, true, true);
    if (pair_fits(pl1, M1, N1, pl2, M2, N2)) return true;
    if (pl1.tile != Tile::T && pl2.tile != Tile::T) return false;
    const Plan q1 = plan_tiles(M1, N1, K1, true, true, true, false);
    const Plan q2 = plan_tiles(M2, N2, K2, true, true, true, false);
    if (!pair_fits(q1, M1, N1, q2, M2, N2)) return false;
    pl1 = q1;
    pl2 = q2;
    return true;
}

// Runs two independent problems: in one launch when pair_fits (the
// wave-group count of the two plans, the larger one, serves both), else one
// after the other.
template <bool BIG1, bool BIG2, class P1, class P2>
int run_plan_pair(P1 p1, const Plan& pl1, P2 p2, const Plan& pl2, hipStream_t st) {
    if constexpr (pipe_ok<P1>::value && pipe_ok<P2>::value) {
        if (pair_fits(pl1, p1.M, p1.N, pl2, p2.M, p2.N)) {
            const Tile t = pl1.tile;
            const int bm = tile_bm(t);
            const int64_t nb1 = tile_count(t, p1.M, p1.N), nb2 = tile_count(t, p2.M, p2.N);
            p1.tiles_n = (p1.N + bm - 1) / bm;
            p2.tiles_n = (p2.N + bm - 1) / bm;
            p1.k_split = std::max(p1.K, 1);
            p2.k_split = std::max(p2.K, 1);
            p1.gm = p2.gm = 4;
            const int g = std::max(pl1.groups, pl2.groups);
            hipError_t e;
            if (t == Tile::T)
                e = g >= 8   ? launch_igemm_pipe_pair<32, 8>(p1, (int)nb1, p2, (int)nb2, st)
                    : g >= 4 ? launch_igemm_pipe_pair<32, 4>(p1, (int)nb1, p2, (int)nb2, st)
                    : g == 2 ? launch_igemm_pipe_pair<32, 2>(p1, (int)nb1, p2, (int)nb2, st)
                             : launch_igemm_pipe_pair<32, 1>(p1, (int)nb1, p2, (int)nb2, st);
            else
                // 64x64 plans take at most two groups (plan_tiles): with
                // four, a pair ran 256x784x512 backward in 7.6 against 6.9 us
                // and 384x640x384 in 7.8 against 6.4.
                e = g >= 2 ? launch_igemm_pipe_pair<64, 2>(p1, (int)nb1, p2, (int)nb2, st)
                           : launch_igemm_pipe_pair<64, 1>(p1, (int)nb1, p2, (int)nb2, st);
            if (e != hipSuccess) return fail_hip(e, "igemm pair launch");
            return SEERA_OK;
        }
    }
    SEERA_TRY(run_plan<BIG1>(p1, pl1, st));
    return run_plan<BIG2>(p2, pl2, st);
}

}  // namespace seera
