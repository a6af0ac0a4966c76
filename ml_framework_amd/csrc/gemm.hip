// gemm.hip -- GEMM forward / backward and transposes for gfx950.
//
// Reference: engine_cuda/src/GEMM.cu. The reference runs one 32-lane warp
// per 16x16 output tile and, for the backward, materialises B^T and A^T and
// loops over the batch on the host (GEMM.cu:164-225). Here:
//   forward  C = A.B        one GEMM with M' = Nbatch*M (A is contiguous
//                           [Nbatch*M, K] and B is shared), B read N-major
//   dA = dC.B^T             one GEMM, B^T read straight from B (K-major)
//   dB = sum_b A_b^T.dC_b   one GEMM with K' = Nbatch*M, A^T read straight
//                           from A; split-K with a deterministic reduce
// No transposed copies and no host loop.
#include <algorithm>

#include "kernels.h"
#include "plan.h"

namespace seera {
namespace {

// Strided fp32 matrix view with an element layout: K-contiguous (KC) means
// element (row, k) at ptr[row*ld + k]; otherwise at ptr[k*ld + row].
template <bool KC, int VEC>
struct Operand {
    template <int ROWS, int BK, int NT>
    using Stager = typename std::conditional<KC, StageKC<ROWS, BK, NT, VEC>,
                                             StageMNC<ROWS, BK, NT, VEC>>::type;
};

// B stagers that also sum, per column, the fp32 values they round into LDS
// (the bias gradient fused into the dB GEMM, db[n] = sum_k dC[k, n]). A
// thread's items all sit in one 4-column group of the tile (col0, its
// reduction slot among the threads of that group: slot), so it keeps 4 sums;
// values outside the tile or past K load as 0. Only the blocks of row tile 0
// count (colsum_begin(true)).
template <int ROWS, int BK, int NT, int VEC>
struct ColSumMNC : StageMNC<ROWS, BK, NT, VEC> {
    using Base = StageMNC<ROWS, BK, NT, VEC>;
    static_assert(NT % Base::CG == 0 && (!Base::kHalfWaveOrder || NT % (4 * Base::CG) == 0),
                  "each thread keeps one 4-column group");
    static __device__ __forceinline__ int col0(int tid) {
        int dr, dk;
        Base::item_pos(tid, dr, dk);
        return dr;
    }
    static __device__ __forceinline__ int slot(int tid) { return Base::item_slot(tid); }
    float cs[4];
    bool on;
    __device__ __forceinline__ void colsum_begin(bool count) {
        on = count;
#pragma unroll
        for (int q = 0; q < 4; ++q) cs[q] = 0.f;
    }
    __device__ __forceinline__ void store(half_t* tile, int tid) {
        if (on) {
#pragma unroll
            for (int p = 0; p < Base::PASSES; ++p)
#pragma unroll
                for (int j = 0; j < Base::KK; ++j)
#pragma unroll
                    for (int q = 0; q < 4; ++q) cs[q] += this->v[p][j][q];
        }
        Base::store(tile, tid);
    }
};

template <int ROWS, int BK, int NP>
struct ColSumWsMNC : WsStageMNC<ROWS, BK, NP> {
    using Base = WsStageMNC<ROWS, BK, NP>;
    static __device__ __forceinline__ int col0(int tid) { return (tid % Base::CG) * 4; }
    static __device__ __forceinline__ int slot(int tid) { return tid / Base::CG; }
    float cs[4];
    bool on;
    __device__ __forceinline__ void colsum_begin(bool count) {
        on = count;
#pragma unroll
        for (int q = 0; q < 4; ++q) cs[q] = 0.f;
    }
    __device__ __forceinline__ void store(const typename Base::Regs& r, int part, half_t* tile,
                                          int tid) {
        if (on) {
#pragma unroll
            for (int j = 0; j < 8; ++j)
#pragma unroll
                for (int q = 0; q < 4; ++q) cs[q] += r.v[part][j][q];
        }
        Base::store(r, part, tile, tid);
    }
};

// EPI: the fused forward epilogue (seera_hip_matmul_bias_act) applies
// C = act(A.B + bias[n]) as each element is stored, and for ReLU also writes
// mask = (pre-activation > 0); under split-K the partials are stored raw and
// splitk_reduce_epi applies it after the sum.
// COLSUM (B MN-contiguous only): also colsum[z * N + n] = sum over split z's K
// range of B(n, k), through the ColSum stagers and p.store_colsum.
template <bool A_KC, int VA, bool B_KC, int VB, bool EPI = false, bool COLSUM = false>
struct GemmProblem {
    static_assert(!COLSUM || !B_KC, "column sums are taken by the MN-contiguous B stagers");
    const float* A;
    const float* B;
    float* C;
    int M, N, K;
    int64_t lda, ldb, ldc;
    int64_t split_stride;  // distance between split-K partial outputs
    int tiles_n, k_split, gm;
    const float* bias;     // EPI: [N] or nullptr
    float* mask;           // EPI, act == kActRelu: [M, ldc] or nullptr
    int act;               // EPI: kActNone or kActRelu
    float* colsum;         // COLSUM: [splits][N]
    static constexpr bool kEpi = EPI;
    static constexpr bool kStoreCol = EPI;
    static constexpr bool kColSum = COLSUM;
    static constexpr bool kPipe = true;  // StageKC / StageMNC load without branches

    template <int R, int BK, int NT>
    using SA = typename Operand<A_KC, VA>::template Stager<R, BK, NT>;
    template <int R, int BK, int NT>
    using SB = typename std::conditional<COLSUM, ColSumMNC<R, BK, NT, VB>,
                                         typename Operand<B_KC, VB>::template Stager<R, BK, NT>>::type;

    template <class S>
    __device__ __forceinline__ void load_a(S& s, int m0, int k0, int k1, int tid) const {
        s.load(A, lda, m0, M, k0, k1, tid);
    }
    template <class S>
    __device__ __forceinline__ void load_b(S& s, int n0, int k0, int k1, int tid) const {
        s.load(B, ldb, n0, N, k0, k1, tid);
    }
    // Streaming stagers for the large warp-specialised tile (vector loads only).
    static constexpr bool kWsStream = VA == 4 && VB == 4;
    template <int R, int BK, int NP>
    using WA = typename std::conditional<A_KC, WsStageKC<R, BK, NP>, WsStageMNC<R, BK, NP>>::type;
    template <int R, int BK, int NP>
    using WB = typename std::conditional<
        COLSUM, ColSumWsMNC<R, BK, NP>,
        typename std::conditional<B_KC, WsStageKC<R, BK, NP>, WsStageMNC<R, BK, NP>>::type>::type;
    template <class S>
    __device__ __forceinline__ void ws_init_a(S& s, int m0, int tid) const {
        s.init(A, lda, m0, M, tid);
    }
    template <class S>
    __device__ __forceinline__ void ws_init_b(S& s, int n0, int tid) const {
        s.init(B, ldb, n0, N, tid);
    }

    template <class S>
    __device__ __forceinline__ void init_a(S&, int, int) const {}
    template <class S>
    __device__ __forceinline__ void init_b(S&, int, int) const {}
    __device__ __forceinline__ void store_colsum(int n, int z, float v) const {
        if (n < N) colsum[(int64_t)z * N + n] = v;
    }
    // One accumulator column (rows mrow + acc_row(r) of column n) under the
    // epilogue: the bias of the column is read once, and (ReLU backward)
    // every mask value before any output is written, so no load waits behind
    // a store it might alias. The arithmetic is store()'s.
    __device__ __forceinline__ void store_col(int n, int z, int mrow, const float (&v)[16]) const {
        const int rem = M - mrow;  // rows acc_row(r) < rem exist
        const int64_t base = (int64_t)mrow * ldc + n;
        if constexpr (EPI) {
            if (split_stride == 0) {
                if (act == kActReluGrad) {
                    const float* const mk0 = mask + base;
                    float* const c0 = C + base;
                    float mk[16];
#pragma unroll
                    for (int r = 0; r < 16; ++r)
                        mk[r] = acc_row(r) < rem ? mk0[acc_row(r) * ldc] : 0.f;
#pragma unroll
                    for (int r = 0; r < 16; ++r)
                        if (acc_row(r) < rem) c0[acc_row(r) * ldc] = v[r] * mk[r];
                    return;
                }
                const float b = bias ? bias[n] : 0.f;
                float* const c0 = C + base;
                float* const m0 = mask ? mask + base : nullptr;
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    if (acc_row(r) >= rem) continue;
                    const int64_t i = acc_row(r) * ldc;
                    epilogue(c0 + i, m0 ? m0 + i : nullptr, v[r], b, act);
                }
                return;
            }
        }
        float* const c0 = C + z * split_stride + base;
#pragma unroll
        for (int r = 0; r < 16; ++r)
            if (acc_row(r) < rem) c0[acc_row(r) * ldc] = v[r];
    }
    __device__ __forceinline__ void store(int m, int n, int z, float v) const {
        const int64_t i = z * split_stride + (int64_t)m * ldc + n;
        if constexpr (EPI) {
            if (split_stride == 0) {  // whole K in this block: finish the element here
                epilogue(C + i, mask ? mask + i : nullptr, v, bias ? bias[n] : 0.f, act);
                return;
            }
        }
        C[i] = v;
    }
};

__global__ void fill_zero_2d(float* __restrict__ C, int M, int N, int64_t ldc) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < (int64_t)M * N) C[(i / N) * ldc + i % N] = 0.f;
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

// out [rows_out, ld_out] = in [rows_in, cols_in] (leading dimension ld_in),
// zero past its rows and columns; ld_out % 4 == 0 (one float4 store per thread).
__global__ __launch_bounds__(256) void pad_2d(const float* __restrict__ in, int64_t ld_in,
                                              int rows_in, int cols_in, float* __restrict__ out,
                                              int rows_out, int ld_out) {
    const int nq = ld_out / 4;
    const int64_t n = (int64_t)rows_out * nq;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
         i += (int64_t)gridDim.x * blockDim.x) {
        const int64_t r = i / nq;
        const int c0 = (int)(i - r * nq) * 4;
        floatx4 v = {0.f, 0.f, 0.f, 0.f};
        if (r < rows_in) {
            const float* src = in + r * ld_in;
#pragma unroll
            for (int j = 0; j < 4; ++j)
                if (c0 + j < cols_in) v[j] = src[c0 + j];
        }
        *reinterpret_cast<floatx4*>(out + r * ld_out + c0) = v;
    }
}

// GEMMs of at least this many multiply-adds whose operands are not
// vector-aligned (or whose K is not a whole number of 32-deep slices) run on
// zero-padded copies of both operands: two copy passes cost less than the
// scalar loads (4095^3: 1.8 ms on scalar loads) or the non-streaming kernel.
constexpr double kPadMinMacs = 4294967296.0;

// Dispatch on operand vector-load eligibility. Only the 64x64 tile carries the
// scalar (any shape / alignment) variants.
// Optional fused forward epilogue of gemm_dispatch<..., true>.
struct Epi {
    const float* bias = nullptr;
    float* mask = nullptr;
    int act = kActNone;
};

template <bool A_KC, bool B_KC, bool EPI = false, bool COLSUM = false>
int gemm_dispatch(const float* A, int64_t lda, const float* B, int64_t ldb, float* C,
                  int64_t ldc, int M, int N, int K, hipStream_t st, Epi epi = Epi{},
                  float* colsum = nullptr, bool padded = false) {
    if (M == 0 || N == 0) return SEERA_OK;
    if (K == 0) {
        // Empty contraction: C = 0 (the reference's K loop never runs), then
        // the epilogue of a zero sum.
        const int64_t n = (int64_t)M * N;
        if constexpr (EPI) {
            hipLaunchKernelGGL(splitk_reduce_epi, dim3((unsigned)((n + 255) / 256)), dim3(256), 0,
                               st, (const float*)nullptr, C, M, N, ldc, 0, (int64_t)0, epi.bias,
                               epi.mask, epi.act);
        } else {
            hipLaunchKernelGGL(fill_zero_2d, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st,
                               C, M, N, ldc);
        }
        SEERA_HIP_TRY(hipGetLastError());
        return SEERA_OK;
    }
    // Tile loads address one tile through a buffer resource with 32-bit
    // offsets: the largest tile's span must stay below kMaxTileSpanBytes, else
    // only the 64x64 tile is used, and past that the shape is rejected.
    auto span = [](bool kc, int rows, int64_t ld) {
        return kc ? span_kc(rows, kMaxBK, ld) : span_mnc(rows, kMaxBK, ld);
    };
    const bool big_ok = span(A_KC, 256, lda) < kMaxTileSpanBytes &&
                        span(B_KC, 256, ldb) < kMaxTileSpanBytes;
    if (span(A_KC, 64, lda) >= kMaxTileSpanBytes || span(B_KC, 64, ldb) >= kMaxTileSpanBytes)
        return fail(SEERA_ERR_INVALID_ARGUMENT,
                    "GEMM leading dimension too large for 32-bit tile offsets (lda=%lld ldb=%lld)",
                    (long long)lda, (long long)ldb);
    // (padded: the staging copies below, whose rows run on in zeros or in
    // rows that are never stored up to a multiple of 4, so that every float4
    // load stays inside the copy)
    const bool va = padded || (aligned16(A) && lda % 4 == 0 && (A_KC ? K : M) % 4 == 0);
    const bool vb = padded || (aligned16(B) && ldb % 4 == 0 && (B_KC ? K : N) % 4 == 0);
    if (!padded && (!va || !vb || K % 32 != 0) && (double)M * N * K >= kPadMinMacs) {
        // Both operands into a staging copy: K-contiguous [rows][K32], or
        // MN-contiguous [K32][rows rounded up to 4], zeros past the data.
        // The zero k slices add nothing (and nothing to the column sums).
        const int K32 = (K + 31) & ~31, M4 = (M + 3) & ~3, N4 = (N + 3) & ~3;
        const int64_t na = A_KC ? (int64_t)M * K32 : (int64_t)K32 * M4;
        const int64_t nb = B_KC ? (int64_t)N * K32 : (int64_t)K32 * N4;
        const int64_t na_al = (na + 63) & ~(int64_t)63;
        void* ws = nullptr;
        bool got = false;
        SEERA_TRY(staging_workspace_try(sizeof(float) * (size_t)(na_al + nb), &ws, st, &got));
        if (got) {
            float* Ap = static_cast<float*>(ws);
            float* Bp = Ap + na_al;
            auto pad = [&](const float* in, int64_t ld_in, int rows_in, int cols_in, float* out,
                           int rows_out, int ld_out) {
                const int64_t q = (int64_t)rows_out * (ld_out / 4);
                const unsigned blocks = (unsigned)std::min<int64_t>((q + 255) / 256, 8192);
                hipLaunchKernelGGL(pad_2d, dim3(blocks), dim3(256), 0, st, in, ld_in, rows_in, cols_in,
                                   out, rows_out, ld_out);
            };
            if (A_KC) pad(A, lda, M, K, Ap, M, K32);
            else pad(A, lda, K, M, Ap, K32, M4);
            if (B_KC) pad(B, ldb, N, K, Bp, N, K32);
            else pad(B, ldb, K, N, Bp, K32, N4);
            SEERA_HIP_TRY(hipGetLastError());
            return gemm_dispatch<A_KC, B_KC, EPI, COLSUM>(Ap, A_KC ? K32 : M4, Bp, B_KC ? K32 : N4, C,
                                                          ldc, M, N, K32, st, epi, colsum, true);
        }
    }
    const Plan pl = plan_tiles(M, N, K, va && vb && big_ok, true, true);
    auto fill = [&](auto prob) {
        prob.A = A; prob.B = B; prob.C = C;
        prob.M = M; prob.N = N; prob.K = K;
        prob.lda = lda; prob.ldb = ldb; prob.ldc = ldc;
        prob.split_stride = 0;
        prob.bias = epi.bias; prob.mask = epi.mask; prob.act = epi.act;
        prob.colsum = colsum;
        return prob;
    };
    if (va && vb) return run_plan<true>(fill(GemmProblem<A_KC, 4, B_KC, 4, EPI, COLSUM>{}), pl, st);
    if (va) return run_plan<false>(fill(GemmProblem<A_KC, 4, B_KC, 1, EPI, COLSUM>{}), pl, st);
    if (vb) return run_plan<false>(fill(GemmProblem<A_KC, 1, B_KC, 4, EPI, COLSUM>{}), pl, st);
    return run_plan<false>(fill(GemmProblem<A_KC, 1, B_KC, 1, EPI, COLSUM>{}), pl, st);
}

// The dA and dB GEMMs of a backward (independent of each other) as one
// launch when both are small (run_plan_pair); any shape or alignment the
// paired kernel does not take runs as two gemm_dispatch calls.
struct GemmArgs {
    const float* A;
    int64_t lda;
    const float* B;
    int64_t ldb;
    float* C;
    int64_t ldc;
    int M, N, K;
};

template <bool A1_KC, bool B1_KC, bool EPI1, bool A2_KC, bool B2_KC, bool CS2>
int gemm_pair(const GemmArgs& g1, Epi e1, const GemmArgs& g2, float* colsum2, hipStream_t st) {
    auto vec = [](const GemmArgs& g, bool a_kc, bool b_kc) {
        return aligned16(g.A) && g.lda % 4 == 0 && (a_kc ? g.K : g.M) % 4 == 0 &&
               aligned16(g.B) && g.ldb % 4 == 0 && (b_kc ? g.K : g.N) % 4 == 0;
    };
    auto span_ok = [](const GemmArgs& g, bool a_kc, bool b_kc) {
        auto span = [](bool kc, int rows, int64_t ld) {
            return kc ? span_kc(rows, kMaxBK, ld) : span_mnc(rows, kMaxBK, ld);
        };
        return span(a_kc, 256, g.lda) < kMaxTileSpanBytes && span(b_kc, 256, g.ldb) < kMaxTileSpanBytes;
    };
    const bool shapes_ok = g1.M > 0 && g1.N > 0 && g1.K > 0 && g2.M > 0 && g2.N > 0 && g2.K > 0 &&
                           span_ok(g1, A1_KC, B1_KC) && span_ok(g2, A2_KC, B2_KC);
    const bool pairable = shapes_ok && vec(g1, A1_KC, B1_KC) && vec(g2, A2_KC, B2_KC);
    if (shapes_ok && !pairable) {
        // An edge that is not a multiple of 4 (the N = 10 head of an MLP):
        // both GEMMs on scalar loads in one launch, when both plans are
        // unsplit 32x32 or 64x64 tiles within one round of the CUs (a launch costs
        // ~4.5 us at these sizes, more than the scalar loads of a small
        // GEMM); otherwise each on its own best path below.
        Plan pl1, pl2;
        if (pair_plans(g1.M, g1.N, g1.K, g2.M, g2.N, g2.K, pl1, pl2)) {
            GemmProblem<A1_KC, 1, B1_KC, 1, EPI1> p1{};
            p1.A = g1.A; p1.B = g1.B; p1.C = g1.C;
            p1.M = g1.M; p1.N = g1.N; p1.K = g1.K;
            p1.lda = g1.lda; p1.ldb = g1.ldb; p1.ldc = g1.ldc;
            p1.bias = e1.bias; p1.mask = e1.mask; p1.act = e1.act;
            const bool va2 = aligned16(g2.A) && g2.lda % 4 == 0 && (A2_KC ? g2.K : g2.M) % 4 == 0;
            auto fill2 = [&](auto p2) {
                p2.A = g2.A; p2.B = g2.B; p2.C = g2.C;
                p2.M = g2.M; p2.N = g2.N; p2.K = g2.K;
                p2.lda = g2.lda; p2.ldb = g2.ldb; p2.ldc = g2.ldc;
                p2.colsum = colsum2;
                return p2;
            };
            // The dB GEMM's A (the layer input, transposed) is aligned even
            // when dC is not: vector loads there take the MLP cfg3 backward
            // GEMMs from 24.8 to 20.7 us.
            using P2V = GemmProblem<A2_KC, 4, B2_KC, 1, false, CS2>;
            using P2S = GemmProblem<A2_KC, 1, B2_KC, 1, false, CS2>;
            if (va2) return run_plan_pair<true, true>(p1, pl1, fill2(P2V{}), pl2, st);
            return run_plan_pair<true, true>(p1, pl1, fill2(P2S{}), pl2, st);
        }
    }
    if (pairable) {
        GemmProblem<A1_KC, 4, B1_KC, 4, EPI1> p1{};
        p1.A = g1.A; p1.B = g1.B; p1.C = g1.C;
        p1.M = g1.M; p1.N = g1.N; p1.K = g1.K;
        p1.lda = g1.lda; p1.ldb = g1.ldb; p1.ldc = g1.ldc;
        p1.bias = e1.bias; p1.mask = e1.mask; p1.act = e1.act;
        GemmProblem<A2_KC, 4, B2_KC, 4, false, CS2> p2{};
        p2.A = g2.A; p2.B = g2.B; p2.C = g2.C;
        p2.M = g2.M; p2.N = g2.N; p2.K = g2.K;
        p2.lda = g2.lda; p2.ldb = g2.ldb; p2.ldc = g2.ldc;
        p2.colsum = colsum2;
        Plan pl1, pl2;
        pair_plans(g1.M, g1.N, g1.K, g2.M, g2.N, g2.K, pl1, pl2);
        return run_plan_pair<true, true>(p1, pl1, p2, pl2, st);
    }
    SEERA_TRY((gemm_dispatch<A1_KC, B1_KC, EPI1>(g1.A, g1.lda, g1.B, g1.ldb, g1.C, g1.ldc, g1.M,
                                                 g1.N, g1.K, st, e1)));
    return gemm_dispatch<A2_KC, B2_KC, false, CS2>(g2.A, g2.lda, g2.B, g2.ldb, g2.C, g2.ldc, g2.M,
                                                   g2.N, g2.K, st, Epi{}, colsum2);
}

// LDS-tiled transposes of `batch` [rows, cols] slices; 64x64 tiles, coalesced
// reads and writes, +1 padding against bank conflicts. Column tiles are on
// blockIdx.x; row tiles and slices loop over blockIdx.y / blockIdx.z in steps
// of the grid, so any extent fits the 65535 limit of those grid dimensions.
__global__ __launch_bounds__(256) void transpose_tiles(const float* __restrict__ in,
                                                       float* __restrict__ out, int batch,
                                                       int rows, int cols) {
    __shared__ float t[64][65];
    const int64_t slice = (int64_t)rows * cols;
    const int nby = (rows + 63) / 64;
    const int c0 = blockIdx.x * 64;
    const int tx = threadIdx.x & 63, ty = threadIdx.x >> 6;
    for (int z = blockIdx.z; z < batch; z += gridDim.z) {
        const float* src = in + z * slice;
        float* dst = out + z * slice;
        for (int by = blockIdx.y; by < nby; by += gridDim.y) {
            const int r0 = by * 64;
            for (int i = ty; i < 64; i += 4) {
                const int r = r0 + i, c = c0 + tx;
                if (r < rows && c < cols) t[i][tx] = src[(int64_t)r * cols + c];
            }
            __syncthreads();
            for (int i = ty; i < 64; i += 4) {
                const int c = c0 + i, r = r0 + tx;
                if (c < cols && r < rows) dst[(int64_t)c * rows + r] = t[tx][i];
            }
            __syncthreads();  // the tile is rewritten by the next step
        }
    }
}

// The same with 16-byte accesses when rows and cols are multiples of 4 and
// both tensors 16-byte aligned: a thread reads 4 consecutive columns of one
// input row and writes 4 consecutive columns (input rows) of one output row.
__global__ __launch_bounds__(256) void transpose_tiles4(const float* __restrict__ in,
                                                        float* __restrict__ out, int batch,
                                                        int rows, int cols) {
    __shared__ float t[64][65];
    const int64_t slice = (int64_t)rows * cols;
    const int nby = (rows + 63) / 64;
    const int c0 = blockIdx.x * 64;
    const int q = threadIdx.x & 15, ty = threadIdx.x >> 4;  // quad column, row group
    for (int z = blockIdx.z; z < batch; z += gridDim.z) {
        const float* src = in + z * slice;
        float* dst = out + z * slice;
        for (int by = blockIdx.y; by < nby; by += gridDim.y) {
            const int r0 = by * 64;
            for (int i = ty; i < 64; i += 16) {
                const int r = r0 + i, c = c0 + 4 * q;
                if (r < rows && c < cols) {  // c < cols means all 4 (cols % 4 == 0)
                    const float4 v =
                        *reinterpret_cast<const float4*>(src + (int64_t)r * cols + c);
                    t[i][4 * q] = v.x;
                    t[i][4 * q + 1] = v.y;
                    t[i][4 * q + 2] = v.z;
                    t[i][4 * q + 3] = v.w;
                }
            }
            __syncthreads();
            for (int i = ty; i < 64; i += 16) {
                const int c = c0 + i, r = r0 + 4 * q;
                if (c < cols && r < rows)
                    *reinterpret_cast<float4*>(dst + (int64_t)c * rows + r) = make_float4(
                        t[4 * q][i], t[4 * q + 1][i], t[4 * q + 2][i], t[4 * q + 3][i]);
            }
            __syncthreads();
        }
    }
}

}  // namespace

int gemm_fwd(const float* A, const float* B, float* C, int M, int N, int K, int Nbatch,
             hipStream_t st) {
    const int64_t Mb = (int64_t)M * Nbatch;
    if (Mb > 0x7fffffff) return fail(SEERA_ERR_INVALID_ARGUMENT, "Nbatch*M exceeds int range");
    // A [Mb, K] row-major (K-contiguous), B [K, N] row-major (N-contiguous).
    return gemm_dispatch<true, false>(A, K, B, N, C, N, (int)Mb, N, K, st);
}

int gemm_fwd_bias_act(const float* A, const float* B, const float* bias, float* C, float* mask,
                      int M, int N, int K, int Nbatch, int act, hipStream_t st) {
    const int64_t Mb = (int64_t)M * Nbatch;
    if (Mb > 0x7fffffff) return fail(SEERA_ERR_INVALID_ARGUMENT, "Nbatch*M exceeds int range");
    Epi e;
    e.bias = bias;
    e.mask = mask;
    e.act = act;
    return gemm_dispatch<true, false, true>(A, K, B, N, C, N, (int)Mb, N, K, st, e);
}

int gemm_bwd_relu(const float* A, const float* B, const float* dC, const float* mask, float* dA,
                  float* dB, int M, int N, int K, int Nbatch, hipStream_t st) {
    const int64_t Mb = (int64_t)M * Nbatch;
    if (Mb > 0x7fffffff) return fail(SEERA_ERR_INVALID_ARGUMENT, "Nbatch*M exceeds int range");
    Epi e;
    e.mask = const_cast<float*>(mask);  // read, not written, under kActReluGrad
    e.act = kActReluGrad;
    return gemm_pair<true, true, true, false, false, false>(
        GemmArgs{dC, N, B, N, dA, K, (int)Mb, K, N}, e, GemmArgs{A, K, dC, N, dB, N, K, N, (int)Mb},
        nullptr, st);
}

// db[n] = sum over rows of dY[row, n]: fixed-order partial sums of the rows a
// thread group owns, added in group order (bit-reproducible run to run).
constexpr int kBgCols = 64, kBgGroups = 8;
__global__ __launch_bounds__(kBgCols * kBgGroups) void bias_grad_kernel(
    const float* __restrict__ dY, float* __restrict__ db, int rows, int N) {
    __shared__ float part[kBgGroups][kBgCols];
    const int col = threadIdx.x % kBgCols, grp = threadIdx.x / kBgCols;
    const int n = blockIdx.x * kBgCols + col;
    const int per = (rows + kBgGroups - 1) / kBgGroups;
    const int r0 = grp * per, r1 = min(rows, r0 + per);
    float s = 0.f;
    if (n < N)
        for (int r = r0; r < r1; ++r) s += dY[(int64_t)r * N + n];
    part[grp][col] = s;
    __syncthreads();
    if (grp != 0 || n >= N) return;
    float t = part[0][col];
#pragma unroll
    for (int g = 1; g < kBgGroups; ++g) t += part[g][col];
    db[n] = t;
}

int bias_grad(const float* dY, float* db, int rows, int N, hipStream_t st) {
    if (N == 0) return SEERA_OK;
    hipLaunchKernelGGL(bias_grad_kernel, dim3((unsigned)((N + kBgCols - 1) / kBgCols)),
                       dim3(kBgCols * kBgGroups), 0, st, dY, db, rows, N);
    SEERA_HIP_TRY(hipGetLastError());
    return SEERA_OK;
}

int gemm_bwd(const float* A, const float* B, const float* dC, float* dA, float* dB, int M,
             int N, int K, int Nbatch, hipStream_t st) {
    const int64_t Mb = (int64_t)M * Nbatch;
    if (Mb > 0x7fffffff) return fail(SEERA_ERR_INVALID_ARGUMENT, "Nbatch*M exceeds int range");
    // dA [Mb, K] = dC [Mb, N] . B^T : B^T element (k, n) = B[k*N + n] is
    // K-contiguous in the GEMM's contraction index n.
    // dB [K, N] = A^T [K, Mb] . dC [Mb, N]: A^T element (k, m) = A[m*K + k]
    // is M-contiguous in the output row index k.
    return gemm_pair<true, true, false, false, false, false>(
        GemmArgs{dC, N, B, N, dA, K, (int)Mb, K, N}, Epi{},
        GemmArgs{A, K, dC, N, dB, N, K, N, (int)Mb}, nullptr, st);
}

int gemm_bwd_bias(const float* A, const float* B, const float* dC, const float* mask, float* dA,
                  float* dB, float* db, int M, int N, int K, int Nbatch, hipStream_t st) {
    const int64_t Mb = (int64_t)M * Nbatch;
    if (Mb > 0x7fffffff) return fail(SEERA_ERR_INVALID_ARGUMENT, "Nbatch*M exceeds int range");
    // dB [K, N] = A^T . dC with db[n] = sum_m dC[m, n] taken from the same
    // loads of dC (the blocks of dB's first row tile count them); with no dB
    // rows, or no rows of dC, db is its own pass (a sum of nothing is 0).
    const GemmArgs ga{dC, N, B, N, dA, K, (int)Mb, K, N}, gb{A, K, dC, N, dB, N, K, N, (int)Mb};
    if (K > 0 && Mb > 0 && N > 0) {
        if (mask) {
            Epi e;
            e.mask = const_cast<float*>(mask);  // read, not written, under kActReluGrad
            e.act = kActReluGrad;
            return gemm_pair<true, true, true, false, false, true>(ga, e, gb, db, st);
        }
        return gemm_pair<true, true, false, false, false, true>(ga, Epi{}, gb, db, st);
    }
    if (mask) {
        Epi e;
        e.mask = const_cast<float*>(mask);
        e.act = kActReluGrad;
        SEERA_TRY((gemm_dispatch<true, true, true>(dC, N, B, N, dA, K, (int)Mb, K, N, st, e)));
    } else {
        SEERA_TRY((gemm_dispatch<true, true>(dC, N, B, N, dA, K, (int)Mb, K, N, st)));
    }
    SEERA_TRY((gemm_dispatch<false, false>(A, K, dC, N, dB, N, K, N, (int)Mb, st)));
    return bias_grad(dC, db, (int)Mb, N, st);
}

int transpose(const float* in, float* out, int batch, int rows, int cols, hipStream_t st) {
    if (batch == 0 || rows == 0 || cols == 0) return SEERA_OK;
    // Column tiles on x (ceil(cols / 64) < 2^26); row tiles and slices are
    // looped in the kernel beyond 65535 each.
    dim3 grid((cols + 63) / 64, std::min((rows + 63) / 64, 65535), std::min(batch, 65535));
    if (rows % 4 == 0 && cols % 4 == 0 && aligned16(in) && aligned16(out))
        hipLaunchKernelGGL(transpose_tiles4, grid, dim3(256), 0, st, in, out, batch, rows, cols);
    else
        hipLaunchKernelGGL(transpose_tiles, grid, dim3(256), 0, st, in, out, batch, rows, cols);
    SEERA_HIP_TRY(hipGetLastError());
    return SEERA_OK;
}

}  // namespace seera
