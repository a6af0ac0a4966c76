// gather.h -- stagers whose elements come from an index map (implicit GEMM).
//
// A gather functor G provides
//   G::Row  row_info(int row)            per-row data, computed once per block
//   G::Kin  k_info(int k, int kmax)      per-k data, computed once per slice
//   float   fetch(const Row&, const Kin&)  element value or 0 outside the
//                                          tensor / the padding
#pragma once

#include "mfma_core.h"

namespace seera {

// Each thread owns 4 consecutive rows x 8 consecutive k (consecutive threads
// take consecutive row groups): used when the rows are the contiguous memory
// direction (output pixels of an NCHW tensor).
template <int ROWS, int BK, int NT, class G>
struct StageGatherMN {
    static constexpr int CG = ROWS / 4;
    static constexpr int KG = BK / 8;
    static constexpr int ITEMS = CG * KG;
    static constexpr int PASSES = (ITEMS + NT - 1) / NT;
    float v[PASSES][8][4];
    typename G::Row ri[PASSES][4];

    __device__ __forceinline__ void init(const G& g, int r0, int tid) {
#pragma unroll
        for (int p = 0; p < PASSES; ++p) {
            const int item = p * NT + tid;
#pragma unroll
            for (int q = 0; q < 4; ++q) ri[p][q] = g.row_info(r0 + (item % CG) * 4 + q);
        }
    }

    __device__ __forceinline__ void load(const G& g, int k0, int kmax, int tid) {
#pragma unroll
        for (int p = 0; p < PASSES; ++p) {
            const int item = p * NT + tid;
            const bool live = ITEMS % NT == 0 || item < ITEMS;
            const int kb = k0 + (item / CG) * 8;
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                const typename G::Kin ki = g.k_info(kb + j, live ? kmax : 0);
#pragma unroll
                for (int q = 0; q < 4; ++q) v[p][j][q] = g.fetch(ri[p][q], ki);
            }
        }
    }

    __device__ __forceinline__ void store(half_t* tile, int tid) const {
#pragma unroll
        for (int p = 0; p < PASSES; ++p) {
            const int item = p * NT + tid;
            if (ITEMS % NT == 0 || item < ITEMS) {
                const int row = (item % CG) * 4;
                const int chunk = item / CG;
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    float col[8];
#pragma unroll
                    for (int j = 0; j < 8; ++j) col[j] = v[p][j][q];
                    lds_write8<BK>(tile, row + q, chunk, pack8(col));
                }
            }
        }
    }
};

// Each thread owns 1 row x 8 consecutive k (consecutive threads take
// consecutive k chunks of a row): used when k is the contiguous direction
// (pixels, in the weight-gradient GEMM).
template <int ROWS, int BK, int NT, class G>
struct StageGatherKC {
    static constexpr int TPR = BK / 8;
    static constexpr int ITEMS = ROWS * TPR;
    static constexpr int PASSES = (ITEMS + NT - 1) / NT;
    float v[PASSES][8];
    typename G::Row ri[PASSES];

    __device__ __forceinline__ void init(const G& g, int r0, int tid) {
#pragma unroll
        for (int p = 0; p < PASSES; ++p) ri[p] = g.row_info(r0 + (p * NT + tid) / TPR);
    }

    __device__ __forceinline__ void load(const G& g, int k0, int kmax, int tid) {
#pragma unroll
        for (int p = 0; p < PASSES; ++p) {
            const int item = p * NT + tid;
            const bool live = ITEMS % NT == 0 || item < ITEMS;
            const int kb = k0 + (item % TPR) * 8;
#pragma unroll
            for (int j = 0; j < 8; ++j) v[p][j] = g.fetch(ri[p], g.k_info(kb + j, live ? kmax : 0));
        }
    }

    __device__ __forceinline__ void store(half_t* tile, int tid) const {
#pragma unroll
        for (int p = 0; p < PASSES; ++p) {
            const int item = p * NT + tid;
            if (ITEMS % NT == 0 || item < ITEMS)
                lds_write8<BK>(tile, item / TPR, item % TPR, pack8(v[p]));
        }
    }
};

}  // namespace seera
