// mfma_core.h -- building blocks of the gfx950 fp16-MFMA tile engine shared by
// the GEMM and convolution kernels.
//
// Numerics (reference GEMM.cu:41,52 and convolution.cu:59,68): every operand
// element is read as fp32 from HBM, rounded to fp16 with round-to-nearest-even
// on its way into LDS, multiplied on the matrix cores and accumulated in fp32.
//
// LDS layout: each operand tile is stored "K-contiguous", one row per M (or N)
// index holding BK fp16 values, so that one 16-byte ds_read_b128 gives a lane
// the 8 consecutive k values that v_mfma_f32_32x32x16_f16 expects. The 16-byte
// chunks of a row are XOR-swizzled by the row index so that the 32 lanes
// reading 32 consecutive rows at the same k spread over all LDS banks.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace seera {

typedef _Float16 half_t;
typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef float floatx16 __attribute__((ext_vector_type(16)));
typedef float floatx4 __attribute__((ext_vector_type(4)));

// Round-to-nearest-even fp32 -> fp16 (v_cvt_f16_f32 under the default mode),
// overflowing to +-inf above 65504 like __float2half.
__device__ __forceinline__ half_t to_half(float x) { return (half_t)x; }

__device__ __forceinline__ half8 pack8(const float* v) {
    half8 h;
#pragma unroll
    for (int i = 0; i < 8; ++i) h[i] = to_half(v[i]);
    return h;
}

__device__ __forceinline__ floatx16 mfma32x32x16(half8 a, half8 b, floatx16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
}

// Element offset (in halves) of 16-byte chunk `chunk` of row `row` in a tile
// whose rows hold BK halves.
template <int BK>
__device__ __forceinline__ int lds_off(int row, int chunk) {
    static_assert(BK == 32 || BK == 64, "BK must be 32 or 64");
    // BK=32: a row is 64 B, two rows share a 128-byte bank window, so the
    // swizzle key changes every second row; BK=64: one row per window.
    const int key = BK == 32 ? ((row >> 1) & 3) : (row & 7);
    return row * BK + ((chunk ^ key) << 3);
}

template <int BK>
__device__ __forceinline__ half8 lds_read8(const half_t* tile, int row, int chunk) {
    return *reinterpret_cast<const half8*>(tile + lds_off<BK>(row, chunk));
}

template <int BK>
__device__ __forceinline__ void lds_write8(half_t* tile, int row, int chunk, half8 v) {
    *reinterpret_cast<half8*>(tile + lds_off<BK>(row, chunk)) = v;
}

// ---------------------------------------------------------------------------
// Operand stagers: global fp32 -> registers (load) -> fp16 LDS tile (store).
// A stager covers a tile of ROWS (M or N) x BK (K) elements.
// ---------------------------------------------------------------------------

// K-contiguous operand: element (row, k) at base[row * ld + k]. Each thread
// owns 8 consecutive k of one row. VEC=4 needs K % 4 == 0, ld % 4 == 0 and a
// 16-byte aligned base; VEC=1 handles any shape.
template <int ROWS, int BK, int NT, int VEC>
struct StageKC {
    static constexpr int TPR = BK / 8;
    static constexpr int ITEMS = ROWS * TPR;
    static constexpr int PASSES = (ITEMS + NT - 1) / NT;
    float v[PASSES][8];

    __device__ __forceinline__ void load(const float* __restrict__ base, int64_t ld,
                                         int r0, int rmax, int k0, int kmax, int tid) {
#pragma unroll
        for (int p = 0; p < PASSES; ++p) {
            const int item = p * NT + tid;
            const int row = r0 + item / TPR;
            const int k = k0 + (item % TPR) * 8;
            const bool live = (ITEMS % NT == 0 || item < ITEMS) && row < rmax;
            const float* src = base + (int64_t)row * ld + k;
            if constexpr (VEC == 4) {
#pragma unroll
                for (int h = 0; h < 2; ++h) {
                    floatx4 x = {0.f, 0.f, 0.f, 0.f};
                    if (live && k + 4 * h < kmax)
                        x = *reinterpret_cast<const floatx4*>(src + 4 * h);
#pragma unroll
                    for (int j = 0; j < 4; ++j) v[p][4 * h + j] = x[j];
                }
            } else {
#pragma unroll
                for (int j = 0; j < 8; ++j)
                    v[p][j] = (live && k + j < kmax) ? src[j] : 0.f;
            }
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

// MN-contiguous operand: element (row, k) at base[k * ld + row]. Each thread
// owns an 8(k) x 4(row) block, loads it as 8 row-vectors and transposes it in
// registers into 4 K-contiguous LDS rows. Consecutive threads take
// consecutive row groups so a wave reads contiguous memory. VEC=4 needs the
// row extent % 4 == 0, ld % 4 == 0 and a 16-byte aligned base.
template <int ROWS, int BK, int NT, int VEC>
struct StageMNC {
    static constexpr int CG = ROWS / 4;
    static constexpr int KG = BK / 8;
    static constexpr int ITEMS = CG * KG;
    static constexpr int PASSES = (ITEMS + NT - 1) / NT;
    float v[PASSES][8][4];

    __device__ __forceinline__ void load(const float* __restrict__ base, int64_t ld,
                                         int r0, int rmax, int k0, int kmax, int tid) {
#pragma unroll
        for (int p = 0; p < PASSES; ++p) {
            const int item = p * NT + tid;
            const int row = r0 + (item % CG) * 4;
            const int k = k0 + (item / CG) * 8;
            const bool live = ITEMS % NT == 0 || item < ITEMS;
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                const float* src = base + (int64_t)(k + j) * ld + row;
                const bool kin = live && k + j < kmax;
                if constexpr (VEC == 4) {
                    floatx4 x = {0.f, 0.f, 0.f, 0.f};
                    if (kin && row < rmax) x = *reinterpret_cast<const floatx4*>(src);
#pragma unroll
                    for (int q = 0; q < 4; ++q) v[p][j][q] = x[q];
                } else {
#pragma unroll
                    for (int q = 0; q < 4; ++q)
                        v[p][j][q] = (kin && row + q < rmax) ? src[q] : 0.f;
                }
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

// ---------------------------------------------------------------------------
// Wave-level MFMA over one BK slice: the wave owns a (TM*32) x (TN*32) block of
// the block tile at (wm0, wn0), accumulators acc[TM][TN].
// Accumulator layout of v_mfma_f32_32x32x16_f16 (lane l, element r):
//   row = 8*(r/4) + 4*(l/32) + r%4, col = l%32.
// ---------------------------------------------------------------------------
template <int BK, int TM, int TN>
__device__ __forceinline__ void mfma_slice(const half_t* As, const half_t* Bs, int wm0,
                                           int wn0, int lane, floatx16 (&acc)[TM][TN]) {
#pragma unroll
    for (int kk = 0; kk < BK / 16; ++kk) {
        const int chunk = kk * 2 + (lane >> 5);
        half8 a[TM], b[TN];
#pragma unroll
        for (int i = 0; i < TM; ++i) a[i] = lds_read8<BK>(As, wm0 + i * 32 + (lane & 31), chunk);
#pragma unroll
        for (int j = 0; j < TN; ++j) b[j] = lds_read8<BK>(Bs, wn0 + j * 32 + (lane & 31), chunk);
#pragma unroll
        for (int i = 0; i < TM; ++i)
#pragma unroll
            for (int j = 0; j < TN; ++j) acc[i][j] = mfma32x32x16(a[i], b[j], acc[i][j]);
    }
}

// Map a linear workgroup id to (tile_m, tile_n) so that the workgroups one XCD
// receives (the dispatcher deals ids round-robin over the 8 XCDs) form compact
// GM-row groups that share A and B panels in that XCD's L2.
__device__ __forceinline__ void tile_coords(int bid, int nblocks, int tiles_n, int gm,
                                            int& tm, int& tn) {
    constexpr int XCD = 8;
    int id = bid;
    if (nblocks % XCD == 0) id = (bid % XCD) * (nblocks / XCD) + bid / XCD;
    const int tiles_m = nblocks / tiles_n;
    const int group = id / (gm * tiles_n);
    const int first = group * gm;
    const int rows = min(tiles_m - first, gm);
    const int in_group = id - group * gm * tiles_n;
    tm = first + in_group % rows;
    tn = in_group / rows;
}

}  // namespace seera
