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
// chunks of a row are XOR-swizzled by the row index so that the lanes reading
// consecutive rows at the same k spread over all LDS banks.
//
// Global loads go through buffer resources: a lane whose element lies outside
// the tensor (edge tiles, K tails) gets an offset past the resource's
// num_records and the hardware returns 0 for it, so predication costs one
// v_cndmask instead of a branch per load.
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

// ---------------------------------------------------------------------------
// Buffer-resource loads. A resource covers kBufRecords bytes from its base;
// offsets at or beyond kBufOOB read as 0. Callers keep every in-range offset
// below kBufOOB (the host checks tile spans against kMaxTileSpanBytes).
// ---------------------------------------------------------------------------
typedef __amdgpu_buffer_rsrc_t rsrc_t;
constexpr uint32_t kBufRecords = 0x7FFFFF00u;
constexpr uint32_t kBufOOB = 0x7FFFFF00u;
constexpr int64_t kMaxTileSpanBytes = 0x7F000000ll;

__device__ __forceinline__ rsrc_t make_rsrc(const void* base) {
    // Word 3 = 0x00020000: raw (untyped) 32-bit data format, no swizzle.
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, kBufRecords,
                                             0x00020000);
}

// A buffer resource at element `off` of a tensor of `total` floats covering
// the rest of the tensor (capped at kBufRecords bytes): a load past the
// tensor's end reads 0 and a store there is dropped, so an offset that leaves
// the tensor cannot fault.
__device__ __forceinline__ rsrc_t make_rsrc_in(const float* tensor, int64_t total, int64_t off) {
    const int64_t bytes = (total - off) * 4;
    const uint32_t n = bytes <= 0 ? 0u : bytes >= (int64_t)kBufRecords ? kBufRecords : (uint32_t)bytes;
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(tensor + off), (short)0, n, 0x00020000);
}

__device__ __forceinline__ floatx4 buf_load4(rsrc_t r, uint32_t byte_off) {
    return __builtin_bit_cast(floatx4, __builtin_amdgcn_raw_buffer_load_b128(r, byte_off, 0, 0));
}

// Per-lane offset plus a wave-uniform one (held in an SGPR). Callers keep
// voff + soff below 2^32; a lane with voff >= kBufOOB reads 0.
__device__ __forceinline__ floatx4 buf_load4s(rsrc_t r, uint32_t voff, uint32_t soff) {
    return __builtin_bit_cast(floatx4, __builtin_amdgcn_raw_buffer_load_b128(r, voff, soff, 0));
}

__device__ __forceinline__ float buf_load1(rsrc_t r, uint32_t byte_off) {
    return __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(r, byte_off, 0, 0));
}

// ---------------------------------------------------------------------------
// LDS tile addressing.
// ---------------------------------------------------------------------------

// Element offset (in halves) of 16-byte chunk `chunk` of row `row` in a tile
// whose rows hold BK halves.
//
// A 128-byte window covers all 32 banks as eight 16-byte slots, and a wave's
// ds_read/write_b128 is served eight lanes at a time, so eight lanes must hit
// eight distinct slots. Three access patterns occur:
//   MFMA fragment reads   8 consecutive rows, one chunk
//   K-contiguous stores   consecutive lanes fill the chunks of consecutive rows
//   transposed stores     rows 4g+q for 8 consecutive g, one chunk and q
// BK=64: one row per window, slot = chunk ^ f(row) with f's three bits
//   (r0^r3, r1^r4, r2): a bijection in (r0,r1,r2) for the reads and in
//   (r2,r3,r4) for the transposed stores.
// BK=32: rows 2j and 2j+1 share window j, slot = (4*(row&1) + chunk) ^ f(j)
//   with f(j) = (j0^j2, j1, j3): its low two bits are a bijection in (j0,j1)
//   for the reads and all three bits one in (j1,j2,j3) for the stores.
template <int BK>
__device__ __forceinline__ int lds_off(int row, int chunk) {
    static_assert(BK == 32 || BK == 64, "BK must be 32 or 64");
    if constexpr (BK == 64) {
        const int f = ((row ^ (row >> 3)) & 3) | (row & 4);
        return row * 64 + ((chunk ^ f) << 3);
    } else {
        const int j = row >> 1;
        const int f = ((j ^ (j >> 2)) & 1) | (j & 2) | ((j >> 1) & 4);
        return j * 64 + (((((row & 1) << 2) | chunk) ^ f) << 3);
    }
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
// A stager covers a tile of ROWS (M or N) x BK (K) elements starting at
// (r0, k0); elements with row >= rmax or k >= kmax read as 0.
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
        const rsrc_t rs = make_rsrc(base + r0 * ld + k0);
#pragma unroll
        for (int p = 0; p < PASSES; ++p) {
            const int item = p * NT + tid;
            const int dr = item / TPR;
            const int dk = (item % TPR) * 8;
            const bool live = (ITEMS % NT == 0 || item < ITEMS) && r0 + dr < rmax;
            const uint32_t off = (uint32_t)(dr * ld + dk) * 4u;
            if constexpr (VEC == 4) {
#pragma unroll
                for (int h = 0; h < 2; ++h) {
                    const bool ok = live && k0 + dk + 4 * h < kmax;
                    const floatx4 x = buf_load4(rs, ok ? off + 16u * h : kBufOOB);
#pragma unroll
                    for (int j = 0; j < 4; ++j) v[p][4 * h + j] = x[j];
                }
            } else {
#pragma unroll
                for (int j = 0; j < 8; ++j) {
                    const bool ok = live && k0 + dk + j < kmax;
                    v[p][j] = buf_load1(rs, ok ? off + 4u * j : kBufOOB);
                }
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
// owns a KK(k) x 4(row) block, loads it as KK row-vectors and transposes it in
// registers into KK-half pieces of 4 K-contiguous LDS rows. KK is 8 (one
// 16-byte chunk per row) when the tile has at least one such block per
// thread; smaller tiles use KK = 4 or 2 so that every thread holds a block:
// with KK = 8 the threads past the tile's blocks would idle while one wave
// issued all of the tile's loads. Consecutive threads take consecutive row
// groups so a wave reads contiguous memory. VEC=4 needs the row extent % 4 ==
// 0, ld % 4 == 0 and a 16-byte aligned base.
template <int ROWS, int BK, int NT, int VEC>
struct StageMNC {
    static constexpr int CG = ROWS / 4;
    static constexpr int KK = CG * BK / 8 >= NT ? 8 : (CG * BK / 4 >= NT ? 4 : 2);
    static constexpr int KG = BK / KK;
    static constexpr int ITEMS = CG * KG;
    static constexpr int PASSES = (ITEMS + NT - 1) / NT;
    float v[PASSES][KK][4];

    // Item -> (first row dr, first k dk). With KK = 2 each store is a 4-byte
    // write per lane, served per 32-lane half; the half's lanes take 8 row
    // groups x the 4 k pairs of one 16-byte chunk, 32 distinct dwords under
    // the lds_off swizzle (16 row groups x 2 k pairs, the plain order, put
    // two lanes on every bank). Otherwise consecutive items take
    // consecutive row groups.
    static constexpr bool kHalfWaveOrder = KK == 2 && CG % 8 == 0 && KG % 4 == 0;
    static __device__ __forceinline__ void item_pos(int item, int& dr, int& dk) {
        if constexpr (kHalfWaveOrder) {
            const int rest = item >> 5;
            dr = ((item & 7) + 8 * (rest % (CG / 8))) * 4;
            dk = (((item >> 3) & 3) + 4 * (rest / (CG / 8))) * KK;
        } else {
            dr = (item % CG) * 4;
            dk = (item / CG) * KK;
        }
    }
    // The other index of the thread's items (0 .. NT/CG - 1): when a thread
    // keeps one row group over all passes (NT % CG == 0, and NT % (4 CG) == 0
    // in the half-wave order), (item_pos row group, item_slot) is a bijection
    // on the threads.
    static __device__ __forceinline__ int item_slot(int tid) {
        if constexpr (kHalfWaveOrder)
            return ((tid >> 3) & 3) + 4 * ((tid >> 5) / (CG / 8));
        else
            return tid / CG;
    }

    __device__ __forceinline__ void load(const float* __restrict__ base, int64_t ld,
                                         int r0, int rmax, int k0, int kmax, int tid) {
        const rsrc_t rs = make_rsrc(base + k0 * ld + r0);
#pragma unroll
        for (int p = 0; p < PASSES; ++p) {
            const int item = p * NT + tid;
            int dr, dk;
            item_pos(item, dr, dk);
            const bool live = ITEMS % NT == 0 || item < ITEMS;
#pragma unroll
            for (int j = 0; j < KK; ++j) {
                const bool kin = live && k0 + dk + j < kmax;
                const uint32_t off = (uint32_t)((dk + j) * ld + dr) * 4u;
                if constexpr (VEC == 4) {
                    const bool ok = kin && r0 + dr < rmax;
                    const floatx4 x = buf_load4(rs, ok ? off : kBufOOB);
#pragma unroll
                    for (int q = 0; q < 4; ++q) v[p][j][q] = x[q];
                } else {
#pragma unroll
                    for (int q = 0; q < 4; ++q) {
                        const bool ok = kin && r0 + dr + q < rmax;
                        v[p][j][q] = buf_load1(rs, ok ? off + 4u * q : kBufOOB);
                    }
                }
            }
        }
    }

    __device__ __forceinline__ void store(half_t* tile, int tid) const {
#pragma unroll
        for (int p = 0; p < PASSES; ++p) {
            const int item = p * NT + tid;
            if (ITEMS % NT == 0 || item < ITEMS) {
                int row, dk;
                item_pos(item, row, dk);
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    if constexpr (KK == 8) {
                        float col[8];
#pragma unroll
                        for (int j = 0; j < 8; ++j) col[j] = v[p][j][q];
                        lds_write8<BK>(tile, row + q, dk / 8, pack8(col));
                    } else {
                        // KK halves at k = dk .. dk+KK-1 of row + q: a piece of
                        // the row's 16-byte chunk dk / 8.
                        typedef _Float16 halfk __attribute__((ext_vector_type(KK)));
                        halfk h;
#pragma unroll
                        for (int j = 0; j < KK; ++j) h[j] = to_half(v[p][j][q]);
                        *reinterpret_cast<halfk*>(tile + lds_off<BK>(row + q, dk / 8) + dk % 8) = h;
                    }
                }
            }
        }
    }
};

// ---------------------------------------------------------------------------
// Streaming stagers for the warp-specialised producers (igemm_ws2_kernel).
// Same tile, same fp16 LDS image as StageKC / StageMNC with VEC=4, but split
// so that a producer can overlap its loads with its stores:
//   init(base, ld, r0, rmax, tid)  per-thread item offsets, once per block
//   slice(k0)                      buffer resource of the K slice at k0
//   load(regs, q, rsrc)            issue the loads of part q into `regs`
//   store(regs, q, tile, tid)      round part q to fp16 and write it to LDS
// A dead row (>= rmax) keeps an offset past num_records and reads 0. Every K
// slice is whole (the host sends K % BK != 0 to igemm_ws_kernel): a per-load
// k predicate costs registers and, under a branch, exact vmcnt waits.
// ---------------------------------------------------------------------------
template <int ROWS, int BK, int NP>
struct WsStageKC {
    static constexpr int TPR = BK / 8;                // threads per row
    static constexpr int PARTS = ROWS * TPR / NP;     // rows NP/TPR apart
    static_assert(ROWS * TPR % NP == 0 && NP % TPR == 0, "tile does not split into parts");
    struct Regs {
        floatx4 v[PARTS][2];
    };
    const float* base;  // element (r0, 0)
    uint32_t off[PARTS];
    int dk;

    __device__ __forceinline__ void init(const float* b, int64_t ld, int r0, int rmax, int tid) {
        base = b + (int64_t)r0 * ld;
        dk = (tid % TPR) * 8;
#pragma unroll
        for (int q = 0; q < PARTS; ++q) {
            const int dr = q * (NP / TPR) + tid / TPR;
            off[q] = r0 + dr < rmax ? (uint32_t)(dr * ld + dk) * 4u : kBufOOB;
        }
    }
    __device__ __forceinline__ rsrc_t slice(int k0) const { return make_rsrc(base + k0); }
    __device__ __forceinline__ void load(Regs& r, int q, rsrc_t rs) const {
#pragma unroll
        for (int h = 0; h < 2; ++h) r.v[q][h] = buf_load4(rs, off[q] + 16u * h);
    }
    __device__ __forceinline__ void store(const Regs& r, int q, half_t* tile, int tid) const {
        float v[8];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            v[j] = r.v[q][0][j];
            v[4 + j] = r.v[q][1][j];
        }
        lds_write8<BK>(tile, q * (NP / TPR) + tid / TPR, tid % TPR, pack8(v));
    }
};

template <int ROWS, int BK, int NP>
struct WsStageMNC {
    static constexpr int CG = ROWS / 4;               // 4-row groups
    static constexpr int PARTS = CG * (BK / 8) / NP;  // k groups NP/CG apart
    static_assert(CG * (BK / 8) % NP == 0 && NP % CG == 0, "tile does not split into parts");
    struct Regs {
        floatx4 v[PARTS][8];
    };
    const float* base;  // element (r0, k = 0)
    uint32_t off[PARTS];
    uint32_t kstep;     // bytes between consecutive k
    int dk[PARTS];

    __device__ __forceinline__ void init(const float* b, int64_t ld, int r0, int rmax, int tid) {
        base = b + r0;
        kstep = (uint32_t)ld * 4u;
        const int dr = (tid % CG) * 4;
#pragma unroll
        for (int q = 0; q < PARTS; ++q) {
            dk[q] = (q * (NP / CG) + tid / CG) * 8;
            off[q] = r0 + dr < rmax ? (uint32_t)(dk[q] * ld + dr) * 4u : kBufOOB;
        }
    }
    __device__ __forceinline__ rsrc_t slice(int k0) const {
        return make_rsrc(base + (int64_t)k0 * (kstep / 4u));
    }
    __device__ __forceinline__ void load(Regs& r, int q, rsrc_t rs) const {
        // k step j rides in the wave-uniform offset; a dead lane's offset
        // stays past num_records (the host bounds BK * ld well below 2^31).
#pragma unroll
        for (int j = 0; j < 8; ++j) r.v[q][j] = buf_load4s(rs, off[q], j * kstep);
    }
    __device__ __forceinline__ void store(const Regs& r, int q, half_t* tile, int tid) const {
        const int dr = (tid % CG) * 4;
#pragma unroll
        for (int c = 0; c < 4; ++c) {
            float col[8];
#pragma unroll
            for (int j = 0; j < 8; ++j) col[j] = r.v[q][j][c];
            lds_write8<BK>(tile, dr + c, dk[q] / 8, pack8(col));
        }
    }
};

// Fused forward epilogue (Dense layer: matmul, broadcast_add_4d, relu --
// engine_cuda/src/broadcast.cu:12-64, activations.cu:9-15): the bias is added
// in fp32 to the fp32 result, and ReLU writes out = v > 0 ? v : 0 and
// mask = v > 0 ? 1 : 0, so the result is the unfused sequence's, bit for bit.
//
// kActReluGrad is the backward of that ReLU fused into the dA GEMM's store:
// out = v * mask with mask the forward's 0/1 buffer (an input here), the
// reference's local_grad * cp (Seera_Engine.py:579); no bias is added.
constexpr int kActNone = 0, kActRelu = 1, kActReluGrad = 2;
__device__ __forceinline__ void epilogue(float* out, float* mask, float v, float bias, int act) {
    if (act == kActReluGrad) {
        *out = v * *mask;
        return;
    }
    v += bias;
    if (act == kActRelu) {
        const bool pos = v > 0.f;
        *out = pos ? v : 0.f;
        if (mask) *mask = pos ? 1.f : 0.f;
    } else {
        *out = v;
    }
}

// Bytes a K-contiguous stager's resource must span for a ROWS x BK tile with
// leading dimension ld (host-side check against kMaxTileSpanBytes).
inline int64_t span_kc(int rows, int bk, int64_t ld) { return ((int64_t)rows * ld + bk) * 4; }
inline int64_t span_mnc(int rows, int bk, int64_t ld) { return ((int64_t)bk * ld + rows) * 4; }

// ---------------------------------------------------------------------------
// Wave-level MFMA over one BK slice: the wave owns a (TM*32) x (TN*32) block of
// the block tile at (wm0, wn0), accumulators acc[TM][TN]. The fragments of
// k-step kk+1 are read from LDS while the matrix cores work on k-step kk.
// Accumulator layout of v_mfma_f32_32x32x16_f16 (lane l, element r):
//   row = 8*(r/4) + 4*(l/32) + r%4, col = l%32.
// Operand layout: lane l holds row l%32, k = 8*(l/32) .. 8*(l/32)+7.
// ---------------------------------------------------------------------------
template <int BK, int TM, int TN>
__device__ __forceinline__ void read_frags(const half_t* As, const half_t* Bs, int wm0, int wn0,
                                           int lane, int kk, half8 (&a)[TM], half8 (&b)[TN]) {
    const int chunk = kk * 2 + (lane >> 5);
#pragma unroll
    for (int i = 0; i < TM; ++i) a[i] = lds_read8<BK>(As, wm0 + i * 32 + (lane & 31), chunk);
#pragma unroll
    for (int j = 0; j < TN; ++j) b[j] = lds_read8<BK>(Bs, wn0 + j * 32 + (lane & 31), chunk);
}

template <int BK, int TM, int TN, bool PREFETCH = true>
__device__ __forceinline__ void mfma_slice(const half_t* As, const half_t* Bs, int wm0,
                                           int wn0, int lane, floatx16 (&acc)[TM][TN]) {
    constexpr int KK = BK / 16;
    if constexpr (PREFETCH) {
        half8 a[2][TM], b[2][TN];
        read_frags<BK, TM, TN>(As, Bs, wm0, wn0, lane, 0, a[0], b[0]);
#pragma unroll
        for (int kk = 0; kk < KK; ++kk) {
            if (kk + 1 < KK)
                read_frags<BK, TM, TN>(As, Bs, wm0, wn0, lane, kk + 1, a[(kk + 1) & 1],
                                       b[(kk + 1) & 1]);
#pragma unroll
            for (int i = 0; i < TM; ++i)
#pragma unroll
                for (int j = 0; j < TN; ++j)
                    acc[i][j] = mfma32x32x16(a[kk & 1][i], b[kk & 1][j], acc[i][j]);
        }
    } else {
        // One fragment set: for waves whose register budget is tight; another
        // wave on the SIMD covers the LDS latency.
#pragma unroll
        for (int kk = 0; kk < KK; ++kk) {
            half8 a[TM], b[TN];
            read_frags<BK, TM, TN>(As, Bs, wm0, wn0, lane, kk, a, b);
#pragma unroll
            for (int i = 0; i < TM; ++i)
#pragma unroll
                for (int j = 0; j < TN; ++j) acc[i][j] = mfma32x32x16(a[i], b[j], acc[i][j]);
        }
    }
}

// gm value asking tile_coords for the round-by-round region order below.
constexpr int kGmRegions = -16;

// Map a linear workgroup id to (tile_m, tile_n) so that the workgroups one XCD
// receives (the dispatcher deals ids round-robin over the 8 XCDs) form compact
// GM-row groups that share A and B panels in that XCD's L2.
//
// gm == kGmRegions (one block per CU, tiles_m and tiles_n multiples of 16,
// more tiles than one round of 256 CUs): each round of 256 blocks covers one
// 16 x 16-tile region, each XCD a 4 x 8-tile block of it (its 32 CUs), and
// consecutive rounds walk the regions in snake order, so that each round
// shares its A row panels or its B column panels with the one before. The
// plain order instead gives every round all tile rows and 8 tile columns:
// all of A plus 8 column panels per round, which at 8192^3 (fp32 operands,
// 512 MB) re-reads A from HBM each round once A and B outgrow the MALL.
__device__ __forceinline__ void tile_coords(int bid, int nblocks, int tiles_n, int gm,
                                            int& tm, int& tn) {
    constexpr int XCD = 8;
    if (gm == kGmRegions) {
        const int x = bid % XCD, j = bid / XCD;   // XCD, and order within it
        const int round = j >> 5, s = j & 31;     // 32 CUs per XCD
        const int rn = tiles_n >> 4;              // regions per region row
        const int rr = round / rn;
        int rc = round - rr * rn;
        if (rr & 1) rc = rn - 1 - rc;             // snake
        tm = 16 * rr + 4 * (x & 3) + (s & 3);
        tn = 16 * rc + 8 * (x >> 2) + (s >> 2);
        return;
    }
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
