// conv_wgrad.hip -- row-streaming weight gradient of a stride-1 convolution.
//
//   dW[f, c, r, s] = sum_{b, oh, ow} dY[b, f, oh, ow] * X[b, c, oh - ph + r, ow - pw + s]
// (convolution.cu:268-366, 431-452): a GEMM with M = filters, N = (tap,
// channel), K = output pixels. A block owns one image, a strip of L output
// rows, 64 filters and 64 channels, and keeps the whole 64 x (64*R*S) partial
// in registers while it walks the strip two output rows per step:
//   * 8 producer waves stream the dY rows of the step and the X rows the step
//     adds (fp16, pixel-contiguous per channel, as in HBM) into two LDS rings,
//     loading two steps ahead;
//   * 8 consumer waves, one per (half of the filters, 16 channels), run
//     v_mfma_f32_16x16x32_f16 with 16 filters x 32 pixels of dY as A and 16
//     channels x 32 pixels of X as B. The S column taps of an X row are one
//     aligned 16-byte read plus the next two pixels, shifted in registers
//     (v_alignbit), so the ring holds each X row once.
// Each block writes its partial; wgrad_reduce (conv_band.hip) adds them in a
// fixed order. HBM sees each dY element once and each X row once per strip
// plus R-1 halo rows. With the bias gradient requested, the producers also
// sum every dY element they load (fp32, before rounding) and each block
// writes 64 per-filter partials that the same reduce adds up: db[f] = sum of
// dY over images and pixels (the reference's three cuten.sum calls,
// Seera_Engine.py:42-65) without a second pass over dY.
#include "conv_band.h"
#include "mfma_core.h"

namespace seera {
namespace {

typedef float floatx4_t __attribute__((ext_vector_type(4)));
typedef uint32_t uintx4_t __attribute__((ext_vector_type(4)));

__device__ __forceinline__ floatx4_t mfma16x16x32(half8 a, half8 b, floatx4_t c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}

constexpr int kG = 2;            // output rows per step
constexpr int kCons = 512;       // 8 consumer waves
constexpr int kProd = 512;       // 8 producer waves
constexpr int kNT = kCons + kProd;
constexpr int kXI = 3;           // X items (1 channel x 8 pixels) per producer thread per step
constexpr int kDI = 2;           // dY items per producer thread per step
constexpr int kTile = 64;        // filters and channels per block

struct WStreamArgs {
    const float* dy;     // [B, F, Ho, Wo]
    const float* x;      // [B, C, H, W]
    float* part;         // [tiles][nsplit][64][64*R*S]
    float* dbpart;       // [ftiles][nsplit][64] bias-gradient partials (nullptr: none)
    int B, C, H, W, F, Ho, Wo, R, S, ph, pw;
    int L, nstrip, nsplit, nctile;
    int ncol;            // column tiles per row (Wo > 64: tiles of Wp = 64 output columns)
    int vP;              // > 0: strips run over all images as one sequence of vP = Ho + R - 1
                         // rows per image (rows Ho.. of each: dY zero); 0: strips of one image
    int vrows;           // B * vP
    int Wp;              // padded row length of a column tile (pixels, multiple of 32)
    int rs;              // LDS row stride in halves (Wp + 16: 2 mod 4 16-byte slots)
    int NR;              // X ring rows (2*kG + R - 1)
    int64_t lds_bytes;
};

// Funnel shift of the 8 halves in b by one half, pulling in the low half of n.
__device__ __forceinline__ half8 shift1(half8 b, uint32_t n) {
    const uintx4_t u = __builtin_bit_cast(uintx4_t, b);
    uintx4_t o;
    o[0] = __builtin_amdgcn_alignbit(u[1], u[0], 16);
    o[1] = __builtin_amdgcn_alignbit(u[2], u[1], 16);
    o[2] = __builtin_amdgcn_alignbit(u[3], u[2], 16);
    o[3] = __builtin_amdgcn_alignbit(n, u[3], 16);
    return __builtin_bit_cast(half8, o);
}
// ... by two halves (one dword).
__device__ __forceinline__ half8 shift2(half8 b, uint32_t n) {
    const uintx4_t u = __builtin_bit_cast(uintx4_t, b);
    uintx4_t o;
    o[0] = u[1];
    o[1] = u[2];
    o[2] = u[3];
    o[3] = n;
    return __builtin_bit_cast(half8, o);
}

// 8 consecutive floats starting D floats into the 12-float window w0|w1|w2.
template <int D>
__device__ __forceinline__ half8 pick8(floatx4 w0, floatx4 w1, floatx4 w2) {
    float v[12] = {w0[0], w0[1], w0[2], w0[3], w1[0], w1[1], w1[2], w1[3], w2[0], w2[1], w2[2], w2[3]};
    float o[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) o[i] = v[D + i];
    return pack8(o);
}

// The 8 floats that start DD floats into the aligned 12-float window whose
// quads sit at byte offsets o0, o1, o2 (kBufOOB: outside the image, reads 0).
// Only those 8 floats are loaded: a loaded register that is never read would
// be free for the register allocator to reuse while its load is in flight,
// and the compiler then waits for that load to land (a full memory round trip
// per step).
template <int DD>
__device__ __forceinline__ void load_x8(rsrc_t r, uint32_t o0, uint32_t o1, uint32_t o2,
                                        float (&v)[8]) {
    static_assert(DD == 0 || DD == 3, "exact X loads exist for misalignment 0 and 3");
    const floatx4 mid = buf_load4(r, o1);
    if constexpr (DD == 0) {
        const floatx4 lo = buf_load4(r, o0);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            v[i] = lo[i];
            v[4 + i] = mid[i];
        }
        (void)o2;
    } else {
        typedef float f3 __attribute__((ext_vector_type(3)));
        const float lo = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(r, o0 + 12u, 0, 0));
        const f3 hi = __builtin_bit_cast(f3, __builtin_amdgcn_raw_buffer_load_b96(r, o2, 0, 0));
        v[0] = lo;
#pragma unroll
        for (int i = 0; i < 4; ++i) v[1 + i] = mid[i];
        v[5] = hi[0];
        v[6] = hi[1];
        v[7] = hi[2];
    }
}

// DD: the column misalignment (-pw) mod 4 when known at compile time (-1: any).
template <int RR, int SS, int DD>
__global__ __launch_bounds__(kNT) void stream_wgrad_kernel(const WStreamArgs a) {
    extern __shared__ __attribute__((aligned(16))) half_t smem[];
    const int split = blockIdx.x, ty = blockIdx.y;
    const int bs = split / a.ncol, ct = split - bs * a.ncol;
    const int b = a.vP ? 0 : bs / a.nstrip, strip = bs - b * a.nstrip;
    const int wc0 = ct * a.Wp;                   // first output column of the tile
    const int ftile = ty / a.nctile, ctile = ty - ftile * a.nctile;
    const int ohA = strip * a.L;                 // first output row (virtual row with vP)
    const int Lb = min(a.L, (a.vP ? a.vrows : a.Ho) - ohA);  // output rows of this strip
    const int nsteps = (Lb + kG - 1) / kG;
    const int xplane = kTile * a.rs;             // halves per X ring row
    half_t* const xr = smem;                     // [NR][64 c][rs]
    half_t* const dr = smem + a.NR * xplane;     // [2*kG][64 f][rs]
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);

    if (wave < kCons / 64) {
        // ---- consumers ----
        const int fh = wave & 1, cg = wave >> 1;
        const int kc = lane >> 4;
        // Fragment offsets within a ring row: dY rows f = 32*fh + 16*fg + lane%16,
        // X rows c = 16*cg + lane%16, pixels 8*kc..8*kc+7 of a 32-pixel block.
        const int aoff = (32 * fh + (lane & 15)) * a.rs + 8 * kc;
        const int boff = (16 * cg + (lane & 15)) * a.rs + 8 * kc;
        floatx4_t acc[2][RR][SS];
#pragma unroll
        for (int fg = 0; fg < 2; ++fg)
#pragma unroll
            for (int r = 0; r < RR; ++r)
#pragma unroll
                for (int s = 0; s < SS; ++s) acc[fg][r][s] = floatx4_t{0.f, 0.f, 0.f, 0.f};
        const int nkb = a.Wp >> 5;
        for (int st = 0; st < nsteps; ++st) {
            __syncthreads();  // the rows of step st are in the rings
            // The step's (row g, 32-pixel block kb) pairs q = g*nkb + kb. The
            // LDS reads run one tap row ahead of the MFMAs (the last tap row
            // of pair q reads pair q+1's dY fragments and first X row), and
            // are issued unconditionally: past the last pair they re-read it.
            const int nq = min(kG, Lb - st * kG) * nkb;
            int gn = 0, kbn = 0;  // pair whose fragments are read next
            const half_t* dln = dr + ((st * kG) % (2 * kG)) * (kTile * a.rs) + aoff;
            half8 fan[2], xbn;
            uint32_t xnn;
#define SEERA_WG_READ_A()                                                                  \
    {                                                                                      \
        _Pragma("unroll") for (int fg = 0; fg < 2; ++fg) fan[fg] =                         \
            *reinterpret_cast<const half8*>(dln + fg * 16 * a.rs + kbn * 32);              \
    }
#define SEERA_WG_READ_X(R_)                                                                \
    {                                                                                      \
        int slot = st * kG + gn + (R_);                                                    \
        slot = slot >= a.NR ? slot % a.NR : slot;                                          \
        const half_t* const xl = xr + slot * xplane + boff + kbn * 32;                     \
        xbn = *reinterpret_cast<const half8*>(xl);                                         \
        xnn = *reinterpret_cast<const uint32_t*>(xl + 8);                                  \
    }
            SEERA_WG_READ_A()
            SEERA_WG_READ_X(0)
            for (int q = 0; q < nq; ++q) {
                const half8 fa[2] = {fan[0], fan[1]};
#pragma unroll
                for (int r = 0; r < RR; ++r) {
                    const half8 base = xbn;
                    const uint32_t nb = xnn;
                    if (r + 1 < RR) {
                        SEERA_WG_READ_X(r + 1)
                    } else {
                        if (q + 1 < nq && ++kbn == nkb) {
                            kbn = 0;
                            ++gn;
                            dln = dr + ((st * kG + gn) % (2 * kG)) * (kTile * a.rs) + aoff;
                        }
                        SEERA_WG_READ_A()
                        SEERA_WG_READ_X(0)
                    }
                    half8 fb[SS];
                    fb[0] = base;
                    if constexpr (SS > 1) fb[1] = shift1(base, nb);
                    if constexpr (SS > 2) fb[2] = shift2(base, nb);
#pragma unroll
                    for (int s = 0; s < SS; ++s)
#pragma unroll
                        for (int fg = 0; fg < 2; ++fg)
                            acc[fg][r][s] = mfma16x16x32(fa[fg], fb[s], acc[fg][r][s]);
                }
            }
#undef SEERA_WG_READ_A
#undef SEERA_WG_READ_X
        }
        // Partial: part[ty][split][f64][n], n = (r*S + s)*64 + c; lane holds
        // filters 4*(lane/16) + i at channel lane%16 of its 16x16 tile.
        const int ntot = kTile * RR * SS;
        float* const dst = a.part + ((int64_t)ty * a.nsplit + split) * 64 * ntot;
#pragma unroll
        for (int fg = 0; fg < 2; ++fg)
#pragma unroll
            for (int r = 0; r < RR; ++r)
#pragma unroll
                for (int s = 0; s < SS; ++s) {
                    const int n = (r * SS + s) * kTile + 16 * cg + (lane & 15);
#pragma unroll
                    for (int i = 0; i < 4; ++i)
                        dst[(int64_t)(32 * fh + 16 * fg + 4 * kc + i) * ntot + n] = acc[fg][r][s][i];
                }
        if (a.dbpart) {
            // The producers' bias-gradient reduction reuses the rings once
            // every consumer is done with them (both barriers are matched
            // by the producers).
            __syncthreads();
            __syncthreads();
        }
        return;
    }

    // ---- producers ----
    // X item (row of the group, channel, octet j): ring columns 8j..8j+7 hold
    // X[.., ih, 8j - pw .. 8j - pw + 7], which lie dd floats into the aligned
    // 12-float window at column 8j - pw - dd. With dd known at compile time
    // exactly those 8 floats are loaded (load_x8); otherwise the window's three
    // float4s are loaded and picked at offset dd (dd uniform). dY item (row,
    // filter, octet j): columns 8j..8j+7 of the dY row (zero past Wo).
    // Buffer resources over this image's tile planes: out-of-range rows,
    // columns, channels and filters read 0.
    const int ptid = tid - kCons;
    const int c0 = ctile * kTile, f0 = ftile * kTile;
    const rsrc_t xsrc = make_rsrc_in(a.x, (int64_t)a.B * a.C * a.H * a.W, ((int64_t)b * a.C + c0) * a.H * a.W);
    const rsrc_t dsrc = make_rsrc_in(a.dy, (int64_t)a.B * a.F * a.Ho * a.Wo, ((int64_t)b * a.F + f0) * a.Ho * a.Wo);
    const int nxo = (a.Wp >> 3) + 1;             // X octets per ring row
    const int ndo = a.Wp >> 3;                   // dY octets per ring row
    const int dd = DD >= 0 ? DD : ((-a.pw) % 4 + 4) % 4;
    const int need = Lb + RR - 1;                // strip-relative X rows used
    const int ih0 = ohA - a.ph;                  // image row of strip X row 0
    // Per X item: row in group (kG: none), channel, first column (aligned),
    // byte offset of (channel, group row, first column) in the image tile, and
    // which of its three column quads lie inside the image.
    int xrow[kXI], xch[kXI], xcol[kXI], xoff[kXI], xqm[kXI];
#pragma unroll
    for (int k = 0; k < kXI; ++k) {
        const int it = ptid + k * kProd;
        const int j = it % nxo, rest = it / nxo;
        xch[k] = rest % kTile;
        xrow[k] = it < kG * kTile * nxo ? rest / kTile : kG;
        xcol[k] = wc0 + 8 * j - a.pw - dd;
        xoff[k] = (xch[k] * a.H * a.W + xcol[k]) * 4;  // row added per load
        xqm[k] = 0;
#pragma unroll
        for (int q = 0; q < 3; ++q) xqm[k] |= (unsigned)(xcol[k] + 4 * q) < (unsigned)a.W ? 1 << q : 0;
    }
    int drow[kDI], dfl[kDI], dcol[kDI], doff[kDI], dqm[kDI];
#pragma unroll
    for (int k = 0; k < kDI; ++k) {
        const int it = ptid + k * kProd;
        const int j = it % ndo, rest = it / ndo;
        dfl[k] = rest % kTile;
        drow[k] = it < kG * kTile * ndo ? rest / kTile : kG;
        dcol[k] = wc0 + 8 * j;
        doff[k] = (dfl[k] * a.Ho * a.Wo + dcol[k]) * 4;  // row added per load
        dqm[k] = (dcol[k] < a.Wo ? 1 : 0) | (dcol[k] + 4 < a.Wo ? 2 : 0);
    }
    floatx4 xv[kXI][3], dv[kDI][2];  // DD < 0: three aligned quads per X item
    float xw[kXI][8];                // DD >= 0: exactly the item's 8 floats
    // Bias gradient: each dY item's fp32 values as they pass through the
    // registers, one running sum per item (the item keeps its filter from
    // step to step). Channel tiles other than the first see the same dY.
    const bool db_on = a.dbpart != nullptr && ctile == 0;
    float dsum[kDI];
#pragma unroll
    for (int k = 0; k < kDI; ++k) dsum[k] = 0.f;

    // Loads of X group rows [I0, I0 + NX) and dY output rows [O0, O0 + ND).
#define SEERA_WG_LOAD(I0, NX, O0, ND)                                                      \
    {                                                                                      \
        _Pragma("unroll") for (int k = 0; k < kXI; ++k) {                                  \
            const int i = (I0) + xrow[k];                                                  \
            int bb = 0, ih = ih0 + i;                                                      \
            if (a.vP) {                                                                    \
                const int u = ohA + i;  /* virtual input row */                            \
                bb = u / a.vP;                                                             \
                ih = u - bb * a.vP - a.ph;                                                 \
            }                                                                              \
            /* (virtual rows: the last strip's X rows run R - 1 rows past    \
               the batch's last period, into an image bb = B that is not     \
               there) */                                                      \
            const bool rok = xrow[k] < (NX) && (unsigned)i < (unsigned)need &&             \
                             (unsigned)ih < (unsigned)a.H && c0 + xch[k] < a.C && bb < a.B; \
            const int xrb = (bb * a.C * a.H + ih) * a.W * 4;                               \
            uint32_t xo[3];                                                                \
            _Pragma("unroll") for (int q = 0; q < 3; ++q)                                  \
                xo[q] = rok && ((xqm[k] >> q) & 1) ? (uint32_t)(xoff[k] + xrb + 16 * q)    \
                                                   : kBufOOB;                              \
            if constexpr (DD >= 0) {                                                       \
                load_x8<DD < 0 ? 0 : DD>(xsrc, xo[0], xo[1], xo[2], xw[k]);                \
            } else {                                                                       \
                _Pragma("unroll") for (int q = 0; q < 3; ++q) xv[k][q] = buf_load4(xsrc, xo[q]); \
            }                                                                              \
        }                                                                                  \
        _Pragma("unroll") for (int k = 0; k < kDI; ++k) {                                  \
            const int o = (O0) + drow[k];                                                  \
            int bb = 0, oh = ohA + o;                                                      \
            if (a.vP) {                                                                    \
                bb = oh / a.vP;                                                            \
                oh -= bb * a.vP;  /* rows Ho.. of an image's period: dY zero */            \
            }                                                                              \
            const bool rok = drow[k] < (ND) && o < Lb && oh < a.Ho && f0 + dfl[k] < a.F;   \
            const int drb = (bb * a.F * a.Ho + oh) * a.Wo * 4;                             \
            _Pragma("unroll") for (int q = 0; q < 2; ++q) {                                \
                const uint32_t off = rok && ((dqm[k] >> q) & 1)                            \
                    ? (uint32_t)(doff[k] + drb + 16 * q) : kBufOOB;                        \
                dv[k][q] = buf_load4(dsrc, off);                                           \
            }                                                                              \
        }                                                                                  \
    }
    // Round and write them into the rings.
#define SEERA_WG_STORE(I0, NX, O0, ND)                                                     \
    {                                                                                      \
        const int xs0 = (I0) % a.NR;  /* ring slot of group row 0 (uniform) */             \
        _Pragma("unroll") for (int k = 0; k < kXI; ++k) {                                  \
            const int i = (I0) + xrow[k];                                                  \
            int slot = xs0 + xrow[k];                                                      \
            slot = slot >= a.NR ? slot - a.NR : slot;                                      \
            if (xrow[k] < (NX) && (unsigned)i < (unsigned)need) {                          \
                half8 h;                                                                   \
                if constexpr (DD >= 0) {                                                   \
                    h = pack8(xw[k]);                                                      \
                } else {                                                                   \
                    switch (dd) {                                                          \
                        case 0: h = pick8<0>(xv[k][0], xv[k][1], xv[k][2]); break;         \
                        case 1: h = pick8<1>(xv[k][0], xv[k][1], xv[k][2]); break;         \
                        case 2: h = pick8<2>(xv[k][0], xv[k][1], xv[k][2]); break;         \
                        default: h = pick8<3>(xv[k][0], xv[k][1], xv[k][2]); break;        \
                    }                                                                      \
                }                                                                          \
                *reinterpret_cast<half8*>(xr + slot * xplane + xch[k] * a.rs +             \
                                          xcol[k] - wc0 + a.pw + dd) = h;                  \
            }                                                                              \
        }                                                                                  \
        _Pragma("unroll") for (int k = 0; k < kDI; ++k) {                                  \
            const int o = (O0) + drow[k];                                                  \
            if (drow[k] < (ND) && o < Lb) {                                                \
                float v8[8];                                                               \
                _Pragma("unroll") for (int q = 0; q < 4; ++q) {                            \
                    v8[q] = dv[k][0][q];                                                   \
                    v8[4 + q] = dv[k][1][q];                                               \
                }                                                                          \
                if (db_on) {                                                               \
                    _Pragma("unroll") for (int q = 0; q < 8; ++q) dsum[k] += v8[q];        \
                }                                                                          \
                *reinterpret_cast<half8*>(dr + (o % (2 * kG)) * (kTile * a.rs) +           \
                                          dfl[k] * a.rs + dcol[k] - wc0) = pack8(v8);      \
            }                                                                              \
        }                                                                                  \
    }
    // Strip X row i sits in ring slot i % NR; the X rows step g adds are
    // [RR-1 + g*kG, RR-1 + (g+1)*kG), after RR-1 halo rows.
    if (RR > 1) {
        SEERA_WG_LOAD(0, RR - 1, 0, 0)
        SEERA_WG_STORE(0, RR - 1, 0, 0)
    }
    SEERA_WG_LOAD(RR - 1, kG, 0, kG)
    SEERA_WG_STORE(RR - 1, kG, 0, kG)
    SEERA_WG_LOAD(RR - 1 + kG, kG, kG, kG)
    __syncthreads();  // releases step 0
    for (int st = 0; st + 1 < nsteps; ++st) {
        // The slots written now held rows only step st-1 read.
        SEERA_WG_STORE(RR - 1 + (st + 1) * kG, kG, (st + 1) * kG, kG)
        SEERA_WG_LOAD(RR - 1 + (st + 2) * kG, kG, (st + 2) * kG, kG)
        __syncthreads();  // releases step st+1
    }
#undef SEERA_WG_LOAD
#undef SEERA_WG_STORE
    if (a.dbpart) {
        __syncthreads();  // every consumer is past its last ring read
        float* const red = reinterpret_cast<float*>(smem);
#pragma unroll
        for (int k = 0; k < kDI; ++k) red[k * kProd + ptid] = dsum[k];
        __syncthreads();
        // Filter f's items are it = (row * 64 + f) * ndo + j (row < kG,
        // j < ndo), stored at red[it]: summed in that order, from +0.
        if (ctile == 0 && ptid < kTile) {
            float sum = 0.f;
            for (int row = 0; row < kG; ++row)
                for (int j = 0; j < ndo; ++j) sum += red[(row * kTile + ptid) * ndo + j];
            a.dbpart[((int64_t)ftile * a.nsplit + split) * kTile + ptid] = sum;
        }
    }
}

template <int RR>
hipError_t launch_rr(const WStreamArgs& a, int ntiles, hipStream_t st) {
    const void* k;
    // 3x3 with pad 0 or 1 (column misalignment 0 or 3) gets the misalignment
    // at compile time; other shapes pick it at run time.
    const int dd = ((-a.pw) % 4 + 4) % 4;
    switch (a.S) {
        case 1: k = reinterpret_cast<const void*>(stream_wgrad_kernel<RR, 1, -1>); break;
        case 2: k = reinterpret_cast<const void*>(stream_wgrad_kernel<RR, 2, -1>); break;
        default:
            if (RR == 3 && dd == 3) k = reinterpret_cast<const void*>(stream_wgrad_kernel<3, 3, 3>);
            else if (RR == 3 && dd == 0) k = reinterpret_cast<const void*>(stream_wgrad_kernel<3, 3, 0>);
            else k = reinterpret_cast<const void*>(stream_wgrad_kernel<RR, 3, -1>);
            break;
    }
    hipError_t e = hipFuncSetAttribute(k, hipFuncAttributeMaxDynamicSharedMemorySize, (int)a.lds_bytes);
    if (e != hipSuccess) return e;
    void* args[] = {const_cast<WStreamArgs*>(&a)};
    return hipLaunchKernel(k, dim3(a.nsplit, ntiles), dim3(kNT), args, (size_t)a.lds_bytes, st);
}

}  // namespace

int stream_wgrad_partials(const float* Y, const float* X, int B, int C, int H, int W, int F,
                          int R, int S, int ph, int pw, bool with_db, hipStream_t st,
                          WgradPartials* out, bool* used) {
    *used = false;
    const int Ho = H + 2 * ph - R + 1, Wo = W + 2 * pw - S + 1;
    if (R < 1 || R > 3 || S < 1 || S > 3 || Ho <= 0 || Wo <= 0 || B <= 0) return SEERA_OK;
    if (W % 4 != 0 || Wo % 4 != 0 || ((reinterpret_cast<uintptr_t>(X) | reinterpret_cast<uintptr_t>(Y)) & 15))
        return SEERA_OK;
    WStreamArgs a{};
    a.dy = Y; a.x = X;
    a.B = B; a.C = C; a.H = H; a.W = W; a.F = F; a.Ho = Ho; a.Wo = Wo;
    a.R = R; a.S = S; a.ph = ph; a.pw = pw;
    // Rows wider than 64 output columns run as column tiles of 64 (the
    // X halo columns loaded by both neighbours; each dY column by one tile).
    a.Wp = Wo > 64 ? 64 : (Wo + 31) & ~31;
    a.ncol = (Wo + a.Wp - 1) / a.Wp;
    // Row stride Wp + 16 halves (2 mod 4 slots of 16 bytes): the fragment
    // reads (16 rows x 4 column chunks per wave) measured free of LDS bank
    // conflicts at that stride and 2-way conflicted at Wp + 8.
    a.rs = a.Wp + 16;
    a.NR = 2 * kG + R - 1;
    // X octets per row: columns up to Wp + 7 (the last 32-pixel block's
    // fragments plus the two pixels the column taps shift in).
    const int nxo = a.Wp / 8 + 1, ndo = a.Wp / 8;
    if (kG * kTile * nxo > kProd * kXI || kG * kTile * ndo > kProd * kDI ||
        (R - 1) * kTile * nxo > kProd * kXI)
        return SEERA_OK;
    a.lds_bytes = (int64_t)(a.NR + 2 * kG) * kTile * a.rs * 2;
    if (a.lds_bytes > kBandMaxLds) return SEERA_OK;
    const int64_t img = (int64_t)kTile * H * W * 4, dimg = (int64_t)kTile * Ho * Wo * 4;
    if (img > kMaxTileSpanBytes || dimg > kMaxTileSpanBytes) return SEERA_OK;
    a.nctile = (C + kTile - 1) / kTile;
    const int ntiles = a.nctile * ((F + kTile - 1) / kTile);
    // Short images whose one-strip-per-image blocks alone exceed two rounds
    // of the CUs run as one sequence of Ho + R - 1 rows per image (the R - 1
    // extra output rows read zero dY), so that a strip spans several images:
    // a strip of one small image writes a whole 64 x 64*R*S partial for a
    // few rows of work (7x7 at 512 channels: 604 MB of partials). Offsets
    // then span the whole batch: it must fit a buffer resource.
    const int ncu = device_cus();
    a.vP = 0;
    a.vrows = 0;
    if (Ho <= 32 && (int64_t)B * a.ncol * ntiles > 2 * ncu &&
        (int64_t)B * C * H * W * 4 < kMaxTileSpanBytes &&
        (int64_t)B * F * Ho * Wo * 4 < kMaxTileSpanBytes) {
        a.vP = Ho + R - 1;
        a.vrows = B * a.vP;
    }
    const int rows = a.vP ? a.vrows : Ho;     // rows a strip is cut from
    const int64_t seqs = a.vP ? 1 : B;        // row sequences
    // Strip length: fewest rounds of one block per CU, each about (steps + 2)
    // step times (the first rows arrive unhidden).
    double best = 1e30;
    for (int L = kG; L < rows + kG; L += kG) {
        const int64_t blocks = seqs * ((rows + L - 1) / L) * a.ncol * ntiles;
        const double cost = (double)((blocks + ncu - 1) / ncu) * ((L + kG - 1) / kG + 2);
        if (cost < best) { best = cost; a.L = L; }
    }
    a.nstrip = (rows + a.L - 1) / a.L;
    if (seqs * a.nstrip * a.ncol > 0x7fffffff) return SEERA_OK;
    a.nsplit = (int)(seqs * a.nstrip * a.ncol);
    // The kernel's producers reuse the rings for the bias-gradient reduction.
    if (with_db && kProd * kDI * 4 > a.lds_bytes) return SEERA_OK;
    const int nftile = (F + kTile - 1) / kTile;
    const size_t part_n = (size_t)ntiles * a.nsplit * 64 * kTile * R * S;
    const size_t db_n = with_db ? (size_t)nftile * a.nsplit * kTile : 0;
    void* ws = nullptr;
    SEERA_TRY(workspace(sizeof(float) * (part_n + db_n), &ws, st));
    a.part = static_cast<float*>(ws);
    a.dbpart = with_db ? a.part + part_n : nullptr;
    hipError_t e;
    switch (R) {
        case 1: e = launch_rr<1>(a, ntiles, st); break;
        case 2: e = launch_rr<2>(a, ntiles, st); break;
        default: e = launch_rr<3>(a, ntiles, st); break;
    }
    if (e != hipSuccess) return fail_hip(e, "stream wgrad launch");
    out->part = a.part;
    out->dbpart = a.dbpart;
    out->CT = kTile;
    out->nctile = a.nctile;
    out->ntiles = ntiles;
    out->nsplit = a.nsplit;
    *used = true;
    return SEERA_OK;
}

}  // namespace seera
