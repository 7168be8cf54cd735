// Submanifold 3x3x3 convolution: one fused gather-GEMM kernel per conv.
//
// Replaces sparse_submconv / submconv_range (src/sparse.cpp:61-92). The reference builds, per
// tap, a materialised get_rows gather of the zero-padded input, a mul_mat with W_t and an add
// into the accumulator (27 x 3 graph nodes, sparse.cpp:68-77). Here every output voxel tile
// keeps its accumulator in registers for all 27 taps; the gather reads input rows straight
// from HBM/L2 by the neighbour table, absent taps (table value N) contribute nothing, and the
// bias is added in the epilogue. Nothing is materialised.
//
// Three kernels:
//   * k_conv_halo (conv_halo.hip) -- the MFMA kernel: bf16/fp16 features and weights, fp32
//                     accumulation, each tile's distinct neighbour rows staged in LDS.
//   * k_conv_mfma  -- MFMA kernel that gathers straight from L2/HBM: a workgroup owns 64*WAVES
//                     output voxels x BN output channels; each wave owns 64 voxels x BN
//                     channels. The weight slice of the current (tap, 32-channel chunk) is
//                     staged in LDS (double-buffered) and shared by all waves; each wave
//                     gathers its own neighbour rows straight into MFMA operand registers,
//                     prefetching the next chunk while the current one multiplies.
//   * k_conv_narrow -- VALU fp32 FMA, any dtype mix and any channel count. LDS-tiled 64 voxels
//                     x 64 channels, each thread a 4x4 register block.
// The entry point also dispatches to the thin kernels (conv_thin.hip, conv_thin_mfma.hip) and the
// fp32 matrix-core kernel (conv_f32_mfma.hip), which AUTO takes for f32 features and weights with
// Ci % 16 == 0 and Co % 32 == 0 before falling back to k_conv_narrow.
#include <algorithm>

#include "conv_internal.hpp"

namespace tsp {
namespace {

// ---------------------------------------------------------------------------------------------
// VALU kernel
// ---------------------------------------------------------------------------------------------
constexpr int NB_M = 64, NB_N = 64, NB_K = 32, NB_THREADS = 256;

// taps = 27 with a neighbour table is the conv; taps = 1 with nbr == nullptr (row i reads row
// i) is a dense linear layer, weight [co][ci]. bias may be null.
//
// KG tap groups of NB_THREADS threads each: in round r, group g runs tap KG r + g of the tile
// (with its own staging), and at the end the groups' partial sums are added in group order
// through LDS -- a deterministic order. KG > 1 serves grids too small to fill the device (the
// tile count is fixed by the voxels): KG times the waves on the same tiles, each with 1/KG of
// the taps to walk.
template <int FDT, int WDT, int ODT, int KG>
__global__ __launch_bounds__(NB_THREADS * KG) void k_conv_narrow(
    const typename Elem<FDT>::storage* __restrict__ feats, int64_t n, int ci,
    const int32_t* __restrict__ nbr, int taps,
    const typename Elem<WDT>::storage* __restrict__ weight, const float* __restrict__ bias,
    int co, typename Elem<ODT>::storage* __restrict__ out, PadRow pad) {
    struct Stage {
        float a[NB_K][NB_M + 4];
        float b[NB_K][NB_N + 4];
        int32_t row[NB_M];
    };
    static_assert(KG == 1 || (KG - 1) * NB_M * NB_N * 4 <= KG * (int)sizeof(Stage), "partials fit the staging");
    __shared__ __attribute__((aligned(16))) Stage sStage[KG];

    const int gid = threadIdx.x / NB_THREADS;      // tap group
    const int tid = threadIdx.x % NB_THREADS;
    float (*sA)[NB_M + 4] = sStage[gid].a;
    float (*sB)[NB_N + 4] = sStage[gid].b;
    int32_t* sRow = sStage[gid].row;
    const int ty = tid / 16, tx = tid % 16;
    const int64_t row0 = (int64_t)blockIdx.x * NB_M;
    const int co0 = blockIdx.y * NB_N;
    const int32_t sentinel = (int32_t)n;
    // whether the padding row 0 * feats[0] (sparse.cpp:81-85) holds a NaN: then no tap is skipped
    // (an exact zero padding row, pad.zero, never does; with pad.row0 that f32 row is the source)
    bool row0_bad = false;
    if (nbr && !pad.zero)
        for (int k = threadIdx.x; k < ci; k += NB_THREADS * KG)
            row0_bad |= !__builtin_isfinite(pad.row0 ? pad.row0[k] : Elem<FDT>::load(feats, k));
    row0_bad = __syncthreads_or(row0_bad);

    float acc[4][4];
#pragma unroll
    for (int a = 0; a < 4; ++a)
#pragma unroll
        for (int b = 0; b < 4; ++b) acc[a][b] = 0.f;

    for (int t0 = 0; t0 < taps; t0 += KG) {
        const int t = t0 + gid;          // this group's tap; past the last one, a group adds nothing
        const bool real = t < taps;
        int valid = 0;
        if (tid < NB_M) {
            const int64_t i = row0 + tid;
            const int32_t r = (real && i < n) ? (nbr ? nbr[(int64_t)t * n + i] : (int32_t)i) : sentinel;
            sRow[tid] = r;
            valid = real && r != sentinel;
        }
        // no voxel of the tile has these neighbours: skipped, unless the padding row is not zero
        if (!__syncthreads_or(valid) && !row0_bad) continue;

        for (int kc = 0; kc < ci; kc += NB_K) {
            {   // gathered input rows -> sA[k][row]
                const int r = tid / 4, kk = (tid % 4) * 8;
                const int32_t src = sRow[r];
#pragma unroll
                for (int j = 0; j < 8; ++j) {
                    const int k = kc + kk + j;
                    float v = 0.f;
                    // unsigned compare: the sentinel N (and any value outside [0,N)) reads the
                    // padding row 0 * feats[0] (sparse.cpp:81-85)
                    if (k < ci && real) {
                        if ((uint32_t)src < (uint32_t)n) v = Elem<FDT>::load(feats, (int64_t)src * ci + k);
                        else if (row0_bad) v = 0.f * (pad.row0 ? pad.row0[k] : Elem<FDT>::load(feats, k));
                    }
                    sA[kk + j][r] = v;
                }
            }
            {   // W[co][t][k] -> sB[k][co]
                const int c = tid / 4, kk = (tid % 4) * 8;
                const int oc = co0 + c;
#pragma unroll
                for (int j = 0; j < 8; ++j) {
                    const int k = kc + kk + j;
                    float v = 0.f;
                    if (oc < co && k < ci && real)
                        v = Elem<WDT>::load(weight, ((int64_t)oc * taps + t) * ci + k);
                    sB[kk + j][c] = v;
                }
            }
            __syncthreads();
#pragma unroll 8
            for (int k = 0; k < NB_K; ++k) {
                const float4 a = *reinterpret_cast<const float4*>(&sA[k][ty * 4]);
                const float4 b = *reinterpret_cast<const float4*>(&sB[k][tx * 4]);
                const float av[4] = {a.x, a.y, a.z, a.w};
                const float bv[4] = {b.x, b.y, b.z, b.w};
#pragma unroll
                for (int p = 0; p < 4; ++p)
#pragma unroll
                    for (int q = 0; q < 4; ++q) acc[p][q] = fmaf(av[p], bv[q], acc[p][q]);
            }
            __syncthreads();
        }
    }

    if constexpr (KG > 1) {
        // groups 1.. KG-1 leave their partial sums in LDS; group 0 adds them in group order
        float* part = reinterpret_cast<float*>(&sStage[0]);
        if (gid > 0) {
#pragma unroll
            for (int p = 0; p < 4; ++p)
#pragma unroll
                for (int q = 0; q < 4; ++q)
                    part[((gid - 1) * NB_M + ty * 4 + p) * NB_N + tx * 4 + q] = acc[p][q];
        }
        __syncthreads();
        if (gid != 0) return;
#pragma unroll
        for (int g = 1; g < KG; ++g)
#pragma unroll
            for (int p = 0; p < 4; ++p)
#pragma unroll
                for (int q = 0; q < 4; ++q) acc[p][q] += part[((g - 1) * NB_M + ty * 4 + p) * NB_N + tx * 4 + q];
    }
#pragma unroll
    for (int p = 0; p < 4; ++p) {
        const int64_t i = row0 + ty * 4 + p;
        if (i >= n) continue;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const int oc = co0 + tx * 4 + q;
            if (oc < co) Elem<ODT>::store(out, i * co + oc, acc[p][q] + (bias ? bias[oc] : 0.f));
        }
    }
}

// ---------------------------------------------------------------------------------------------
// MFMA kernel gathering from L2/HBM
// ---------------------------------------------------------------------------------------------
constexpr int MK = 32;            // channels per pipeline stage
constexpr int MPAD = 8;           // LDS row padding (elements) of the staged weight slice

template <bool BF16, int BN, int WAVES, int ODT>
__global__ __launch_bounds__(WAVES * 64) void k_conv_mfma(
    const uint16_t* __restrict__ feats, int64_t n, int ci, const int32_t* __restrict__ nbr,
    const uint16_t* __restrict__ weight, const float* __restrict__ bias, int co,
    void* __restrict__ out, int64_t n_tiles, int n_ctiles, int64_t per_xcd, int taps, PadRow pad) {
    constexpr int NT = WAVES * 64;
    constexpr int BM = 64 * WAVES;
    constexpr int CB = BN / 32;                       // 32-wide column blocks per wave
    constexpr int PIECES = BN * (MK / 8);             // 16-byte pieces of one weight stage
    constexpr int PPT = (PIECES + NT - 1) / NT;       // pieces per thread
    static_assert(PIECES % NT == 0 || PIECES < NT, "weight stage must split evenly");

    __shared__ __attribute__((aligned(16))) uint16_t sB[2][BN][MK + MPAD];
    __shared__ uint32_t sMask;
    __shared__ int8_t sTaps[kTaps];
    __shared__ int sNTaps;

    // XCD-aware tile order: consecutive workgroup ids go round-robin over the 8 XCDs, so give
    // each XCD one contiguous range of (tile, column-tile) pairs; neighbouring tiles then
    // gather from rows already resident in that XCD's L2.
    const int64_t b = blockIdx.x;
    const int64_t lin = (b % 8) * per_xcd + b / 8;
    if (lin >= n_tiles * n_ctiles) return;
    const int64_t tile = lin / n_ctiles;
    const int co0 = (int)(lin % n_ctiles) * BN;

    const int tid = threadIdx.x;
    const int wave = tid / 64, lane = tid % 64;
    const int lr = lane & 31, g = lane >> 5;
    const int64_t wrow0 = tile * BM + (int64_t)wave * 64;   // this wave's first voxel
    const int32_t sentinel = (int32_t)n;

    // Taps that some voxel of the workgroup has (wave ballots, OR in LDS). Absent taps read the
    // padding row 0 * feats[0] (sparse.cpp:81-85): zeros, unless row 0 holds an Inf or a NaN --
    // then every tap counts, as the padding row makes the sums of absent taps NaN. An exact zero
    // padding row (pad.zero) reads zeros; with pad.row0 the padding row is 0 * that f32 row,
    // rounded (a NaN where it is not finite, else 0).
    if (tid == 0) sMask = 0;
    bool row0_bad = false;
    if (!pad.zero) {
        if (pad.row0) {
            for (int k = tid; k < ci; k += NT) row0_bad |= !__builtin_isfinite(pad.row0[k]);
        } else {
            for (int k = tid * 8; k < ci; k += NT * 8) {
                const u32x4_t v = *reinterpret_cast<const u32x4_t*>(feats + k);
                const u32x4_t z = zero_times16<BF16>(v);
#pragma unroll
                for (int e = 0; e < 4; ++e) row0_bad |= (z[e] & 0x7fff7fffu) != 0;
            }
        }
    }
    row0_bad = __syncthreads_or(row0_bad);
    {
        uint32_t wm = 0;
        const int64_t i = wrow0 + lane;
        for (int t = 0; t < taps; ++t) {
            const bool v = (i < n) && (row0_bad || !nbr || nbr[(int64_t)t * n + i] != sentinel);
            if (__ballot(v)) wm |= 1u << t;
        }
        if (lane == 0 && wm) atomicOr(&sMask, wm);
    }
    __syncthreads();
    if (tid == 0) {
        uint32_t m = sMask;
        int k = 0;
        while (m) {
            const int t = __builtin_ctz(m);
            sTaps[k++] = (int8_t)t;
            m &= m - 1;
        }
        sNTaps = k;
    }
    __syncthreads();
    const int ntaps = sNTaps;
    const int nkc = ci / MK;
    const int iters = ntaps * nkc;

    f32x16_t acc[2][CB];
#pragma unroll
    for (int rb = 0; rb < 2; ++rb)
#pragma unroll
        for (int cb = 0; cb < CB; ++cb)
#pragma unroll
            for (int j = 0; j < 16; ++j) acc[rb][cb][j] = 0.f;

    if (iters == 0) goto epilogue;
    {
        // neighbour rows of this wave for the current tap: lanes l and l+32 share row l%32
        int32_t rowsA[2];
        auto load_rows = [&](int t, int32_t* r) {
#pragma unroll
            for (int rb = 0; rb < 2; ++rb) {
                const int64_t i = wrow0 + rb * 32 + lr;
                r[rb] = (i < n) ? (nbr ? nbr[(int64_t)t * n + i] : (int32_t)i) : sentinel;
            }
        };
        auto load_a = [&](const int32_t* r, int kc, u32x4_t (*a)[2]) {
#pragma unroll
            for (int rb = 0; rb < 2; ++rb)
#pragma unroll
                for (int s = 0; s < 2; ++s) {
                    if ((uint32_t)r[rb] < (uint32_t)n) {   // sentinel N -> the padding row
                        a[rb][s] = *reinterpret_cast<const u32x4_t*>(
                            feats + (int64_t)r[rb] * ci + kc + s * 16 + g * 8);
                    } else if (pad.zero || !row0_bad) {
                        a[rb][s] = u32x4_t{0, 0, 0, 0};
                    } else if (pad.row0) {
                        // 16-bit NaN where the f32 source is not finite (either type's quiet NaN
                        // pattern 0x7FC0 / 0x7E00), zero elsewhere
                        constexpr uint32_t kNaN = BF16 ? 0x7FC0u : 0x7E00u;
                        u32x4_t z;
#pragma unroll
                        for (int e = 0; e < 4; ++e) {
                            const int k = kc + s * 16 + g * 8 + 2 * e;
                            z[e] = (__builtin_isfinite(pad.row0[k]) ? 0u : kNaN) |
                                   ((__builtin_isfinite(pad.row0[k + 1]) ? 0u : kNaN) << 16);
                        }
                        a[rb][s] = z;
                    } else {
                        a[rb][s] = zero_times16<BF16>(
                            *reinterpret_cast<const u32x4_t*>(feats + kc + s * 16 + g * 8));
                    }
                }
        };
        auto load_b = [&](int t, int kc, u32x4_t* regs) {
#pragma unroll
            for (int p = 0; p < PPT; ++p) {
                const int piece = tid + p * NT;
                if (piece < PIECES) {
                    const int c = piece / (MK / 8), kq = piece % (MK / 8);
                    regs[p] = *reinterpret_cast<const u32x4_t*>(
                        weight + ((int64_t)(co0 + c) * taps + t) * ci + kc + kq * 8);
                }
            }
        };
        auto store_b = [&](int buf, const u32x4_t* regs) {
#pragma unroll
            for (int p = 0; p < PPT; ++p) {
                const int piece = tid + p * NT;
                if (piece < PIECES) {
                    const int c = piece / (MK / 8), kq = piece % (MK / 8);
                    *reinterpret_cast<u32x4_t*>(&sB[buf][c][kq * 8]) = regs[p];
                }
            }
        };

        u32x4_t aCur[2][2], aNext[2][2];
        u32x4_t bRegs[PPT];
        int t = sTaps[0];
        load_rows(t, rowsA);
        load_a(rowsA, 0, aCur);
        load_b(t, 0, bRegs);
        store_b(0, bRegs);
        __syncthreads();

        for (int it = 0; it < iters; ++it) {
            const int buf = it & 1;
            const bool more = it + 1 < iters;
            if (more) {
                const int nt = sTaps[(it + 1) / nkc];
                const int nkcoff = ((it + 1) % nkc) * MK;
                if (nkcoff == 0) load_rows(nt, rowsA);
                load_a(rowsA, nkcoff, aNext);
                load_b(nt, nkcoff, bRegs);
            }
#pragma unroll
            for (int s = 0; s < 2; ++s) {
#pragma unroll
                for (int cb = 0; cb < CB; ++cb) {
                    const u32x4_t bf =
                        *reinterpret_cast<const u32x4_t*>(&sB[buf][cb * 32 + lr][s * 16 + g * 8]);
#pragma unroll
                    for (int rb = 0; rb < 2; ++rb)
                        acc[rb][cb] = mfma32x32x16<BF16>(aCur[rb][s], bf, acc[rb][cb]);
                }
            }
            if (more) {
                store_b(buf ^ 1, bRegs);
#pragma unroll
                for (int rb = 0; rb < 2; ++rb)
#pragma unroll
                    for (int s = 0; s < 2; ++s) aCur[rb][s] = aNext[rb][s];
            }
            __syncthreads();
        }
    }

epilogue:
#pragma unroll
    for (int cb = 0; cb < CB; ++cb) {
        const int oc = co0 + cb * 32 + lr;
        const float bv = bias ? bias[oc] : 0.f;
#pragma unroll
        for (int rb = 0; rb < 2; ++rb)
#pragma unroll
            for (int j = 0; j < 16; ++j) {
                const int64_t i = wrow0 + rb * 32 + 8 * (j / 4) + 4 * g + (j % 4);
                if (i < n) store_out<ODT>(out, i * co + oc, acc[rb][cb][j] + bv);
            }
    }
}


// ---------------------------------------------------------------------------------------------
// Dispatch
// ---------------------------------------------------------------------------------------------
template <int FDT, int WDT, int ODT>
int launch_narrow(const void* feats, int64_t n, int ci, const int32_t* nbr, const void* weight,
                  const float* bias, int co, void* out, hipStream_t s, PadRow pad) {
    dim3 grid((unsigned)ceil_div(n, NB_M), (unsigned)ceil_div(co, NB_N));
    const auto* f = reinterpret_cast<const typename Elem<FDT>::storage*>(feats);
    const auto* w = reinterpret_cast<const typename Elem<WDT>::storage*>(weight);
    auto* o = reinterpret_cast<typename Elem<ODT>::storage*>(out);
    // a conv whose tiles leave most of the device idle (fewer than two a CU, e.g. the 64^3 shell
    // of ~15K voxels) splits each tile's taps over four groups of threads
    int cus = 0, dev = 0;
    if (hipGetDevice(&dev) != hipSuccess ||
        hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0)
        cus = 256;
    if (nbr && (int64_t)grid.x * grid.y < 2 * (int64_t)cus)
        hipLaunchKernelGGL((k_conv_narrow<FDT, WDT, ODT, 4>), grid, dim3(NB_THREADS * 4), 0, s, f, n, ci, nbr, kTaps,
                           w, bias, co, o, pad);
    else
        hipLaunchKernelGGL((k_conv_narrow<FDT, WDT, ODT, 1>), grid, dim3(NB_THREADS), 0, s, f, n, ci, nbr,
                           nbr ? kTaps : 1, w, bias, co, o, pad);
    TSP_CHECK_LAUNCH();
    return TSP_OK;
}

template <int FDT, int WDT>
int narrow_out(int odt, const void* feats, int64_t n, int ci, const int32_t* nbr,
               const void* weight, const float* bias, int co, void* out, hipStream_t s, PadRow pad) {
    switch (odt) {
        case TSP_F32: return launch_narrow<FDT, WDT, TSP_F32>(feats, n, ci, nbr, weight, bias, co, out, s, pad);
        case TSP_F16: return launch_narrow<FDT, WDT, TSP_F16>(feats, n, ci, nbr, weight, bias, co, out, s, pad);
        case TSP_BF16: return launch_narrow<FDT, WDT, TSP_BF16>(feats, n, ci, nbr, weight, bias, co, out, s, pad);
    }
    set_error("tsp_subm_conv3x3: bad out dtype %d", odt);
    return TSP_ERR_INVALID;
}

int dispatch_narrow(int fdt, int wdt, int odt, const void* feats, int64_t n, int ci,
                    const int32_t* nbr, const void* weight, const float* bias, int co, void* out,
                    hipStream_t s, PadRow pad = {}) {
    if (fdt == TSP_F32 && wdt == TSP_F32) return narrow_out<TSP_F32, TSP_F32>(odt, feats, n, ci, nbr, weight, bias, co, out, s, pad);
    if (fdt == TSP_F32 && wdt == TSP_F16) return narrow_out<TSP_F32, TSP_F16>(odt, feats, n, ci, nbr, weight, bias, co, out, s, pad);
    if (fdt == TSP_F32 && wdt == TSP_BF16) return narrow_out<TSP_F32, TSP_BF16>(odt, feats, n, ci, nbr, weight, bias, co, out, s, pad);
    if (fdt == TSP_F16 && wdt == TSP_F16) return narrow_out<TSP_F16, TSP_F16>(odt, feats, n, ci, nbr, weight, bias, co, out, s, pad);
    if (fdt == TSP_BF16 && wdt == TSP_BF16) return narrow_out<TSP_BF16, TSP_BF16>(odt, feats, n, ci, nbr, weight, bias, co, out, s, pad);
    set_error("tsp_subm_conv3x3: unsupported dtype pair feats=%d weight=%d", fdt, wdt);
    return TSP_ERR_UNSUPPORTED;
}

template <bool BF16, int BN, int WAVES, int ODT>
int launch_gather(const void* feats, int64_t n, int ci, const int32_t* nbr, int taps,
                  const void* weight, const float* bias, int co, void* out, hipStream_t s, PadRow pad) {
    constexpr int BM = 64 * WAVES;
    const int64_t n_tiles = ceil_div(n, BM);
    const int n_ctiles = co / BN;
    const int64_t total = n_tiles * n_ctiles;
    const int64_t per_xcd = ceil_div(total, 8);
    hipLaunchKernelGGL((k_conv_mfma<BF16, BN, WAVES, ODT>), dim3((unsigned)(per_xcd * 8)),
                       dim3(WAVES * 64), 0, s, reinterpret_cast<const uint16_t*>(feats), n, ci,
                       nbr, reinterpret_cast<const uint16_t*>(weight), bias, co, out, n_tiles,
                       n_ctiles, per_xcd, taps, pad);
    TSP_CHECK_LAUNCH();
    return TSP_OK;
}

template <bool BF16, int BN>
int gather_out(int odt, const void* feats, int64_t n, int ci, const int32_t* nbr, int taps,
               const void* weight, const float* bias, int co, void* out, hipStream_t s, PadRow pad) {
    if (odt == TSP_F32) return launch_gather<BF16, BN, 4, TSP_F32>(feats, n, ci, nbr, taps, weight, bias, co, out, s, pad);
    if (BF16 && odt == TSP_BF16) return launch_gather<BF16, BN, 4, TSP_BF16>(feats, n, ci, nbr, taps, weight, bias, co, out, s, pad);
    if (!BF16 && odt == TSP_F16) return launch_gather<BF16, BN, 4, TSP_F16>(feats, n, ci, nbr, taps, weight, bias, co, out, s, pad);
    set_error("tsp_subm_conv3x3: MFMA path writes f32 or the feature dtype, not %d", odt);
    return TSP_ERR_UNSUPPORTED;
}

// taps = 27 with a neighbour table is the conv; taps = 1 with nbr == nullptr (row i reads row i)
// is a linear layer.
int dispatch_gather(int fdt, int odt, const void* feats, int64_t n, int ci, const int32_t* nbr,
                    int taps, const void* weight, const float* bias, int co, void* out,
                    hipStream_t s, PadRow pad = {}) {
    const bool bn128 = co % 128 == 0;
    if (fdt == TSP_BF16)
        return bn128 ? gather_out<true, 128>(odt, feats, n, ci, nbr, taps, weight, bias, co, out, s, pad)
                     : gather_out<true, 64>(odt, feats, n, ci, nbr, taps, weight, bias, co, out, s, pad);
    return bn128 ? gather_out<false, 128>(odt, feats, n, ci, nbr, taps, weight, bias, co, out, s, pad)
                 : gather_out<false, 64>(odt, feats, n, ci, nbr, taps, weight, bias, co, out, s, pad);
}

// MFMA kernels: 16-bit feats and weights of one dtype, out f32 or that dtype, ci % 32 == 0,
// co % 64 == 0, 16-byte aligned operands, and a weight below 4 GiB (32-bit offsets).
bool mfma_eligible(int fdt, int wdt, int odt, int ci, int co, const void* f, const void* w,
                   const void* o) {
    if (fdt != wdt || fdt == TSP_F32) return false;
    if (odt != TSP_F32 && odt != fdt) return false;
    if (reinterpret_cast<uintptr_t>(f) % 16 || reinterpret_cast<uintptr_t>(w) % 16 ||
        reinterpret_cast<uintptr_t>(o) % 16)
        return false;
    return ci % MK == 0 && co % 64 == 0 && (int64_t)kTaps * ci * co * 2 < ((int64_t)1 << 32);
}

}  // namespace
}  // namespace tsp

using namespace tsp;

#define TSP_CONV_COMMON_CHECKS(fn)                                                             \
    TSP_REQUIRE(n >= 0 && n < (int64_t)INT32_MAX, TSP_ERR_INVALID, fn ": n=%lld out of range", \
                (long long)n);                                                                \
    TSP_REQUIRE(ci > 0 && co > 0, TSP_ERR_INVALID, fn ": ci=%d co=%d", ci, co);               \
    TSP_REQUIRE((int64_t)ci * kTaps * co < (int64_t)1 << 40, TSP_ERR_INVALID,                 \
                fn ": weight too large")

extern "C" int tsp_subm_conv3x3_ex(const void* d_feats, int feat_dtype, int64_t n, int ci,
                                   const int32_t* d_nbr, const void* d_weight, int weight_dtype,
                                   const float* d_bias, int co, void* d_out, int out_dtype, int algo,
                                   int flags, const float* d_row0, void* stream) {
    clear_error();
    TSP_CONV_COMMON_CHECKS("tsp_subm_conv3x3");
    TSP_REQUIRE(dtype_valid(feat_dtype) && dtype_valid(weight_dtype) && dtype_valid(out_dtype),
                TSP_ERR_INVALID, "tsp_subm_conv3x3: bad dtype");
    TSP_REQUIRE(algo >= TSP_ALGO_AUTO && algo <= TSP_ALGO_F32_MFMA, TSP_ERR_INVALID,
                "tsp_subm_conv3x3: bad algo %d", algo);
    TSP_REQUIRE((flags & ~TSP_CONV_ZERO_PAD) == 0, TSP_ERR_INVALID, "tsp_subm_conv3x3: bad flags %d",
                flags);
    if (n == 0) return TSP_OK;
    TSP_REQUIRE(d_feats && d_nbr && d_weight && d_bias && d_out, TSP_ERR_INVALID,
                "tsp_subm_conv3x3: null pointer");
    TSP_REQUIRE(d_out != d_feats, TSP_ERR_INVALID, "tsp_subm_conv3x3: out aliases feats");
    hipStream_t s = as_stream(stream);
    PadRow pad;
    pad.zero = (flags & TSP_CONV_ZERO_PAD) != 0;
    pad.row0 = pad.zero ? nullptr : d_row0;
    const bool eligible =
        mfma_eligible(feat_dtype, weight_dtype, out_dtype, ci, co, d_feats, d_weight, d_out);
    if (algo == TSP_ALGO_MFMA || algo == TSP_ALGO_MFMA_GATHER) {
        TSP_REQUIRE(eligible, TSP_ERR_UNSUPPORTED,
                    "tsp_subm_conv3x3: MFMA path needs f16/bf16 feats and weights of one dtype, "
                    "16-byte aligned buffers, ci %% 32 == 0 and co %% 64 == 0 (got ci=%d co=%d)",
                    ci, co);
    }
    if (algo == TSP_ALGO_MFMA_GATHER)
        return dispatch_gather(feat_dtype, out_dtype, d_feats, n, ci, d_nbr, kTaps, d_weight,
                               d_bias, co, d_out, s, pad);
    if (algo == TSP_ALGO_AUTO && eligible && !halo_fits(n, ci))
        return dispatch_gather(feat_dtype, out_dtype, d_feats, n, ci, d_nbr, kTaps, d_weight,
                               d_bias, co, d_out, s, pad);
    if (algo == TSP_ALGO_MFMA || (algo == TSP_ALGO_AUTO && eligible))
        return halo_conv_launch(feat_dtype, out_dtype, d_feats, n, ci, d_nbr, nullptr, d_weight,
                                d_bias, co, d_out, s, OctantScatter{}, SkipAdd{}, pad);
    if (algo == TSP_ALGO_THIN_MFMA || algo == TSP_ALGO_AUTO) {
        const int st = thin_mfma_launch(feat_dtype, weight_dtype, out_dtype, d_feats, n, ci, d_nbr, d_weight,
                                        d_bias, co, d_out, s, pad);
        if (st != TSP_ERR_UNSUPPORTED || algo == TSP_ALGO_THIN_MFMA) {
            TSP_REQUIRE(st != TSP_ERR_UNSUPPORTED, TSP_ERR_UNSUPPORTED,
                        "tsp_subm_conv3x3: the thin matrix-core kernel needs f16/bf16 feats and weights of "
                        "one dtype, ci in {8, 16, 32}, co in {4, 8, 16, 32}, ci * co <= 512, out f32 or the "
                        "feats' dtype and 16-byte aligned feats and weights (got ci=%d co=%d)", ci, co);
            return st;
        }
    }
    if (algo == TSP_ALGO_THIN || algo == TSP_ALGO_AUTO) {
        const int st = thin_conv_launch(feat_dtype, weight_dtype, out_dtype, d_feats, n, ci, d_nbr, d_weight,
                                        d_bias, co, d_out, s, pad);
        if (st != TSP_ERR_UNSUPPORTED || algo == TSP_ALGO_THIN) {
            TSP_REQUIRE(st != TSP_ERR_UNSUPPORTED, TSP_ERR_UNSUPPORTED,
                        "tsp_subm_conv3x3: the thin kernel needs co in {4, 8, 16, 32}, ci %% 4 == 0, "
                        "ci * co <= 512, n * ci < 2^32, 16-byte aligned feats and a dtype pair of the "
                        "VALU kernel (got ci=%d co=%d)", ci, co);
            return st;
        }
    }
    if (algo == TSP_ALGO_F32_MFMA || algo == TSP_ALGO_AUTO) {
        const int st = f32_mfma_launch(feat_dtype, weight_dtype, out_dtype, d_feats, n, ci, d_nbr, d_weight, d_bias,
                                       co, d_out, s, pad);
        if (st != TSP_ERR_UNSUPPORTED || algo == TSP_ALGO_F32_MFMA) {
            TSP_REQUIRE(st != TSP_ERR_UNSUPPORTED, TSP_ERR_UNSUPPORTED,
                        "tsp_subm_conv3x3: the fp32 matrix-core kernel needs f32 feats and weights, ci %% 16 == 0, "
                        "co %% 32 == 0 and 16-byte aligned feats and weights (got ci=%d co=%d)", ci, co);
            return st;
        }
    }
    return dispatch_narrow(feat_dtype, weight_dtype, out_dtype, d_feats, n, ci, d_nbr, d_weight,
                           d_bias, co, d_out, s, pad);
}

extern "C" int tsp_subm_conv3x3(const void* d_feats, int feat_dtype, int64_t n, int ci,
                                const int32_t* d_nbr, const void* d_weight, int weight_dtype,
                                const float* d_bias, int co, void* d_out, int out_dtype, int algo,
                                void* stream) {
    return tsp_subm_conv3x3_ex(d_feats, feat_dtype, n, ci, d_nbr, d_weight, weight_dtype, d_bias, co,
                               d_out, out_dtype, algo, 0, nullptr, stream);
}

extern "C" size_t tsp_conv_plan_bytes(int64_t n) { return n < 0 ? 0 : halo_plan_bytes(n); }

static int plan_build_checked(const char* fn, const int32_t* d_nbr, const int32_t* d_coords, int64_t n,
                              void* d_plan, size_t plan_bytes, void* stream) {
    clear_error();
    TSP_REQUIRE(n >= 0 && n < (int64_t)INT32_MAX, TSP_ERR_INVALID, "%s: n=%lld out of range", fn,
                (long long)n);
    if (n == 0) return TSP_OK;
    TSP_REQUIRE(d_nbr && d_plan, TSP_ERR_INVALID, "%s: null pointer", fn);
    TSP_REQUIRE(plan_bytes >= halo_plan_bytes(n), TSP_ERR_WORKSPACE, "%s: plan buffer %zu < %zu bytes", fn,
                plan_bytes, halo_plan_bytes(n));
    TSP_REQUIRE((reinterpret_cast<uintptr_t>(d_plan) & 15) == 0, TSP_ERR_INVALID,
                "%s: the plan buffer must be 16-byte aligned", fn);
    return halo_plan_build(d_nbr, d_coords, n, d_plan, as_stream(stream));
}

extern "C" int tsp_conv_plan_build(const int32_t* d_nbr, int64_t n, void* d_plan,
                                   size_t plan_bytes, void* stream) {
    return plan_build_checked("tsp_conv_plan_build", d_nbr, nullptr, n, d_plan, plan_bytes, stream);
}

extern "C" int tsp_conv_plan_build_ordered(const int32_t* d_nbr, const int32_t* d_coords, int64_t n,
                                           void* d_plan, size_t plan_bytes, void* stream) {
    if (!d_coords && n > 0) {
        clear_error();
        set_error("tsp_conv_plan_build_ordered: null coordinates");
        return TSP_ERR_INVALID;
    }
    return plan_build_checked("tsp_conv_plan_build_ordered", d_nbr, d_coords, n, d_plan, plan_bytes, stream);
}

extern "C" int tsp_conv_weight_pack(const void* d_weight, int dtype, int ci, int co,
                                    void* d_packed, void* stream) {
    clear_error();
    TSP_REQUIRE(dtype == TSP_F16 || dtype == TSP_BF16, TSP_ERR_UNSUPPORTED,
                "tsp_conv_weight_pack: packed weights are f16 or bf16, not dtype %d", dtype);
    TSP_REQUIRE(ci > 0 && co > 0 && ci % 16 == 0 && co % 32 == 0, TSP_ERR_UNSUPPORTED,
                "tsp_conv_weight_pack: needs ci %% 16 == 0 and co %% 32 == 0 (ci=%d co=%d)", ci, co);
    TSP_REQUIRE((int64_t)kTaps * ci * co * 2 < ((int64_t)1 << 32), TSP_ERR_UNSUPPORTED,
                "tsp_conv_weight_pack: weight of 4 GiB or more");
    TSP_REQUIRE(d_weight && d_packed && d_weight != d_packed, TSP_ERR_INVALID,
                "tsp_conv_weight_pack: null or aliased pointer");
    TSP_REQUIRE(reinterpret_cast<uintptr_t>(d_weight) % 16 == 0 &&
                    reinterpret_cast<uintptr_t>(d_packed) % 16 == 0,
                TSP_ERR_INVALID, "tsp_conv_weight_pack: buffers must be 16-byte aligned");
    return halo_weight_pack(d_weight, dtype, ci, co, d_packed, as_stream(stream));
}

extern "C" size_t tsp_conv_weight_packed_bytes(int ci, int co) {
    if (ci <= 0 || co <= 0) return 0;
    return packed_weight_bytes(ci, co);
}

extern "C" int tsp_subm_conv3x3_planned_ex(const void* d_feats, int dtype, int64_t n, int ci,
                                           const int32_t* d_nbr, const void* d_plan,
                                           const void* d_packed_weight, const float* d_bias, int co,
                                           void* d_out, int out_dtype, int flags, const float* d_row0,
                                           void* stream) {
    clear_error();
    TSP_CONV_COMMON_CHECKS("tsp_subm_conv3x3_planned");
    TSP_REQUIRE(dtype == TSP_F16 || dtype == TSP_BF16, TSP_ERR_UNSUPPORTED,
                "tsp_subm_conv3x3_planned: features are f16 or bf16, not dtype %d", dtype);
    TSP_REQUIRE(out_dtype == TSP_F32 || out_dtype == dtype, TSP_ERR_UNSUPPORTED,
                "tsp_subm_conv3x3_planned: out is f32 or the feature dtype");
    TSP_REQUIRE(ci % 16 == 0 && co % 64 == 0, TSP_ERR_UNSUPPORTED,
                "tsp_subm_conv3x3_planned: needs ci %% 16 == 0 and co %% 64 == 0 (ci=%d co=%d)",
                ci, co);
    TSP_REQUIRE((int64_t)kTaps * ci * co * 2 < ((int64_t)1 << 32), TSP_ERR_UNSUPPORTED,
                "tsp_subm_conv3x3_planned: weight of 4 GiB or more");
    TSP_REQUIRE((flags & ~TSP_CONV_ZERO_PAD) == 0, TSP_ERR_INVALID,
                "tsp_subm_conv3x3_planned: bad flags %d", flags);
    if (n == 0) return TSP_OK;
    TSP_REQUIRE(d_feats && d_nbr && d_plan && d_packed_weight && d_bias && d_out,
                TSP_ERR_INVALID, "tsp_subm_conv3x3_planned: null pointer");
    TSP_REQUIRE(d_out != d_feats, TSP_ERR_INVALID, "tsp_subm_conv3x3_planned: out aliases feats");
    TSP_REQUIRE(reinterpret_cast<uintptr_t>(d_feats) % 16 == 0 &&
                    reinterpret_cast<uintptr_t>(d_packed_weight) % 16 == 0 &&
                    reinterpret_cast<uintptr_t>(d_out) % 16 == 0,
                TSP_ERR_INVALID, "tsp_subm_conv3x3_planned: buffers must be 16-byte aligned");
    PadRow pad;
    pad.zero = (flags & TSP_CONV_ZERO_PAD) != 0;
    pad.row0 = d_row0;
    return halo_conv_launch(dtype, out_dtype, d_feats, n, ci, d_nbr, d_plan, d_packed_weight,
                            d_bias, co, d_out, as_stream(stream), OctantScatter{}, SkipAdd{}, pad);
}

extern "C" int tsp_subm_conv3x3_planned(const void* d_feats, int dtype, int64_t n, int ci,
                                        const int32_t* d_nbr, const void* d_plan,
                                        const void* d_packed_weight, const float* d_bias, int co,
                                        void* d_out, int out_dtype, void* stream) {
    return tsp_subm_conv3x3_planned_ex(d_feats, dtype, n, ci, d_nbr, d_plan, d_packed_weight, d_bias,
                                       co, d_out, out_dtype, 0, nullptr, stream);
}

int tsp::planned_octants(const void* d_feats, int dtype, int64_t n, int ci, const int32_t* d_nbr, const void* d_plan,
                         const void* d_packed_weight, const float* d_bias, int cout, const uint8_t* d_mask,
                         const int32_t* d_mstart, float* d_out, const uint32_t* d_blocks, hipStream_t s) {
    TSP_REQUIRE(n >= 0 && n < (int64_t)INT32_MAX && ci > 0 && cout > 0, TSP_ERR_INVALID,
                "tsp_subm_conv3x3_planned_octants: n=%lld ci=%d cout=%d", (long long)n, ci, cout);
    TSP_REQUIRE(dtype == TSP_F16 || dtype == TSP_BF16, TSP_ERR_UNSUPPORTED,
                "tsp_subm_conv3x3_planned_octants: features are f16 or bf16, not dtype %d", dtype);
    TSP_REQUIRE(ci % 16 == 0 && cout % 64 == 0 && cout <= INT32_MAX / 8, TSP_ERR_UNSUPPORTED,
                "tsp_subm_conv3x3_planned_octants: needs ci %% 16 == 0 and cout %% 64 == 0 "
                "(ci=%d cout=%d)", ci, cout);
    const int co = 8 * cout;
    TSP_REQUIRE((int64_t)kTaps * ci * co * 2 < ((int64_t)1 << 32), TSP_ERR_UNSUPPORTED,
                "tsp_subm_conv3x3_planned_octants: weight of 4 GiB or more");
    if (n == 0) return TSP_OK;
    TSP_REQUIRE(d_feats && d_nbr && d_plan && d_packed_weight && d_bias && d_mask && d_mstart && d_out,
                TSP_ERR_INVALID, "tsp_subm_conv3x3_planned_octants: null pointer");
    TSP_REQUIRE(static_cast<const void*>(d_out) != d_feats, TSP_ERR_INVALID,
                "tsp_subm_conv3x3_planned_octants: out aliases feats");
    TSP_REQUIRE(reinterpret_cast<uintptr_t>(d_feats) % 16 == 0 &&
                    reinterpret_cast<uintptr_t>(d_packed_weight) % 16 == 0 &&
                    reinterpret_cast<uintptr_t>(d_out) % 16 == 0 &&
                    reinterpret_cast<uintptr_t>(d_mask) % 8 == 0,
                TSP_ERR_INVALID,
                "tsp_subm_conv3x3_planned_octants: feats, weights and out must be 16-byte aligned, "
                "mask 8-byte aligned");
    OctantScatter osc;
    osc.mask = d_mask;
    osc.mstart = d_mstart;
    osc.cout = cout;
    osc.blocks = d_blocks;
    return halo_conv_launch(dtype, TSP_F32, d_feats, n, ci, d_nbr, d_plan, d_packed_weight, d_bias,
                            co, d_out, s, osc);
}

extern "C" int tsp_subm_conv3x3_planned_octants(const void* d_feats, int dtype, int64_t n, int ci,
                                                const int32_t* d_nbr, const void* d_plan,
                                                const void* d_packed_weight, const float* d_bias,
                                                int cout, const uint8_t* d_mask,
                                                const int32_t* d_mstart, float* d_out,
                                                void* stream) {
    clear_error();
    return planned_octants(d_feats, dtype, n, ci, d_nbr, d_plan, d_packed_weight, d_bias, cout, d_mask, d_mstart,
                           d_out, nullptr, as_stream(stream));
}

int tsp::planned_skip(const void* d_feats, int dtype, int64_t n, int ci, const int32_t* d_nbr, const void* d_plan,
                      const void* d_packed_weight, const float* d_bias, int co, const float* d_x, int cin,
                      const int32_t* d_gidx, float* d_out, void* d_out16, int out16_dtype, hipStream_t s,
                      TileRange tr) {
    TSP_REQUIRE(n >= 0 && n < (int64_t)INT32_MAX && ci > 0 && co > 0 && cin > 0, TSP_ERR_INVALID,
                "tsp_subm_conv3x3_planned_skip: n=%lld ci=%d co=%d cin=%d", (long long)n, ci, co, cin);
    TSP_REQUIRE(dtype == TSP_F16 || dtype == TSP_BF16, TSP_ERR_UNSUPPORTED,
                "tsp_subm_conv3x3_planned_skip: features are f16 or bf16, not dtype %d", dtype);
    TSP_REQUIRE(ci % 16 == 0 && co % 64 == 0, TSP_ERR_UNSUPPORTED,
                "tsp_subm_conv3x3_planned_skip: needs ci %% 16 == 0 and co %% 64 == 0 (ci=%d co=%d)",
                ci, co);
    TSP_REQUIRE(cin % 8 == 0 && co % (cin / 8) == 0 && (co / (cin / 8)) % 4 == 0, TSP_ERR_UNSUPPORTED,
                "tsp_subm_conv3x3_planned_skip: needs cin %% 8 == 0 and co / (cin / 8) a multiple of 4 "
                "(cin=%d co=%d)", cin, co);
    TSP_REQUIRE((int64_t)kTaps * ci * co * 2 < ((int64_t)1 << 32), TSP_ERR_UNSUPPORTED,
                "tsp_subm_conv3x3_planned_skip: weight of 4 GiB or more");
    TSP_REQUIRE(!d_out16 || out16_dtype == TSP_BF16 || out16_dtype == TSP_F16, TSP_ERR_INVALID,
                "tsp_subm_conv3x3_planned_skip: the 16-bit copy is bf16 or f16, not dtype %d", out16_dtype);
    if (n == 0) return TSP_OK;
    TSP_REQUIRE(d_feats && d_nbr && d_plan && d_packed_weight && d_bias && d_x && d_gidx && d_out,
                TSP_ERR_INVALID, "tsp_subm_conv3x3_planned_skip: null pointer");
    TSP_REQUIRE(static_cast<const void*>(d_out) != d_feats && d_out != d_x, TSP_ERR_INVALID,
                "tsp_subm_conv3x3_planned_skip: out aliases feats or x");
    TSP_REQUIRE(reinterpret_cast<uintptr_t>(d_feats) % 16 == 0 &&
                    reinterpret_cast<uintptr_t>(d_packed_weight) % 16 == 0 &&
                    reinterpret_cast<uintptr_t>(d_out) % 16 == 0 && reinterpret_cast<uintptr_t>(d_out16) % 8 == 0,
                TSP_ERR_INVALID, "tsp_subm_conv3x3_planned_skip: buffers must be 16-byte aligned (the 16-bit "
                "copy 8-byte)");
    SkipAdd skip;
    skip.x = d_x;
    skip.gidx = d_gidx;
    skip.cin = cin;
    skip.out16 = d_out16;
    skip.out16_bf16 = out16_dtype == TSP_BF16;
    // the C2S conv2 reads an exact zero padding column (sparse.cpp:289-306)
    PadRow pad;
    pad.zero = true;
    return halo_conv_launch(dtype, TSP_F32, d_feats, n, ci, d_nbr, d_plan, d_packed_weight, d_bias, co,
                            d_out, s, OctantScatter{}, skip, pad, RowNorm{}, tr);
}

extern "C" int tsp_subm_conv3x3_planned_skip(const void* d_feats, int dtype, int64_t n, int ci,
                                             const int32_t* d_nbr, const void* d_plan,
                                             const void* d_packed_weight, const float* d_bias, int co,
                                             const float* d_x, int cin, const int32_t* d_gidx,
                                             float* d_out, void* stream) {
    clear_error();
    return planned_skip(d_feats, dtype, n, ci, d_nbr, d_plan, d_packed_weight, d_bias, co, d_x, cin, d_gidx, d_out,
                        nullptr, TSP_BF16, as_stream(stream));
}

extern "C" int tsp_subm_conv3x3_planned_ln(const void* d_feats, int dtype, int64_t n, int ci,
                                           const int32_t* d_nbr, const void* d_plan,
                                           const void* d_packed_weight, const float* d_bias, int co,
                                           const float* d_norm_weight, const float* d_norm_bias, float eps,
                                           void* d_out, const float* d_row0, void* stream) {
    clear_error();
    TSP_REQUIRE(n >= 0 && n < (int64_t)INT32_MAX && ci > 0 && co > 0, TSP_ERR_INVALID,
                "tsp_subm_conv3x3_planned_ln: n=%lld ci=%d co=%d", (long long)n, ci, co);
    TSP_REQUIRE(dtype == TSP_F16 || dtype == TSP_BF16, TSP_ERR_UNSUPPORTED,
                "tsp_subm_conv3x3_planned_ln: features are f16 or bf16, not dtype %d", dtype);
    TSP_REQUIRE(ci % 16 == 0 && (co == 64 || co == 128), TSP_ERR_UNSUPPORTED,
                "tsp_subm_conv3x3_planned_ln: needs ci %% 16 == 0 and co = 64 or 128 (ci=%d co=%d)", ci, co);
    TSP_REQUIRE(eps >= 0.f, TSP_ERR_INVALID, "tsp_subm_conv3x3_planned_ln: eps < 0");
    if (n == 0) return TSP_OK;
    TSP_REQUIRE(d_feats && d_nbr && d_plan && d_packed_weight && d_bias && d_norm_weight && d_norm_bias && d_out,
                TSP_ERR_INVALID, "tsp_subm_conv3x3_planned_ln: null pointer");
    TSP_REQUIRE(d_out != d_feats, TSP_ERR_INVALID, "tsp_subm_conv3x3_planned_ln: out aliases feats");
    TSP_REQUIRE(reinterpret_cast<uintptr_t>(d_feats) % 16 == 0 &&
                    reinterpret_cast<uintptr_t>(d_packed_weight) % 16 == 0 &&
                    reinterpret_cast<uintptr_t>(d_out) % 16 == 0,
                TSP_ERR_INVALID, "tsp_subm_conv3x3_planned_ln: buffers must be 16-byte aligned");
    TSP_REQUIRE(halo_fits(n, ci), TSP_ERR_UNSUPPORTED,
                "tsp_subm_conv3x3_planned_ln: %lld rows of %d channels exceed 4 GiB of features", (long long)n, ci);
    PadRow pad;
    pad.row0 = d_row0;
    RowNorm ln;
    ln.w = d_norm_weight;
    ln.b = d_norm_bias;
    ln.eps = eps;
    return halo_conv_launch(dtype, dtype, d_feats, n, ci, d_nbr, d_plan, d_packed_weight, d_bias, co, d_out,
                            as_stream(stream), OctantScatter{}, SkipAdd{}, pad, ln);
}

extern "C" int tsp_linear(const void* d_x, int x_dtype, int64_t n, int ci, const void* d_weight,
                          int weight_dtype, const float* d_bias, int co, void* d_out,
                          int out_dtype, void* stream) {
    clear_error();
    TSP_REQUIRE(n >= 0 && ci > 0 && co > 0, TSP_ERR_INVALID, "tsp_linear: n=%lld ci=%d co=%d",
                (long long)n, ci, co);
    TSP_REQUIRE(dtype_valid(x_dtype) && dtype_valid(weight_dtype) && dtype_valid(out_dtype),
                TSP_ERR_INVALID, "tsp_linear: bad dtype");
    if (n == 0) return TSP_OK;
    TSP_REQUIRE(d_x && d_weight && d_out, TSP_ERR_INVALID, "tsp_linear: null pointer");
    TSP_REQUIRE(d_out != d_x, TSP_ERR_INVALID, "tsp_linear: out aliases x");
    TSP_REQUIRE(n < (int64_t)INT32_MAX, TSP_ERR_INVALID, "tsp_linear: n=%lld out of range",
                (long long)n);
    // 16-bit x and weights of one dtype as a library GEMM, else on the matrix-core kernel;
    // everything else on the VALU kernel
    if (blaslt_eligible(x_dtype, weight_dtype, out_dtype, ci, co, d_x, d_weight, d_out)) {
        const int st = blaslt_linear(d_x, x_dtype, n, ci, d_weight, d_bias, co, TSP_ACT_NONE, nullptr,
                                     d_out, out_dtype, as_stream(stream));
        if (st != TSP_ERR_UNSUPPORTED) return st;
        clear_error();
    }
    if (mfma_eligible(x_dtype, weight_dtype, out_dtype, ci, co, d_x, d_weight, d_out))
        return dispatch_gather(x_dtype, out_dtype, d_x, n, ci, nullptr, 1, d_weight, d_bias, co,
                               d_out, as_stream(stream));
    return dispatch_narrow(x_dtype, weight_dtype, out_dtype, d_x, n, ci, nullptr, d_weight,
                           d_bias, co, d_out, as_stream(stream));
}
