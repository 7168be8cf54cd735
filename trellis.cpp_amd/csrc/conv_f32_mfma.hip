// Submanifold conv on fp32 features and fp32 weights with the fp32 matrix cores: the reference's
// cast-to-f32 mode (g_sparse_cast_f32, sparse.cpp:16-19) and the fp32 64^3 shell configuration.
// Replaces the same per-tap gather + mul_mat + add of submconv_range (sparse.cpp:61-79).
//
// v_mfma_f32_32x32x2_f32 adds a 32 x 2 by 2 x 32 product to a 32 x 32 block: lane l holds
// A[l % 32][l / 32] and B[l / 32][l % 32]; the block D is laid out as in the 16-bit kernels (lane l,
// element j: D[8 (j / 4) + 4 (l / 32) + j % 4][l % 32]). One 16-channel chunk of a tap is 8 such
// steps: lane l loads channels 8 (l / 32) .. + 7 of its voxel's neighbour row (two 16-byte loads)
// and of its output channel's weights, and step j pairs channel j with channel 8 + j of the chunk
// (the order of the contraction changes only the rounding of the sum, not its terms).
//
// Each wave owns 32 RB rows x 32 CB output channels for a group of taps: with KG > 1 the KG waves
// of a workgroup take taps g, g + KG, ... of one tile and add their partial sums in wave order
// through LDS (deterministic). That serves convs with too few tiles to give every SIMD a few
// waves: the 64^3 shell's ~15 K voxels make 455 tiles of 32 rows for 1,024 SIMDs. (Skipping the
// taps absent from a whole 32-row tile would save ~1 % there: rows in table order leave few.)
//
// Absent taps read the padding row 0 * feats[0] (sparse.cpp:81-85) -- zeros, or NaN in the
// channels where row 0 (or the caller's f32 source row) holds an Inf or a NaN -- and every tap is
// computed, so a non-finite weight or padding row gives NaN exactly where the reference's sum does.
// Operands are read straight from L2 (the weights are shared by every tile); nothing but the
// partial sums goes through LDS.
#include <algorithm>

#include "conv_internal.hpp"

namespace tsp {
namespace {

__device__ __forceinline__ f32x16_t mfma32x32x2(float a, float b, const f32x16_t& c) {
    return __builtin_amdgcn_mfma_f32_32x32x2f32(a, b, c, 0, 0, 0);
}

template <int ODT, int RB, int CB, int KG>
__global__ __launch_bounds__(64 * KG) void k_conv_f32_mfma(const float* __restrict__ feats, int64_t n, int ci,
                                                          const int32_t* __restrict__ nbr,
                                                          const float* __restrict__ weight,
                                                          const float* __restrict__ bias, int co,
                                                          void* __restrict__ out, int n_ctiles, PadRow pad) {
    constexpr int NACC = RB * CB;
    constexpr int PART = KG > 1 ? (KG - 1) * NACC * 16 * 64 : 1;
    __shared__ __attribute__((aligned(16))) float sPart[PART];

    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int r32 = lane & 31, h = lane >> 5;
    const int64_t tile = blockIdx.x / n_ctiles;
    const int c0 = (int)(blockIdx.x % n_ctiles) * 32 * CB;
    const int64_t row0 = tile * 32 * RB;
    const uint32_t un = (uint32_t)n;

    // whether the padding row holds a NaN (an exact zero row, pad.zero, never does)
    bool bad = false;
    if (!pad.zero)
        for (int k = tid; k < ci; k += 64 * KG) bad |= !__builtin_isfinite(pad.row0 ? pad.row0[k] : feats[k]);
    bad = __syncthreads_or(bad);
    const float* prow = pad.row0 ? pad.row0 : feats;

    f32x16_t acc[RB][CB];
#pragma unroll
    for (int rb = 0; rb < RB; ++rb)
#pragma unroll
        for (int cb = 0; cb < CB; ++cb)
#pragma unroll
            for (int e = 0; e < 16; ++e) acc[rb][cb][e] = 0.f;

    // neighbour rows of this lane's voxels at tap t (N for an absent tap or a row past the end)
    auto load_rows = [&](int t, int32_t (&v)[RB]) {
#pragma unroll
        for (int rb = 0; rb < RB; ++rb) {
            const int64_t i = row0 + 32 * rb + r32;
            v[rb] = (t < kTaps && i < n) ? nbr[(int64_t)t * n + i] : (int32_t)n;
        }
    };
    // the lane's 8 channels of chunk kc: its rows' (or the padding row's) and its columns' weights
    auto load_ops = [&](int t, int kc, const int32_t (&v)[RB], float4 (&a)[RB][2], float4 (&b)[CB][2]) {
        const int k0 = kc * 16 + 8 * h;
#pragma unroll
        for (int rb = 0; rb < RB; ++rb) {
            if ((uint32_t)v[rb] < un) {
                const float4* p = reinterpret_cast<const float4*>(feats + (int64_t)v[rb] * ci + k0);
                a[rb][0] = p[0];
                a[rb][1] = p[1];
            } else if (bad) {   // element loads: the caller's source row need not be 16-byte aligned
                const float* p = prow + k0;
                a[rb][0] = make_float4(0.f * p[0], 0.f * p[1], 0.f * p[2], 0.f * p[3]);
                a[rb][1] = make_float4(0.f * p[4], 0.f * p[5], 0.f * p[6], 0.f * p[7]);
            } else {
                a[rb][0] = make_float4(0.f, 0.f, 0.f, 0.f);
                a[rb][1] = a[rb][0];
            }
        }
#pragma unroll
        for (int cb = 0; cb < CB; ++cb) {
            const float4* p = reinterpret_cast<const float4*>(
                weight + ((int64_t)(c0 + 32 * cb + r32) * kTaps + t) * ci + k0);
            b[cb][0] = p[0];
            b[cb][1] = p[1];
        }
    };

    // this wave's taps t = wave, wave + KG, ... times ci / 16 chunks, each chunk's operands
    // loaded one chunk ahead and each tap's rows one tap ahead
    const int nkc = ci >> 4;
    int t = wave, kc = 0;
    int32_t v[RB], vn[RB];
    load_rows(t, v);
    load_rows(t + KG, vn);
    float4 aC[RB][2], bC[CB][2];
    if (t < kTaps) load_ops(t, 0, v, aC, bC);
    while (t < kTaps) {
        int tn = t, kcn = kc + 1;
        if (kcn == nkc) {
            kcn = 0;
            tn = t + KG;
        }
        const bool more = tn < kTaps;
        float4 aN[RB][2], bN[CB][2];
        if (more) load_ops(tn, kcn, kcn == 0 ? vn : v, aN, bN);
#pragma unroll
        for (int j = 0; j < 8; ++j) {
#pragma unroll
            for (int rb = 0; rb < RB; ++rb) {
                const float4 aq = aC[rb][j >> 2];
                const float av = (j & 3) == 0 ? aq.x : (j & 3) == 1 ? aq.y : (j & 3) == 2 ? aq.z : aq.w;
#pragma unroll
                for (int cb = 0; cb < CB; ++cb) {
                    const float4 bq = bC[cb][j >> 2];
                    const float bv = (j & 3) == 0 ? bq.x : (j & 3) == 1 ? bq.y : (j & 3) == 2 ? bq.z : bq.w;
                    acc[rb][cb] = mfma32x32x2(av, bv, acc[rb][cb]);
                }
            }
        }
        if (!more) break;
#pragma unroll
        for (int rb = 0; rb < RB; ++rb) {
            aC[rb][0] = aN[rb][0];
            aC[rb][1] = aN[rb][1];
        }
#pragma unroll
        for (int cb = 0; cb < CB; ++cb) {
            bC[cb][0] = bN[cb][0];
            bC[cb][1] = bN[cb][1];
        }
        if (kcn == 0) {
#pragma unroll
            for (int rb = 0; rb < RB; ++rb) v[rb] = vn[rb];
            load_rows(tn + KG, vn);
        }
        t = tn;
        kc = kcn;
    }

    if constexpr (KG > 1) {
        // waves 1 .. KG-1 leave their partial sums in LDS (lane-major); wave 0 adds them in order
        if (wave > 0) {
#pragma unroll
            for (int rb = 0; rb < RB; ++rb)
#pragma unroll
                for (int cb = 0; cb < CB; ++cb)
#pragma unroll
                    for (int e = 0; e < 16; ++e)
                        sPart[(((wave - 1) * NACC + rb * CB + cb) * 16 + e) * 64 + lane] = acc[rb][cb][e];
        }
        __syncthreads();
        if (wave != 0) return;
        for (int g = 0; g < KG - 1; ++g)
#pragma unroll
            for (int rb = 0; rb < RB; ++rb)
#pragma unroll
                for (int cb = 0; cb < CB; ++cb)
#pragma unroll
                    for (int e = 0; e < 16; ++e)
                        acc[rb][cb][e] += sPart[((g * NACC + rb * CB + cb) * 16 + e) * 64 + lane];
    }

    // lanes 0-31 store 32 consecutive channels of one row, lanes 32-63 of the row 4 below
#pragma unroll
    for (int cb = 0; cb < CB; ++cb) {
        const int oc = c0 + 32 * cb + r32;
        const float bv = bias[oc];
#pragma unroll
        for (int rb = 0; rb < RB; ++rb)
#pragma unroll
            for (int e = 0; e < 16; ++e) {
                const int64_t i = row0 + 32 * rb + 8 * (e >> 2) + 4 * h + (e & 3);
                if (i < n) store_out<ODT>(out, i * co + oc, acc[rb][cb][e] + bv);
            }
    }
}

int cu_count_f32() {
    static int cached[64] = {0};
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
    if (!cached[dev]) {
        int cus = 0;
        if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0)
            cus = 256;
        cached[dev] = cus;
    }
    return cached[dev];
}

template <int ODT, int CB>
int launch_cb(const float* feats, int64_t n, int ci, const int32_t* nbr, const float* weight, const float* bias,
              int co, void* out, hipStream_t s, PadRow pad) {
    const int n_ctiles = co / (32 * CB);
    // 64-row tiles of one wave where they give at least ~4 waves a SIMD, else 32-row tiles whose
    // taps are split over 4 waves (on the 64^3 shell 6 % faster than over 8, whose 512-thread
    // workgroups hold one a CU)
    const int64_t waves_wanted = 16LL * cu_count_f32();
    const int64_t t64 = ceil_div(n, 64) * n_ctiles, t32 = ceil_div(n, 32) * n_ctiles;
    if (t64 >= waves_wanted)
        hipLaunchKernelGGL((k_conv_f32_mfma<ODT, 2, CB, 1>), dim3((unsigned)t64), dim3(64), 0, s, feats, n, ci,
                           nbr, weight, bias, co, out, n_ctiles, pad);
    else
        hipLaunchKernelGGL((k_conv_f32_mfma<ODT, 1, CB, 4>), dim3((unsigned)t32), dim3(256), 0, s, feats, n, ci,
                           nbr, weight, bias, co, out, n_ctiles, pad);
    TSP_CHECK_LAUNCH();
    return TSP_OK;
}

template <int ODT>
int launch_f32(const float* feats, int64_t n, int ci, const int32_t* nbr, const float* weight, const float* bias,
               int co, void* out, hipStream_t s, PadRow pad) {
    if (co % 64 == 0) return launch_cb<ODT, 2>(feats, n, ci, nbr, weight, bias, co, out, s, pad);
    return launch_cb<ODT, 1>(feats, n, ci, nbr, weight, bias, co, out, s, pad);
}

}  // namespace

bool f32_mfma_fits(int fdt, int wdt, int ci, int co, const void* feats, const void* weight) {
    return fdt == TSP_F32 && wdt == TSP_F32 && ci % 16 == 0 && co % 32 == 0 &&
           (reinterpret_cast<uintptr_t>(feats) & 15) == 0 && (reinterpret_cast<uintptr_t>(weight) & 15) == 0;
}

int f32_mfma_launch(int fdt, int wdt, int odt, const void* feats, int64_t n, int ci, const int32_t* nbr,
                    const void* weight, const float* bias, int co, void* out, hipStream_t s, PadRow pad) {
    if (!nbr || !f32_mfma_fits(fdt, wdt, ci, co, feats, weight)) return TSP_ERR_UNSUPPORTED;
    // grid.x is a tile count below 2^31: n < 2^31 rows, 32-row tiles, co / 32 column tiles
    if (ceil_div(n, 32) * (co / 32) >= ((int64_t)1 << 31)) return TSP_ERR_UNSUPPORTED;
    const float* f = static_cast<const float*>(feats);
    const float* w = static_cast<const float*>(weight);
    switch (odt) {
        case TSP_F32: return launch_f32<TSP_F32>(f, n, ci, nbr, w, bias, co, out, s, pad);
        case TSP_F16: return launch_f32<TSP_F16>(f, n, ci, nbr, w, bias, co, out, s, pad);
        case TSP_BF16: return launch_f32<TSP_BF16>(f, n, ci, nbr, w, bias, co, out, s, pad);
    }
    return TSP_ERR_UNSUPPORTED;
}

}  // namespace tsp
