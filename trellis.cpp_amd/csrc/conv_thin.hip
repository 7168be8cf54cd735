// Submanifold conv for thin channel counts (Co <= 32, Ci * Co <= 512) on the VALU.
//
// Matrix-core tiles are 32 or 64 output channels wide and 16 input channels deep, so a conv with
// a few channels would leave most of each tile empty; the tiled VALU kernel's 64 x 64 output tile
// wastes as much. Here one thread owns one voxel's whole output row: its Co accumulators stay in
// registers while it walks the 27 taps, reading the table entry (coalesced across the wave), the
// neighbour's Ci features (a few 8- or 16-byte loads, mostly L2 hits: neighbours of nearby voxels
// coincide) and the tap's weights from LDS, where all lanes read the same address (a broadcast).
// The 27 table entries are loaded first and the rows then nine taps at a time, so many loads are
// in flight per lane (an absent tap loads row 0 and adds zeros). The weights, converted to f32
// once per workgroup, take 27 * Ci * Co * 4 <= 55 KB of LDS; a persistent grid of as many
// workgroups per CU as the LDS allows walks the voxels, so each workgroup converts them once.
//
// Bytes per voxel: 108 (its table column) + Ci * s (its own features, as some neighbour's) +
// Co * s_out, so at Co <= 8 the kernel is bound by HBM and above that by fp32 FMA issue.
#include <algorithm>

#include "conv_internal.hpp"

namespace tsp {
namespace {

constexpr int TH_THREADS = 256;
constexpr int TH_WMAX = 512;        // Ci * Co

// Compute units of the current device (cached per device).
int cu_count_thin() {
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

template <int DT> struct Vec4;      // four consecutive elements as floats
template <> struct Vec4<TSP_F32> {
    __device__ __forceinline__ static void load(const float* p, float (&v)[4]) {
        const float4 q = *reinterpret_cast<const float4*>(p);
        v[0] = q.x; v[1] = q.y; v[2] = q.z; v[3] = q.w;
    }
};
template <> struct Vec4<TSP_BF16> {
    __device__ __forceinline__ static void load(const uint16_t* p, float (&v)[4]) {
        const uint2 q = *reinterpret_cast<const uint2*>(p);
        v[0] = __uint_as_float(q.x << 16); v[1] = __uint_as_float(q.x & 0xffff0000u);
        v[2] = __uint_as_float(q.y << 16); v[3] = __uint_as_float(q.y & 0xffff0000u);
    }
};
template <> struct Vec4<TSP_F16> {
    __device__ __forceinline__ static void load(const uint16_t* p, float (&v)[4]) {
        const uint2 q = *reinterpret_cast<const uint2*>(p);
        v[0] = f16_bits_to_f32((uint16_t)(q.x & 0xffffu)); v[1] = f16_bits_to_f32((uint16_t)(q.x >> 16));
        v[2] = f16_bits_to_f32((uint16_t)(q.y & 0xffffu)); v[3] = f16_bits_to_f32((uint16_t)(q.y >> 16));
    }
};

template <int FDT, int WDT, int ODT, int CO>
__global__ __launch_bounds__(TH_THREADS) void k_conv_thin(
    const typename Elem<FDT>::storage* __restrict__ feats, int64_t n, int ci,
    const int32_t* __restrict__ nbr, const typename Elem<WDT>::storage* __restrict__ weight,
    const float* __restrict__ bias, typename Elem<ODT>::storage* __restrict__ out, PadRow pad) {
    extern __shared__ __attribute__((aligned(16))) float sW[];   // [tap][k][o], 27 * ci * CO
    const int tid = threadIdx.x;
    const int nw = kTaps * ci * CO;
    for (int e = tid; e < nw; e += TH_THREADS) {
        const int o = e % CO, k = (e / CO) % ci, t = e / (CO * ci);
        sW[e] = Elem<WDT>::load(weight, ((int64_t)o * kTaps + t) * ci + k);
    }
    // the padding row 0 * feats[0] (sparse.cpp:81-85): NaN where row 0 is not finite, and then
    // every output row with an absent tap is NaN (an exact zero padding row never is)
    bool row0_bad = false;
    if (!pad.zero)
        for (int k = tid; k < ci; k += TH_THREADS)
            row0_bad |= !__builtin_isfinite(pad.row0 ? pad.row0[k] : Elem<FDT>::load(feats, k));
    row0_bad = __syncthreads_or(row0_bad);
    float bv[CO];
#pragma unroll
    for (int o = 0; o < CO; ++o) bv[o] = bias ? bias[o] : 0.f;

    const int64_t step = (int64_t)gridDim.x * TH_THREADS;
    for (int64_t i = blockIdx.x * (int64_t)TH_THREADS + tid; i < n; i += step) {
        // the voxel's 27 table entries first (independent, coalesced loads); an absent tap reads
        // row 0 and discards it, so every tap's loads are issued alike and overlap
        uint32_t roff[kTaps];
        uint32_t present = 0;
#pragma unroll
        for (int t = 0; t < kTaps; ++t) {
            const int32_t r = nbr[(int64_t)t * n + i];
            const bool v = (uint32_t)r < (uint32_t)n;
            present |= (v ? 1u : 0u) << t;
            roff[t] = v ? (uint32_t)r * (uint32_t)ci : 0u;
        }
        float acc[CO];
#pragma unroll
        for (int o = 0; o < CO; ++o) acc[o] = 0.f;
        // four channels of 9 taps at a time: 9 loads in flight, then their FMAs
        for (int k0 = 0; k0 < ci; k0 += 4) {
#pragma unroll
            for (int tg = 0; tg < 3; ++tg) {
                float xv[9][4];
#pragma unroll
                for (int j = 0; j < 9; ++j) {
                    const int t = 9 * tg + j;
                    Vec4<FDT>::load(feats + roff[t] + k0, xv[j]);
                }
                // one tap's weights at a time: unconstrained, the scheduler would hoist every
                // tap's LDS reads above the FMAs and run out of registers
                __builtin_amdgcn_sched_barrier(0);
#pragma unroll
                for (int j = 0; j < 9; ++j) {
                    const int t = 9 * tg + j;
                    const bool v = (present >> t) & 1u;
                    const float* w = sW + (t * ci + k0) * CO;
#pragma unroll
                    for (int kk = 0; kk < 4; ++kk) {
                        const float x = v ? xv[j][kk] : 0.f;
#pragma unroll
                        for (int o = 0; o < CO; ++o) acc[o] = fmaf(x, w[kk * CO + o], acc[o]);
                    }
                    __builtin_amdgcn_sched_barrier(0);
                }
            }
        }
        const bool nan_row = row0_bad && present != (1u << kTaps) - 1u;
#pragma unroll
        for (int o = 0; o < CO; ++o)
            Elem<ODT>::store(out, i * CO + o, nan_row ? __builtin_nanf("") : acc[o] + bv[o]);
    }
}

template <int FDT, int WDT, int ODT, int CO>
int launch_thin(const void* feats, int64_t n, int ci, const int32_t* nbr, const void* weight,
                const float* bias, void* out, hipStream_t s, PadRow pad) {
    const size_t lds = (size_t)kTaps * ci * CO * 4;
    // workgroups a CU can hold by LDS (160 KB) and by waves (up to 8 per SIMD over 4 SIMDs = 32,
    // i.e. 8 workgroups of 4 waves), a persistent grid of that many per CU
    const int per_cu = (int)std::max<size_t>(1, std::min<size_t>(8, (160 * 1024) / std::max<size_t>(lds, 1)));
    const int64_t blocks = std::min<int64_t>(ceil_div(n, TH_THREADS), (int64_t)per_cu * cu_count_thin());
    hipLaunchKernelGGL((k_conv_thin<FDT, WDT, ODT, CO>), dim3((unsigned)std::max<int64_t>(blocks, 1)),
                       dim3(TH_THREADS), lds, s, reinterpret_cast<const typename Elem<FDT>::storage*>(feats), n,
                       ci, nbr, reinterpret_cast<const typename Elem<WDT>::storage*>(weight), bias,
                       reinterpret_cast<typename Elem<ODT>::storage*>(out), pad);
    TSP_CHECK_LAUNCH();
    return TSP_OK;
}

template <int FDT, int WDT, int ODT>
int thin_co(int co, const void* feats, int64_t n, int ci, const int32_t* nbr, const void* weight,
            const float* bias, void* out, hipStream_t s, PadRow pad) {
    switch (co) {
        case 4: return launch_thin<FDT, WDT, ODT, 4>(feats, n, ci, nbr, weight, bias, out, s, pad);
        case 8: return launch_thin<FDT, WDT, ODT, 8>(feats, n, ci, nbr, weight, bias, out, s, pad);
        case 16: return launch_thin<FDT, WDT, ODT, 16>(feats, n, ci, nbr, weight, bias, out, s, pad);
        case 32: return launch_thin<FDT, WDT, ODT, 32>(feats, n, ci, nbr, weight, bias, out, s, pad);
    }
    return TSP_ERR_UNSUPPORTED;
}

template <int FDT, int WDT>
int thin_out(int odt, int co, const void* feats, int64_t n, int ci, const int32_t* nbr, const void* weight,
             const float* bias, void* out, hipStream_t s, PadRow pad) {
    if (odt == TSP_F32) return thin_co<FDT, WDT, TSP_F32>(co, feats, n, ci, nbr, weight, bias, out, s, pad);
    if (odt == TSP_F16) return thin_co<FDT, WDT, TSP_F16>(co, feats, n, ci, nbr, weight, bias, out, s, pad);
    return thin_co<FDT, WDT, TSP_BF16>(co, feats, n, ci, nbr, weight, bias, out, s, pad);
}

}  // namespace

bool thin_fits(int ci, int co) {
    return (co == 4 || co == 8 || co == 16 || co == 32) && ci % 4 == 0 && ci > 0 && ci * co <= TH_WMAX;
}

int thin_conv_launch(int fdt, int wdt, int odt, const void* feats, int64_t n, int ci, const int32_t* nbr,
                     const void* weight, const float* bias, int co, void* out, hipStream_t s, PadRow pad) {
    if (!thin_fits(ci, co) || !nbr) return TSP_ERR_UNSUPPORTED;
    // the kernel's feature offsets (row * ci) are 32-bit
    if ((uint64_t)n * (uint64_t)ci >= ((uint64_t)1 << 32)) return TSP_ERR_UNSUPPORTED;
    if (reinterpret_cast<uintptr_t>(feats) % 16) return TSP_ERR_UNSUPPORTED;
    if (fdt == TSP_F32 && wdt == TSP_F32) return thin_out<TSP_F32, TSP_F32>(odt, co, feats, n, ci, nbr, weight, bias, out, s, pad);
    if (fdt == TSP_F32 && wdt == TSP_F16) return thin_out<TSP_F32, TSP_F16>(odt, co, feats, n, ci, nbr, weight, bias, out, s, pad);
    if (fdt == TSP_F32 && wdt == TSP_BF16) return thin_out<TSP_F32, TSP_BF16>(odt, co, feats, n, ci, nbr, weight, bias, out, s, pad);
    if (fdt == TSP_F16 && wdt == TSP_F16) return thin_out<TSP_F16, TSP_F16>(odt, co, feats, n, ci, nbr, weight, bias, out, s, pad);
    if (fdt == TSP_BF16 && wdt == TSP_BF16) return thin_out<TSP_BF16, TSP_BF16>(odt, co, feats, n, ci, nbr, weight, bias, out, s, pad);
    return TSP_ERR_UNSUPPORTED;
}

}  // namespace tsp
