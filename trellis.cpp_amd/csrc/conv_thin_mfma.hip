// Submanifold conv for thin channel counts on 16-bit features, bound by memory rather than by
// arithmetic: a layer with Ci * Co <= 512 does 2 * Ci * Co FLOPs per (voxel, tap) against the 4
// bytes of its table entry and the Ci * 2 bytes of the gathered row, ~17 FLOP per compulsory byte
// at Ci = Co = 8 -- far below the matrix cores' ridge (~310), but above what the VALU issues
// without packed fp32 (a VALU kernel there is FMA-issue bound at ~2.5x the HBM time).
//
// The 27 taps are folded into the contraction: out[i] = bias + sum_k A[i][k] W'[k][o] with
// k = (tap, channel), A[i][(t, c)] = feats[nbr[t][i]][c] (zero for an absent tap) and
// W'[(t, c)][o] = W[o][t][c], K = 27 Ci padded to a multiple of 32. Each 16-voxel block is one
// column of v_mfma_f32_16x16x32 steps: in step s, lane l (voxel l % 16, k chunk l / 16) holds the
// 8 channels k = 32 s + 8 (l / 16) .. + 7 -- one tap's row (Ci = 8) or a half / quarter of it
// (Ci = 16, 32) -- which it gathers with a single 16-byte load straight into the operand
// register, after its table entry. The weights (B operand, 16 output channels a block) sit in
// registers for the whole launch; nothing goes through LDS but the output rows, staged so that
// each lane stores whole 8- or 16-byte pieces of rows.
//
// Bytes per voxel: 108 (its table column) + Ci * s_in (its own row, as some neighbour's; the 27
// gathers are L2 hits) + Co * s_out. A persistent grid of waves walks 16 RB-voxel chunks.
#include <algorithm>

#include "conv_internal.hpp"

namespace tsp {
namespace {

constexpr int TM_THREADS = 256;
constexpr int TM_WAVES = TM_THREADS / 64;

template <bool BF16>
__device__ __forceinline__ f32x4_t mfma16x16x32(const u32x4_t& a, const u32x4_t& b, const f32x4_t& c) {
    if constexpr (BF16)
        return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, a), __builtin_bit_cast(bf16x8_t, b),
                                                       c, 0, 0, 0);
    else
        return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8_t, a), __builtin_bit_cast(f16x8_t, b),
                                                      c, 0, 0, 0);
}

int cu_count_tm() {
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

// CI input channels (8, 16 or 32), NCB blocks of 16 output channels (co <= 16 NCB), RB 16-voxel
// blocks per chunk, output dtype ODT.
template <bool BF16, int ODT, int CI, int NCB, int RB>
__global__ __launch_bounds__(TM_THREADS) void k_conv_thin_mfma(
    const uint16_t* __restrict__ feats, int64_t n, const int32_t* __restrict__ nbr,
    const uint16_t* __restrict__ weight, const float* __restrict__ bias, int co,
    typename Elem<ODT>::storage* __restrict__ out, PadRow pad) {
    constexpr int NS = (kTaps * CI + 31) / 32;   // k steps
    constexpr int COP = 16 * NCB;                // output channels padded to the blocks
    constexpr int CH = RB * 16;                  // voxels per chunk
    __shared__ __attribute__((aligned(16))) float sO[TM_WAVES][CH][COP + 1];
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int v16 = lane & 15, kq = lane >> 4;

    // the padding row 0 * feats[0] (sparse.cpp:81-85): NaN where row 0 is not finite, and then
    // every output row with an absent tap is NaN (an exact zero padding row never is)
    bool row0_bad = false;
    if (!pad.zero) {
        if (pad.row0) {
            for (int k = tid; k < CI; k += TM_THREADS) row0_bad |= !__builtin_isfinite(pad.row0[k]);
        } else {
            constexpr uint32_t kExp = BF16 ? 0x7F80u : 0x7C00u;
            for (int k = tid; k < CI; k += TM_THREADS) row0_bad |= (feats[k] & kExp) == kExp;
        }
    }
    row0_bad = __syncthreads_or(row0_bad);

    // the tap and channel of this lane's k chunk in each step (t = 27: padding, zero operands)
    int tap[NS], ch0[NS];
#pragma unroll
    for (int s = 0; s < NS; ++s) {
        const int k = 32 * s + 8 * kq;
        tap[s] = k / CI;
        ch0[s] = k % CI;
    }
    // B operands: W'[(t, c)][o] for o = 16 cb + v16, held for the whole launch
    u32x4_t bw[NS][NCB];
#pragma unroll
    for (int s = 0; s < NS; ++s)
#pragma unroll
        for (int cb = 0; cb < NCB; ++cb) {
            const int o = 16 * cb + v16;
            bw[s][cb] = u32x4_t{0u, 0u, 0u, 0u};
            if (tap[s] < kTaps && o < co)
                bw[s][cb] = *reinterpret_cast<const u32x4_t*>(weight + ((int64_t)o * kTaps + tap[s]) * CI + ch0[s]);
        }
    float bv[NCB];
#pragma unroll
    for (int cb = 0; cb < NCB; ++cb) {
        const int o = 16 * cb + v16;
        bv[cb] = bias && o < co ? bias[o] : 0.f;
    }

    const __amdgpu_buffer_rsrc_t rn = __builtin_amdgcn_make_buffer_rsrc(const_cast<int32_t*>(nbr), (short)0,
                                                                         (int)(kTaps * n * 4), 0x00020000);
    const __amdgpu_buffer_rsrc_t rf = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t*>(feats), (short)0,
                                                                         (int)(n * CI * 2), 0x00020000);
    // first byte past each buffer's range: a load there reads zeros and touches no memory
    const uint32_t tab_end = (uint32_t)(kTaps * n * 4), feat_end = (uint32_t)(n * CI * 2);
    // XCD-aware order: workgroup ids go round-robin over the 8 XCDs, so each XCD takes one
    // contiguous range of chunks, walked by its waves together -- the rows they gather (neighbours
    // of nearby voxels) stay in that XCD's L2
    const int64_t nchunks = (n + CH - 1) / CH;
    const int64_t per_xcd = (nchunks + 7) / 8;
    const int64_t xlo = (int64_t)(blockIdx.x % 8) * per_xcd;
    const int64_t xhi = xlo + per_xcd < nchunks ? xlo + per_xcd : nchunks;
    for (int64_t chunk = xlo + (int64_t)(blockIdx.x / 8) * TM_WAVES + wave; chunk < xhi;
         chunk += (int64_t)(gridDim.x / 8) * TM_WAVES) {
        // table entries of every (block, step) first, then the rows they name: all loads of the
        // chunk in flight together. Both go through buffer resources with 32-bit offsets (the
        // launch checks that the table and the features span less than 2 GiB): an entry of a
        // padding tap or a voxel past n is read out of range (0) and replaced by n, and the row of
        // an absent tap is read out of range: zeros.
        int32_t e[RB][NS];
#pragma unroll
        for (int rb = 0; rb < RB; ++rb) {
            const int64_t i = chunk * CH + 16 * rb + v16;
#pragma unroll
            for (int s = 0; s < NS; ++s) {
                const bool real = tap[s] < kTaps && i < n;
                const uint32_t off = real ? ((uint32_t)tap[s] * (uint32_t)n + (uint32_t)i) * 4u : tab_end;
                const int32_t v = (int32_t)__builtin_amdgcn_raw_buffer_load_b32(rn, off, 0, 0);
                e[rb][s] = real ? v : (int32_t)n;
            }
        }
        u32x4_t a[RB][NS];
        uint64_t absent_bits[RB];
#pragma unroll
        for (int rb = 0; rb < RB; ++rb) {
            absent_bits[rb] = 0;
#pragma unroll
            for (int s = 0; s < NS; ++s) {
                const bool have = (uint32_t)e[rb][s] < (uint32_t)n;
                const uint32_t off = have ? (uint32_t)e[rb][s] * (uint32_t)(CI * 2) + (uint32_t)(ch0[s] * 2) : feat_end;
                a[rb][s] = __builtin_bit_cast(u32x4_t, __builtin_amdgcn_raw_buffer_load_b128(rf, off, 0, 0));
                // an absent real tap (the padding rows of k beyond 27 taps do not count)
                absent_bits[rb] |= __ballot(!have && tap[s] < kTaps);
            }
        }
        f32x4_t acc[RB][NCB];
#pragma unroll
        for (int rb = 0; rb < RB; ++rb)
#pragma unroll
            for (int cb = 0; cb < NCB; ++cb) {
                acc[rb][cb] = f32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
                for (int s = 0; s < NS; ++s) acc[rb][cb] = mfma16x16x32<BF16>(a[rb][s], bw[s][cb], acc[rb][cb]);
            }
        // staging: lane l holds output channel 16 cb + l % 16 of rows 4 (l / 16) .. + 3 of block rb
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
#pragma unroll
        for (int rb = 0; rb < RB; ++rb) {
            // rows of this block with an absent tap: the four lanes v, v + 16, v + 32, v + 48
            // cover voxel v's taps
            const uint64_t ab = absent_bits[rb];
            const uint32_t vox_absent = (uint32_t)((ab | (ab >> 16) | (ab >> 32) | (ab >> 48)) & 0xffffu);
#pragma unroll
            for (int cb = 0; cb < NCB; ++cb)
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const int r = 4 * kq + j;
                    float v = acc[rb][cb][j] + bv[cb];
                    if (row0_bad && ((vox_absent >> r) & 1u)) v = __builtin_nanf("");
                    sO[wave][16 * rb + r][16 * cb + v16] = v;
                }
        }
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        // stores: 4 consecutive elements of the chunk's [CH][co] output per lane and pass
        const int total = CH * co;
        for (int q = 4 * lane; q < total; q += 4 * 64) {
            const int r = q / co, c = q % co;          // co % 4 == 0: the 4 stay in one row
            const int64_t i = chunk * CH + r;
            if (i >= n) continue;
            const float* src = &sO[wave][r][c];
            if constexpr (ODT == TSP_F32) {
                *reinterpret_cast<f32x4_t*>(out + i * co + c) = f32x4_t{src[0], src[1], src[2], src[3]};
            } else {
                uint32_t w0, w1;
                if constexpr (ODT == TSP_BF16) {
                    w0 = f32x2_to_bf16x2_bits(src[0], src[1]);
                    w1 = f32x2_to_bf16x2_bits(src[2], src[3]);
                } else {
                    w0 = f32_to_f16_bits(src[0]) | ((uint32_t)f32_to_f16_bits(src[1]) << 16);
                    w1 = f32_to_f16_bits(src[2]) | ((uint32_t)f32_to_f16_bits(src[3]) << 16);
                }
                *reinterpret_cast<uint2*>(out + i * co + c) = uint2{w0, w1};
            }
        }
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    }
}

template <bool BF16, int ODT, int CI, int NCB>
int launch_tm(const void* feats, int64_t n, const int32_t* nbr, const void* weight, const float* bias, int co,
              void* out, hipStream_t s, PadRow pad) {
    // 16-voxel blocks per chunk: two at Ci = 8, where a block's operands take 28 registers
    constexpr int RB = CI == 8 ? 2 : 1;
    const int64_t nchunks = ceil_div(n, 16 * RB);
    // a multiple of 8 workgroups (one range per XCD), at most 4 a CU
    const int64_t blocks = std::max<int64_t>(
        8, std::min<int64_t>(ceil_div(nchunks, TM_WAVES * 8) * 8, (int64_t)cu_count_tm() * 4 / 8 * 8));
    hipLaunchKernelGGL((k_conv_thin_mfma<BF16, ODT, CI, NCB, RB>), dim3((unsigned)blocks),
                       dim3(TM_THREADS), 0, s, static_cast<const uint16_t*>(feats), n, nbr,
                       static_cast<const uint16_t*>(weight), bias, co,
                       static_cast<typename Elem<ODT>::storage*>(out), pad);
    TSP_CHECK_LAUNCH();
    return TSP_OK;
}

template <bool BF16, int ODT>
int tm_shape(int ci, int co, const void* feats, int64_t n, const int32_t* nbr, const void* weight,
             const float* bias, void* out, hipStream_t s, PadRow pad) {
    const bool two = co > 16;
    switch (ci) {
        case 8:
            return two ? launch_tm<BF16, ODT, 8, 2>(feats, n, nbr, weight, bias, co, out, s, pad)
                       : launch_tm<BF16, ODT, 8, 1>(feats, n, nbr, weight, bias, co, out, s, pad);
        case 16:
            return two ? launch_tm<BF16, ODT, 16, 2>(feats, n, nbr, weight, bias, co, out, s, pad)
                       : launch_tm<BF16, ODT, 16, 1>(feats, n, nbr, weight, bias, co, out, s, pad);
        case 32:
            return launch_tm<BF16, ODT, 32, 1>(feats, n, nbr, weight, bias, co, out, s, pad);
    }
    return TSP_ERR_UNSUPPORTED;
}

}  // namespace

bool thin_mfma_fits(int fdt, int wdt, int ci, int co) {
    return (fdt == TSP_BF16 || fdt == TSP_F16) && wdt == fdt && (ci == 8 || ci == 16 || ci == 32) &&
           (co == 4 || co == 8 || co == 16 || co == 32) && ci * co <= 512;
}

int thin_mfma_launch(int fdt, int wdt, int odt, const void* feats, int64_t n, int ci, const int32_t* nbr,
                     const void* weight, const float* bias, int co, void* out, hipStream_t s, PadRow pad) {
    if (!thin_mfma_fits(fdt, wdt, ci, co) || !nbr) return TSP_ERR_UNSUPPORTED;
    // the table and the features addressed with 32-bit byte offsets (buffer loads); the resource's
    // record count is an int
    if ((int64_t)kTaps * n * 4 >= (int64_t)INT32_MAX || n * ci * 2 >= (int64_t)INT32_MAX) return TSP_ERR_UNSUPPORTED;
    // 16-byte gathers of feature rows and of weight rows
    if (reinterpret_cast<uintptr_t>(feats) % 16 || reinterpret_cast<uintptr_t>(weight) % 16) return TSP_ERR_UNSUPPORTED;
    if (reinterpret_cast<uintptr_t>(out) % (odt == TSP_F32 ? 16 : 8)) return TSP_ERR_UNSUPPORTED;
    const bool bf = fdt == TSP_BF16;
    if (odt == TSP_F32)
        return bf ? tm_shape<true, TSP_F32>(ci, co, feats, n, nbr, weight, bias, out, s, pad)
                  : tm_shape<false, TSP_F32>(ci, co, feats, n, nbr, weight, bias, out, s, pad);
    if (odt == TSP_BF16 && bf) return tm_shape<true, TSP_BF16>(ci, co, feats, n, nbr, weight, bias, out, s, pad);
    if (odt == TSP_F16 && !bf) return tm_shape<false, TSP_F16>(ci, co, feats, n, nbr, weight, bias, out, s, pad);
    return TSP_ERR_UNSUPPORTED;
}

}  // namespace tsp
