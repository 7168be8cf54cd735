// The LDS-staged MFMA conv's entry points: weight packing and the dispatch to the kernel
// instantiations (conv_halo_kernel.hpp holds the kernel; conv_halo_{bf16,f16}_{128,64}.hip
// instantiate it, one translation unit per family so that they compile in parallel).
#include "conv_halo_kernel.hpp"

namespace tsp {
namespace {

// packed[((c32 * nkc + kc) * 27 + t) * 64 + lane][0..7] = W[32 c32 + lane%32][t][16 kc + 8 (lane/32) ..];
// *nonfinite (the first word of the trailer, cleared before) |= 1 where a weight is an Inf or a NaN.
__global__ void k_weight_pack(const uint16_t* __restrict__ w, int ci, int co, bool bf16,
                              uint16_t* __restrict__ packed, uint32_t* __restrict__ nonfinite) {
    const int nkc = ci / HB_KC;
    const int64_t blk = blockIdx.x;                    // (c32 * nkc + kc) * 27 + t
    const int t = (int)(blk % kTaps);
    const int64_t ck = blk / kTaps;
    const int kc = (int)(ck % nkc), c32 = (int)(ck / nkc);
    const int lane = threadIdx.x;
    const int col = c32 * 32 + (lane & 31);
    const u32x4_t v = *reinterpret_cast<const u32x4_t*>(
        w + ((int64_t)col * kTaps + t) * ci + kc * HB_KC + (lane >> 5) * 8);
    reinterpret_cast<u32x4_t*>(packed)[blk * 64 + lane] = v;
    const uint32_t e = bf16 ? 0x7F80u : 0x7C00u;     // exponent all ones: Inf or NaN
    bool bad = false;
#pragma unroll
    for (int k = 0; k < 4; ++k) bad |= (v[k] & e) == e || ((v[k] >> 16) & e) == e;
    if (bad) atomicOr(nonfinite, 1u);
}

__global__ void k_pack_trailer_clear(uint32_t* __restrict__ trailer) {
    trailer[threadIdx.x] = 0u;
}

// One workgroup per tile, one thread per position: the octants each position's parent keeps
// (mask bytes != 0), ORed over each 32-position block (a wave's ballot covers two) into the word
// of its row group: bit 4 o + b for block b (0..3) of the 128 positions of row group p / 128.
__global__ __launch_bounds__(HB_M) void k_octant_blocks(const int32_t* __restrict__ vox, int64_t n,
                                                       const uint8_t* __restrict__ mask,
                                                       uint32_t* __restrict__ out) {
    __shared__ uint32_t sw[HB_M / 128];
    const int64_t tile = blockIdx.x;
    const int p = threadIdx.x, lane = p & 63, wave = p >> 6;
    if (p < HB_M / 128) sw[p] = 0u;
    __syncthreads();
    const int32_t v = vox[tile * HB_M + p];
    uint32_t kept = 0;
    if (v >= 0 && v < n) {
#pragma unroll
        for (int o = 0; o < 8; ++o) kept |= (mask[8 * (int64_t)v + o] != 0 ? 1u : 0u) << o;
    }
    uint32_t bits = 0;
    const int b0 = (wave & 1) * 2;   // this wave's first block within its row group
#pragma unroll
    for (int o = 0; o < 8; ++o) {
        const uint64_t b = __ballot((kept >> o) & 1u);
        bits |= ((uint32_t)(b & 0xffffffffull) != 0u ? 1u : 0u) << (4 * o + b0);
        bits |= ((uint32_t)(b >> 32) != 0u ? 1u : 0u) << (4 * o + b0 + 1);
    }
    if (lane == 0 && bits) atomicOr(&sw[wave >> 1], bits);
    __syncthreads();
    if (p < HB_M / 128) out[tile * (HB_M / 128) + p] = sw[p];
}

}  // namespace

int octant_blocks(const void* plan, int64_t n, const uint8_t* mask, uint32_t* out, hipStream_t s) {
    const int64_t n_tiles = ceil_div(n, HB_M);
    if (n_tiles == 0) return TSP_OK;
    const PlanView pv = carve_plan(const_cast<void*>(plan), n_tiles);
    hipLaunchKernelGGL(k_octant_blocks, dim3((unsigned)n_tiles), dim3(HB_M), 0, s, pv.vox, n, mask, out);
    TSP_CHECK_LAUNCH();
    return TSP_OK;
}

bool halo_fits(int64_t n, int ci) { return n * (int64_t)ci * 2 < ((int64_t)1 << 32); }

int halo_weight_pack(const void* w, int wdt, int ci, int co, void* packed, hipStream_t s) {
    const int64_t blocks = (int64_t)(co / 32) * (ci / HB_KC) * kTaps;
    uint32_t* trailer = reinterpret_cast<uint32_t*>(static_cast<char*>(packed) + (size_t)kTaps * ci * co * 2);
    hipLaunchKernelGGL(k_pack_trailer_clear, dim3(1), dim3(HB_PACK_TRAILER / 4), 0, s, trailer);
    TSP_CHECK_LAUNCH();
    if (blocks == 0) return TSP_OK;
    hipLaunchKernelGGL(k_weight_pack, dim3((unsigned)blocks), dim3(64), 0, s,
                       reinterpret_cast<const uint16_t*>(w), ci, co, wdt == TSP_BF16,
                       reinterpret_cast<uint16_t*>(packed), trailer);
    TSP_CHECK_LAUNCH();
    return TSP_OK;
}

int64_t column_split_tiles(int64_t n_tiles, int nct, int cus) {
    if (n_tiles <= 0 || nct <= 0 || cus <= 0) return 0;
    // the planned grid at 128 channels a unit: cus / 8 workgroups per XCD rounded down to a
    // multiple of the nct column tiles, each XCD walking its contiguous share of the units a round
    // at a time
    const int64_t g128 = 8 * std::max<int64_t>(1, cus / 8 / nct) * nct;
    const int64_t rounds = n_tiles * nct / g128;
    if (rounds < 1) return 0;
    const int64_t t_split = rounds * (g128 / nct);   // whole rounds of every workgroup
    const int64_t left = n_tiles - t_split;
    if (left <= 0) return 0;
    // the last round's units as 64-channel units: worth it while they make one round of the
    // 64-channel grid (each unit half the products, at 0.64-0.83 of a 128-channel unit's time)
    const int64_t fit64 = std::max<int64_t>(1, cus / 8 / (2 * nct)) * (2 * nct);
    return ceil_div(left * 2 * nct, 8) <= fit64 ? t_split : 0;
}

int halo_conv_launch(int fdt, int odt, const void* feats, int64_t n, int ci, const int32_t* nbr,
                     const void* plan, const void* weight, const float* bias, int co, void* out,
                     hipStream_t s, OctantScatter osc, SkipAdd skip, PadRow pad, RowNorm ln, TileRange tr) {
    const bool planned = plan != nullptr;
    const bool all_tiles = tr.t0 == 0 && tr.nt < 0;
    if (!all_tiles && !planned) {
        set_error("MFMA conv: a tile range needs a plan");
        return TSP_ERR_INVALID;
    }
    if (ln.w && (!planned || !(co == 64 || co == 128) || odt != fdt || osc.cout || skip.cin)) {
        set_error("MFMA conv: a row norm needs a plan, co = 64 or 128 and output in the feature type "
                  "(co=%d)", co);
        return TSP_ERR_UNSUPPORTED;
    }
    const bool bn128 = co % 128 == 0;
    if (osc.cout && (!planned || osc.cout % (bn128 ? 64 : 32) != 0 || (int64_t)osc.cout * 8 != co)) {
        set_error("MFMA conv: an octant scatter needs a plan, co = 8 * cout and cout %% %d == 0 "
                  "(co=%d cout=%d)", bn128 ? 64 : 32, co, osc.cout);
        return TSP_ERR_UNSUPPORTED;
    }
    if (osc.norm_silu && (!bn128 || (osc.cout != 64 && osc.cout != 128) || odt != fdt)) {
        set_error("MFMA conv: octant stores with the child norm need cout = 64 or 128, co %% 128 == 0 and "
                  "output in the feature type (co=%d cout=%d)", co, osc.cout);
        return TSP_ERR_UNSUPPORTED;
    }
    if (skip.cin && (!planned || skip.cin % 8 != 0 || co % (skip.cin / 8) != 0 || (co / (skip.cin / 8)) % 4 != 0)) {
        set_error("MFMA conv: a skip add needs a plan, cin %% 8 == 0 and co / (cin / 8) a multiple of 4 "
                  "(cin=%d co=%d)", skip.cin, co);
        return TSP_ERR_UNSUPPORTED;
    }
    // the slice DMA addresses feature rows with 32-bit byte offsets
    if (!halo_fits(n, ci)) {
        set_error("MFMA conv: n * ci * 2 = %lld bytes of features exceed the 4 GiB the LDS-staged "
                  "kernel addresses", (long long)(n * ci * 2));
        return TSP_ERR_UNSUPPORTED;
    }
    auto* fn64 = fdt == TSP_BF16 ? halo_launch_bf16_64 : halo_launch_f16_64;
    auto* fn = bn128 ? (fdt == TSP_BF16 ? halo_launch_bf16_128 : halo_launch_f16_128) : fn64;
    // With a plan, whole rounds of 128-channel units and the tiles left over as 64-channel units
    // (kernels where either width runs: not the row norms, which need whole rows in a workgroup)
    if (!all_tiles) return fn(odt, planned, feats, n, ci, nbr, plan, weight, bias, co, out, s, osc, skip, pad, ln, tr);
    if (planned && bn128 && !ln.w && !osc.norm_silu) {
        const int64_t t_split = column_split_tiles(ceil_div(n, HB_M), co / 128, cu_count());
        if (t_split > 0) {
            if (int st = fn(odt, planned, feats, n, ci, nbr, plan, weight, bias, co, out, s, osc, skip, pad, ln,
                            TileRange{0, t_split}))
                return st;
            return fn64(odt, planned, feats, n, ci, nbr, plan, weight, bias, co, out, s, osc, skip, pad, ln,
                        TileRange{t_split, -1});
        }
    }
    return fn(odt, planned, feats, n, ci, nbr, plan, weight, bias, co, out, s, osc, skip, pad, ln, TileRange{});
}

}  // namespace tsp
