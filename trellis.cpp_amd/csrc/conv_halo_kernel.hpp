#pragma once
// MFMA submanifold conv with each tile's neighbour rows staged in LDS: the kernel templates and
// their launch, instantiated per (feature dtype, output-channel tile) in conv_halo_*.hip.
//
// A workgroup owns HB_M = 512 consecutive output voxels x BN output channels and runs 8 waves,
// two per SIMD: wave w owns voxels [128 (w%4), +128) x channels [(w/4) BN/2, +BN/2) (the
// kernel is written for any split of RB 32-row x CB 32-column MFMA blocks per wave). On
// sorted surface sets those 512 voxels reference only ~1700 distinct input rows (against
// ~9600 (voxel, tap) pairs), so instead of gathering every pair from L2 the tile gathers each
// distinct row once:
//   * tile plan: mark every referenced row in a bitmap over [lo, hi] (the range of the tile's
//     table entries; one level for spans up to 64K rows, two beyond), exclusive-scan the
//     popcounts, and give each (tap, voxel) its rank in the set -- its slot. Slots are sorted
//     by row, so consecutive voxels at one tap mostly get consecutive slots. Absent taps get
//     the zero slot. The plan depends only on
//     the neighbour table, so it is built once and reused by every conv on that table (the
//     reference shares one table across a decoder stage, shape_decoder.cpp:93-103); without a
//     stored plan the kernel builds it in LDS itself.
//   * the distinct rows stream through LDS 16 channels at a time (two buffers, each a separate
//     LDS object), the next slice loading while the current one runs all 27 taps: each lane
//     loads its 16-byte pieces (a lane pair per row, so a load touches 32 rows) into registers
//     and writes them to LDS a few taps later. Each buffer holds the two 8-channel halves of a
//     row in separate planes, so the 32 lanes that feed one MFMA operand read 32 consecutive
//     16-byte words when the slots are consecutive; absent taps read a zero slot kept past the
//     loaded ones.
//   * per tap, A operands are read from LDS by slot and B operands (weights) come from L2 two
//     taps ahead. Packed weights ([co/32][ci/16][27][64 lanes][8]) make every weight load one
//     contiguous 1 KiB per wave. All 27 taps are unrolled and slices go in pairs, so every
//     register ring index is static and the compiler's load waits are exact.
//   * the epilogue stages row blocks of the accumulators in LDS and writes whole rows.
//   * with a stored plan the grid is persistent (one workgroup per CU, each XCD's workgroups
//     walking its range of tiles) and tiles are pipelined: a tile's last slice loads the next
//     tile's first slice, first weight taps and slot table, so a tile starts with no round trip.
// A tile whose row range or distinct-row count does not fit (scattered or unsorted inputs)
// takes the direct path: the same MFMA loop with A gathered straight from global memory.
// Two more kernels instantiate the same loop for the C2S block with f32 output: its conv1 with
// octant stores (each parent's octant channels go straight to the child rows, so the
// [N][8 Cout] intermediate and the gather pass are never needed) and its conv2 with skip stores
// (the block's repeat-interleaved skip added as the rows are stored).
#include <algorithm>
#include <type_traits>

#include "tile_plan.hpp"

namespace tsp {
namespace {

__device__ __forceinline__ void wait_vmcnt0() { __builtin_amdgcn_s_waitcnt(0x0070 | 0x0f00); }

// The plan of tile row0 (HB_M consecutive rows) built in LDS by the conv itself when no stored
// plan is given: tile positions are the rows in order.
template <int NT>
__device__ void tile_plan(const int32_t* __restrict__ nbr, int64_t n, int64_t row0,
                          uint16_t (*sL)[4][32][4], int32_t* sRowOf, uint32_t* scratch,
                          int* sRed, int& H_out, bool& direct_out) {
    constexpr int VPT = HB_M / NT;         // voxels per thread
    const int tid = threadIdx.x;
    int64_t i[VPT];
    int pos[VPT];
#pragma unroll
    for (int h = 0; h < VPT; ++h) {
        pos[h] = tid + NT * h;
        i[h] = row0 + pos[h] < n ? row0 + pos[h] : -1;
    }
    int32_t nv[kTaps][VPT];
    load_entries<VPT>(nbr, n, i, nv);
    tile_plan_core<NT, VPT>(nv, pos, sL, sRowOf, scratch, sRed, H_out, direct_out);
}


// ---- the conv ---------------------------------------------------------------------------------
// WAVES = 4 (one wave per SIMD, each owning 128 voxels x all BN channels, accumulators in the
// upper register file, weights PD taps ahead) or 8 (two per SIMD, each 128 voxels x BN/2).
template <int BN, int RB, int CB>
constexpr int hb_waves() { return (HB_M / (32 * RB)) * (BN / (32 * CB)); }

template <bool BF16, int BN, int ODT, bool PLANNED, int RB, int CB, int PD, int SP, int STG, int EPI>
__device__ __forceinline__ void conv_tiles(
    const uint16_t* __restrict__ feats, int64_t n, int ci, const int32_t* __restrict__ nbr,
    PlanView plan, const uint16_t* __restrict__ weight, const float* __restrict__ bias, int co,
    void* __restrict__ out, int n_ctiles, int64_t lin0, int64_t stride, int64_t xhi,
    uint16_t (&sH0)[2][HB_ROWS][8], uint16_t (&sH1)[2][HB_ROWS][8],
    uint16_t (&sL)[kTaps][4][32][4], int* sRed, OctantScatter osc, SkipAdd skip, PadRow pad, RowNorm ln);

template <bool BF16, int BN, int ODT, bool PLANNED, int RB, int CB, int PD, int SP, int STG, int EPI>
__device__ __forceinline__ void conv_grid(
    const uint16_t* __restrict__ feats, int64_t n, int ci, const int32_t* __restrict__ nbr,
    PlanView plan, const uint16_t* __restrict__ weight, const float* __restrict__ bias, int co,
    void* __restrict__ out, int64_t n_tiles, int n_ctiles, int64_t per_xcd, OctantScatter osc,
    SkipAdd skip, PadRow pad, RowNorm ln) {
    // wave w owns voxels [32 RB rg, +32 RB) x channels [32 CB cg, +32 CB) of the tile, with
    // rg = w % NRG and cg = w / NRG
    constexpr int NRG = HB_M / (32 * RB), NCG = BN / (32 * CB);
    constexpr int WAVES = NRG * NCG;
    constexpr int NT = WAVES * 64;
    static_assert(WAVES == 4 || WAVES == 8, "4 or 8 waves");
    static_assert(RB % 4 == 0 && HB_M % (32 * RB) == 0 && BN % (32 * CB) == 0, "tile split");
    // the two slice buffers [half][slot][8 ch] -- separate objects, so that alias analysis sees
    // that the writes into one never feed the reads of the other and the compiler need not wait
    // for them before every LDS read -- and the slot table [tap][row block][voxel%32][rb]
    __shared__ __attribute__((aligned(16))) uint16_t sH0[2][HB_ROWS][8];
    __shared__ __attribute__((aligned(16))) uint16_t sH1[2][HB_ROWS][8];
    __shared__ __attribute__((aligned(16))) uint16_t sL[kTaps][4][32][4];
    __shared__ int sRed[2 * NT / 64];

    // XCD-aware order: workgroup ids go round-robin over the 8 XCDs, so each XCD gets one
    // contiguous range of (tile, column-tile) pairs and gathers from rows its L2 already holds.
    // The workgroups of an XCD walk its range with a stride of their count (a multiple of
    // n_ctiles, so a workgroup keeps one column tile): with a stored plan the grid is one
    // workgroup per CU, otherwise one workgroup per pair.
    const int64_t total = n_tiles * n_ctiles;
    const int xcd = (int)(blockIdx.x % 8);
    const int64_t xlo = xcd * per_xcd, xhi = xlo + per_xcd < total ? xlo + per_xcd : total;
    conv_tiles<BF16, BN, ODT, PLANNED, RB, CB, PD, SP, STG, EPI>(
        feats, n, ci, nbr, plan, weight, bias, co, out, n_ctiles, xlo + blockIdx.x / 8,
        gridDim.x / 8, xhi, sH0, sH1, sL, sRed, osc, skip, pad, ln);
}

template <bool BF16, int BN, int ODT, bool PLANNED, int RB, int CB, int PD, int SP, int STG>
__global__ __launch_bounds__((hb_waves<BN, RB, CB>() * 64), 1) void k_conv_halo(
    const uint16_t* __restrict__ feats, int64_t n, int ci, const int32_t* __restrict__ nbr,
    PlanView plan, const uint16_t* __restrict__ weight, const float* __restrict__ bias, int co,
    void* __restrict__ out, int64_t n_tiles, int n_ctiles, int64_t per_xcd, PadRow pad) {
    conv_grid<BF16, BN, ODT, PLANNED, RB, CB, PD, SP, STG, 0>(
        feats, n, ci, nbr, plan, weight, bias, co, out, n_tiles, n_ctiles, per_xcd, OctantScatter{},
        SkipAdd{}, pad, RowNorm{});
}

// The same conv with f32 output rows scattered to the children of a 2x subdivision (stored plan).
template <bool BF16, int BN, int RB, int CB, int PD, int SP, int STG>
__global__ __launch_bounds__((hb_waves<BN, RB, CB>() * 64), 1) void k_conv_halo_octants(
    const uint16_t* __restrict__ feats, int64_t n, int ci, const int32_t* __restrict__ nbr,
    PlanView plan, const uint16_t* __restrict__ weight, const float* __restrict__ bias, int co,
    void* __restrict__ out, int64_t n_tiles, int n_ctiles, int64_t per_xcd, OctantScatter osc,
    PadRow pad) {
    conv_grid<BF16, BN, TSP_F32, true, RB, CB, PD, SP, STG, 1>(
        feats, n, ci, nbr, plan, weight, bias, co, out, n_tiles, n_ctiles, per_xcd, osc, SkipAdd{}, pad,
        RowNorm{});
}

// The same octant stores with each child row normalised (no affine) and passed through SiLU, in
// the feature type (stored plan, cout == the channels of one wave).
template <bool BF16, int BN, int RB, int CB, int PD, int SP, int STG>
__global__ __launch_bounds__((hb_waves<BN, RB, CB>() * 64), 1) void k_conv_halo_octants_norm(
    const uint16_t* __restrict__ feats, int64_t n, int ci, const int32_t* __restrict__ nbr,
    PlanView plan, const uint16_t* __restrict__ weight, const float* __restrict__ bias, int co,
    void* __restrict__ out, int64_t n_tiles, int n_ctiles, int64_t per_xcd, OctantScatter osc,
    PadRow pad) {
    conv_grid<BF16, BN, BF16 ? TSP_BF16 : TSP_F16, true, RB, CB, PD, SP, STG, 4>(
        feats, n, ci, nbr, plan, weight, bias, co, out, n_tiles, n_ctiles, per_xcd, osc, SkipAdd{}, pad,
        RowNorm{});
}

// The same with cout == BN: each child row normalised across the workgroup's two column waves
// (as k_conv_halo_ln, no affine) and passed through SiLU.
template <bool BF16, int BN, int RB, int CB, int PD, int SP, int STG>
__global__ __launch_bounds__((hb_waves<BN, RB, CB>() * 64), 1) void k_conv_halo_octants_rownorm(
    const uint16_t* __restrict__ feats, int64_t n, int ci, const int32_t* __restrict__ nbr,
    PlanView plan, const uint16_t* __restrict__ weight, const float* __restrict__ bias, int co,
    void* __restrict__ out, int64_t n_tiles, int n_ctiles, int64_t per_xcd, OctantScatter osc,
    PadRow pad) {
    conv_grid<BF16, BN, BF16 ? TSP_BF16 : TSP_F16, true, RB, CB, PD, SP, STG, 5>(
        feats, n, ci, nbr, plan, weight, bias, co, out, n_tiles, n_ctiles, per_xcd, osc, SkipAdd{}, pad,
        RowNorm{});
}

// The same conv with f32 output and the C2S skip added by its stores (stored plan).
template <bool BF16, int BN, int RB, int CB, int PD, int SP, int STG>
__global__ __launch_bounds__((hb_waves<BN, RB, CB>() * 64), 1) void k_conv_halo_skip(
    const uint16_t* __restrict__ feats, int64_t n, int ci, const int32_t* __restrict__ nbr,
    PlanView plan, const uint16_t* __restrict__ weight, const float* __restrict__ bias, int co,
    void* __restrict__ out, int64_t n_tiles, int n_ctiles, int64_t per_xcd, SkipAdd skip,
    PadRow pad) {
    conv_grid<BF16, BN, TSP_F32, true, RB, CB, PD, SP, STG, 2>(
        feats, n, ci, nbr, plan, weight, bias, co, out, n_tiles, n_ctiles, per_xcd, OctantScatter{}, skip, pad, RowNorm{});
}

// The same conv with the ConvNeXt block's LayerNorm done by its stores (stored plan, co == BN,
// output in the feature type).
template <bool BF16, int BN, int RB, int CB, int PD, int SP, int STG>
__global__ __launch_bounds__((hb_waves<BN, RB, CB>() * 64), 1) void k_conv_halo_ln(
    const uint16_t* __restrict__ feats, int64_t n, int ci, const int32_t* __restrict__ nbr,
    PlanView plan, const uint16_t* __restrict__ weight, const float* __restrict__ bias, int co,
    void* __restrict__ out, int64_t n_tiles, int n_ctiles, int64_t per_xcd, PadRow pad, RowNorm ln) {
    conv_grid<BF16, BN, BF16 ? TSP_BF16 : TSP_F16, true, RB, CB, PD, SP, STG, 3>(
        feats, n, ci, nbr, plan, weight, bias, co, out, n_tiles, n_ctiles, per_xcd, OctantScatter{}, SkipAdd{},
        pad, ln);
}

// The tiles lin0, lin0 + stride, ... (< xhi) of one workgroup. With a stored plan and an even
// number of slices, tiles are pipelined: the last slice of a tile streams the next tile's first
// slice into the idle buffer, the first taps of its weights into the ring and its slot table into
// registers, so the next tile starts without a memory round trip and its loads are in flight
// before this tile's output stores.
template <bool BF16, int BN, int ODT, bool PLANNED, int RB, int CB, int PD, int SP, int STG, int EPI>
__device__ __forceinline__ void conv_tiles(
    const uint16_t* __restrict__ feats, int64_t n, int ci, const int32_t* __restrict__ nbr,
    PlanView plan, const uint16_t* __restrict__ weight, const float* __restrict__ bias, int co,
    void* __restrict__ out, int n_ctiles, int64_t lin0, int64_t stride, int64_t xhi,
    uint16_t (&sH0)[2][HB_ROWS][8], uint16_t (&sH1)[2][HB_ROWS][8],
    uint16_t (&sL)[kTaps][4][32][4], int* sRed, OctantScatter osc, SkipAdd skip, PadRow pad, RowNorm ln) {
    constexpr int NRG = HB_M / (32 * RB), NCG = BN / (32 * CB);
    constexpr int WAVES = NRG * NCG;
    constexpr int NT = WAVES * 64;
    constexpr int WN = 32 * CB;              // output channels per wave
    constexpr int PIECES = 2 * HB_SLOTS / 64 / WAVES;   // slice loads per wave and slice
    constexpr int NSTG = (STG + SP - 1) / SP + 1;       // slice pieces in flight
    constexpr int SLOT_BLOCKS = (HB_SLOT_TABLE * 2 / 1024 + WAVES - 1) / WAVES;   // 1 KiB each
    constexpr int T_FREE = (PIECES - 1) * SP + STG + 1;   // first tap with the piece ring idle

    const int tid = threadIdx.x;
    const int wave = tid >> 6;
    const int wave_s = __builtin_amdgcn_readfirstlane(wave);   // the same, as a uniform value
    // lane-dependent values are re-defined (by an empty asm) at every tile, so that the
    // compiler does not hoist the unrolled loops' per-tap addresses out of the tile loop and
    // keep them all in registers
    int lane = tid & 63;
    int r32 = lane & 31, g = lane >> 5;
    int rg = wave % NRG;                     // row group: voxels [32 RB rg, +32 RB)
    const int c0 = (int)(lin0 % n_ctiles) * BN + (wave / NRG) * WN;   // first channel of wave
    // with an octant scatter, the wave's channels lie in octant oct, from column ocol of a child
    const int oct = EPI == 1 || EPI == 4 || EPI == 5 ? c0 / osc.cout : 0;
    const int ocol = EPI == 1 || EPI == 4 || EPI == 5 ? c0 - oct * osc.cout : 0;
    const int nkc = ci / HB_KC;
    // The reference's absent taps read the padding row 0 * feats[0] (submconv_pad,
    // sparse.cpp:81-85), zeros here. Where row 0 holds an Inf or a NaN that row is NaN in those
    // channels, so every output row with an absent tap is NaN in every channel: the epilogue then
    // writes NaN for those rows (found in the table), as the reference's sum would. With a zero
    // padding row (the C2S conv2) nothing is tested; with an f32 source row, that row is tested.
    bool row0_bad = false;
    if (!pad.zero) {
        if (pad.row0) {
            for (int k = tid; k < ci; k += NT) row0_bad |= !__builtin_isfinite(pad.row0[k]);
        } else {
            for (int k = tid * 8; k < ci; k += NT * 8) {
                const u32x4_t v = *reinterpret_cast<const u32x4_t*>(feats + k);
                constexpr uint32_t kExp = BF16 ? 0x7F807F80u : 0x7C007C00u;
#pragma unroll
                for (int e = 0; e < 4; ++e)
                    row0_bad |= ((v[e] & kExp & 0xffffu) == (kExp & 0xffffu)) ||
                                ((v[e] & kExp & 0xffff0000u) == (kExp & 0xffff0000u));
            }
        }
    }
    row0_bad = __syncthreads_or(row0_bad);
    // A tap absent from all 32 rows of an MFMA block (the plan's act bit clear) only adds the zero
    // slot times W: exact zeros when the weights are finite (the packed weights' trailer says
    // so), so its MFMAs and A reads are skipped; with an Inf or a NaN in W every block is computed.
    bool may_skip = false;
    if constexpr (PLANNED)
        may_skip = *reinterpret_cast<const uint32_t*>(reinterpret_cast<const char*>(weight) +
                                                      (size_t)kTaps * ci * co * 2) == 0u;
    // act words of this wave's row group for the current tile (wave-uniform; all set = no skip)
    uint32_t ab[HB_ACT_WORDS];
#pragma unroll
    for (int k = 0; k < HB_ACT_WORDS; ++k) ab[k] = ~0u;
    auto load_act = [&](int64_t tl, uint32_t (&dst)[HB_ACT_WORDS]) {
        const int rgs = __builtin_amdgcn_readfirstlane(rg);
#pragma unroll
        for (int k = 0; k < HB_ACT_WORDS; ++k)
            dst[k] = may_skip ? (uint32_t)__builtin_amdgcn_readfirstlane(
                                    (int)plan.act[(tl * 4 + rgs) * HB_ACT_WORDS + k])
                              : ~0u;
    };
    // With octant stores: the wave's 4 blocks that hold a parent keeping the wave's octant
    // (wave-uniform; all set when the caller gave no block words). Every tap's MFMAs of the other
    // blocks are skipped, whatever the weights: their outputs are never stored.
    uint32_t ob = 15u;
    auto load_ob = [&](int64_t tl) -> uint32_t {
        if constexpr (EPI == 1 || EPI == 4 || EPI == 5) {
            if (osc.blocks) {
                const int rgs = __builtin_amdgcn_readfirstlane(rg);
                const uint32_t w = (uint32_t)__builtin_amdgcn_readfirstlane((int)osc.blocks[tl * 4 + rgs]);
                return (w >> (4 * __builtin_amdgcn_readfirstlane(oct))) & 15u;
            }
        }
        return 15u;
    };
    // the act bits of tap t for the wave's 4 blocks (t compile-time after unrolling). The empty
    // asm re-reads the word in a scalar register at each use: the tests stay scalar branches on
    // it, rather than 108 lane masks computed once and spilled.
    auto tap_bits = [&](int t) -> uint32_t {
        uint32_t v = (uint32_t)__builtin_amdgcn_readfirstlane((int)ab[(4 * t) >> 5]);
        asm volatile("" : "+s"(v));
        return (v >> ((4 * t) & 31)) & ob;
    };

    // slice loads: wave w streams the 32-slot blocks w + WAVES j, lane pairs loading the two
    // planes of one row (32 contiguous bytes; a load touches 32 rows, not 64)
    int plane = lane & 1;
    auto piece_slot = [&](int j) { return 32 * (wave + WAVES * j); };
    // cross-tile pipelining needs slices in pairs and the slot table in the idle piece ring
    constexpr bool CAN_PIPE = PLANNED && WAVES == 8 && SLOT_BLOCKS <= NSTG && T_FREE < kTaps;

    // the bias of this lane's output channels (one column tile per workgroup)
    float bv[CB];
#pragma unroll
    for (int cb = 0; cb < CB; ++cb) bv[cb] = bias[c0 + cb * 32 + r32];

    // weights of (tap t, slice kc), column block cb of this wave
    uint32_t boff[CB];
#pragma unroll
    for (int cb = 0; cb < CB; ++cb) {
        if constexpr (PLANNED)   // packed: block ((co/32 index) * nkc + kc) * 27 + t, 1 KiB each
            boff[cb] = (uint32_t)((((c0 >> 5) + cb) * nkc * kTaps * 64 + lane) * 16u);
        else                     // [co][27][ci]
            boff[cb] = (uint32_t)(((uint32_t)(c0 + cb * 32 + r32) * (uint32_t)(kTaps * ci) + g * 8) * 2u);
    }
    // The tap's base address is wave-uniform and each lane adds a 32-bit offset (the
    // scalar-base + vector-offset load form). The empty asm hides that boff is the same for every
    // tap; otherwise the compiler precomputes a 64-bit address per (tap, column block) of the
    // unrolled loop and runs out of registers.
    auto load_b = [&](int t, int kc, u32x4_t* dst) {
        const char* wt;
        if constexpr (PLANNED) wt = reinterpret_cast<const char*>(weight) + ((int64_t)kc * kTaps + t) * 1024;
        else wt = reinterpret_cast<const char*>(weight + (t * ci + kc * HB_KC));
#pragma unroll
        for (int cb = 0; cb < CB; ++cb) {
            uint32_t o = boff[cb];
            asm volatile("" : "+v"(o));
            dst[cb] = *reinterpret_cast<const u32x4_t*>(wt + o);
        }
    };

    // byte offset (from feats) of the 8 channels this lane copies for each slice piece at
    // slice 0: row * ci * 2 + plane * 16; slots past H copy row 0 into an unused slot
    uint32_t poff[PIECES];
    auto set_poff = [&](int32_t (&prow)[PIECES], int H) {
#pragma unroll
        for (int j = 0; j < PIECES; ++j) {
            const int32_t r = (piece_slot(j) + (lane >> 1) < H && (uint32_t)prow[j] < (uint32_t)n) ? prow[j] : 0;
            poff[j] = (uint32_t)r * (uint32_t)ci * 2u + plane * 16u;
            // kept as 32-bit offsets for the scalar-base + vector-offset load form
            asm volatile("" : "+v"(poff[j]));
        }
    };
    auto fetch_piece = [&](int kc, int j, u32x4_t& r) {
        r = *reinterpret_cast<const u32x4_t*>(reinterpret_cast<const char*>(feats) + poff[j] +
                                              (uint32_t)kc * (HB_KC * 2));
    };
    auto put_piece = [&](uint16_t (*dst)[HB_ROWS][8], int j, const u32x4_t& r) {
        *reinterpret_cast<u32x4_t*>(&dst[plane][piece_slot(j) + (lane >> 1)][0]) = r;
    };
    // A operands of tap t: per 128 voxels one 8-byte read of four slots, then one 16-byte
    // read per 32-row block
    static_assert(RB == 4, "act bits cover the 4 blocks of a row group");
    auto load_a = [&](const uint16_t (*cur)[HB_ROWS][8], int t, u32x4_t* a) {
        const uint2 sl = *reinterpret_cast<const uint2*>(&sL[t][rg][r32][0]);
        const int slots[4] = {(int)(sl.x & 0xffffu), (int)(sl.x >> 16),
                              (int)(sl.y & 0xffffu), (int)(sl.y >> 16)};
#pragma unroll
        for (int k = 0; k < 4; ++k) a[k] = *reinterpret_cast<const u32x4_t*>(&cur[g][slots[k]][0]);
    };
    // zero slot of both planes of a buffer (a barrier before its first read publishes it)
    auto zero_slot = [&](uint16_t (*buf)[HB_ROWS][8]) {
        if (tid < 2) {
            u32x4_t z{0, 0, 0, 0};
            asm volatile("" : "+v"(z));   // made here, not held in registers across tiles
            *reinterpret_cast<u32x4_t*>(&buf[tid][HB_ZERO][0]) = z;
        }
    };
    // Each path below owns its accumulators (zeroed there and passed to the epilogue): one set
    // live across both paths would be zeroed in the lower registers and spilled.
    auto zero = [](f32x16_t (&acc)[RB][CB]) {
#pragma unroll
        for (int rb = 0; rb < RB; ++rb)
#pragma unroll
            for (int cb = 0; cb < CB; ++cb)
#pragma unroll
                for (int j = 0; j < 16; ++j) acc[rb][cb][j] = 0.f;
    };

    // ---- epilogue: each wave stages row blocks of its accumulators (fp32, + bias) in its own part
    // of the slice buffers (idle: every wave passed the last barrier of the main loop, or never
    // used them on the direct path), then writes whole row segments, 16 bytes per lane. The row
    // stride WN*4+32 bytes puts the two 32-lane halves of a staging write on disjoint banks.
    // NR rows at a time: 32 over both buffers, or 16 in sH1 alone while sH0 holds the next
    // tile's first slice.
    auto epilogue = [&](auto nr_c, f32x16_t (&acc)[RB][CB], int64_t tile) {
        constexpr int NR = decltype(nr_c)::value;
        constexpr int RS = WN * 4 + 32;
        static_assert(NR == 32 || NR == 16, "row rounds of 32 or 16");
        static_assert((NR == 32 ? WAVES / 2 : WAVES) * NR * RS <= (int)sizeof(sH0),
                      "staging must fit a slice buffer");
        char* stage = NR == 32 ? reinterpret_cast<char*>(wave < WAVES / 2 ? &sH0[0][0][0] : &sH1[0][0][0]) +
                                     (wave % (WAVES / 2)) * 32 * RS
                               : reinterpret_cast<char*>(&sH1[0][0][0]) + wave * 16 * RS;
        constexpr int CH = ODT == TSP_F32 ? 4 : 8;     // channels per 16-byte store
        constexpr int NQ = NR * (WN / CH) / 64;        // stores per lane and round
        static_assert(NR * (WN / CH) % 64 == 0, "whole stores per lane");
        // The output row of each of the wave's 32 RB tile positions (the plan's order, or the
        // tile's rows in order without one), -1 where there is none: lane l holds positions 2l and
        // 2l + 1, and row_at(lr) shuffles position lr's row to the lane that stores it.
        static_assert(RB == 4, "two positions per lane");
        int vrow[2];
#pragma unroll
        for (int k = 0; k < 2; ++k) {
            const int p = 32 * RB * rg + 2 * lane + k;
            if constexpr (PLANNED) vrow[k] = plan.vox[tile * HB_M + p];
            else vrow[k] = tile * HB_M + p < n ? (int)(tile * HB_M + p) : -1;
        }
        auto row_at = [&](int lr) {
            const int a = __shfl(vrow[0], lr >> 1, 64), b = __shfl(vrow[1], lr >> 1, 64);
            return (lr & 1) ? b : a;
        };
        // Octant stores: the child row of octant oct of each of the wave's rows, or -1, looked up
        // once per tile for the lane's two positions and shuffled the same way.
        int child2[2] = {-1, -1};
        if constexpr (EPI == 1 || EPI == 4) {
#pragma unroll
            for (int k = 0; k < 2; ++k) {
                const int64_t i = vrow[k];
                if (i >= 0) {
                    constexpr uint64_t kLow7 = 0x7f7f7f7f7f7f7f7full;
                    const uint64_t mw = *reinterpret_cast<const uint64_t*>(osc.mask + 8 * i);
                    const uint64_t kept = (((mw & kLow7) + kLow7) | mw) & ~kLow7;   // bit 8b+7: byte b != 0
                    const int rank = __popcll(kept & ((1ull << (8 * oct)) - 1));
                    child2[k] = ((kept >> (8 * oct + 7)) & 1) ? osc.mstart[i] + rank : -1;
                }
            }
        }
        // Skip add: the gidx of each of the wave's rows (-1 for none), looked up and shuffled
        // the same way.
        int gidx2[2] = {-1, -1};
        if constexpr (EPI == 2) {
#pragma unroll
            for (int k = 0; k < 2; ++k)
                if (vrow[k] >= 0) gidx2[k] = skip.gidx[vrow[k]];
        }
        // the skip elements of round (rb, h), one per store (its 4 channels share one); loaded a
        // round ahead of their use, so the loads' latency overlaps a round of staging and stores
        auto skip_vals = [&](int rb, int h, float (&sv)[NQ]) {
#pragma unroll
            for (int q = 0; q < NQ; ++q) {
                const int c = q * 64 + lane;
                const int r = c / (WN / CH), cq = c % (WN / CH);
                const int lr = 32 * rb + NR * h + r;
                const int a = __shfl(gidx2[0], lr >> 1, 64), b = __shfl(gidx2[1], lr >> 1, 64);
                const int gi = (lr & 1) ? b : a;
                const int kk = skip.cin / 8, rep_r = co / kk;
                sv[q] = gi >= 0 ? skip.x[(int64_t)(gi >> 3) * skip.cin + (gi & 7) * kk + (c0 + cq * CH) / rep_r]
                                : 0.f;
            }
        };
        float sv_cur[NQ] = {}, sv_nxt[NQ] = {};
        if constexpr (EPI == 2) skip_vals(0, 0, sv_cur);
        // a plain conv with 16-bit output stages the rounded values: half the LDS bytes, the same
        // bits (the one rounding happens before the staging instead of after it)
        constexpr bool S16 = EPI == 0 && ODT != TSP_F32;
        constexpr int RS16 = WN * 2 + 16;
        static_assert(!S16 || (RS16 % 16 == 0 && (NR == 32 ? WAVES / 2 : WAVES) * NR * RS16 <= (int)sizeof(sH0)),
                      "16-bit staging");
        if constexpr (S16) {
#pragma unroll
            for (int rb = 0; rb < RB; ++rb) {
#pragma unroll
                for (int h = 0; h < 32 / NR; ++h) {
#pragma unroll
                    for (int cb = 0; cb < CB; ++cb)
#pragma unroll
                        for (int j = 16 * h * NR / 32; j < 16 * (h + 1) * NR / 32; j += 2) {
                            const int r = 8 * (j / 4) + 4 * g + (j % 4) - NR * h;   // rows r, r + 1
                            const float a = acc[rb][cb][j] + bv[cb], b = acc[rb][cb][j + 1] + bv[cb];
                            const uint32_t pk = ODT == TSP_BF16 ? f32x2_to_bf16x2_bits(a, b)
                                                                : f32_to_f16_bits(a) | ((uint32_t)f32_to_f16_bits(b) << 16);
                            char* at = stage + r * RS16 + (cb * 32 + r32) * 2;
                            *reinterpret_cast<uint16_t*>(at) = (uint16_t)(pk & 0xffffu);
                            *reinterpret_cast<uint16_t*>(at + RS16) = (uint16_t)(pk >> 16);
                        }
                    constexpr int NQ16 = NR * (WN / 8) / 64;
                    u32x4_t v16[NQ16];
#pragma unroll
                    for (int q = 0; q < NQ16; ++q) {
                        const int c = q * 64 + lane;
                        v16[q] = *reinterpret_cast<const u32x4_t*>(stage + (c / (WN / 8)) * RS16 + (c % (WN / 8)) * 16);
                    }
#pragma unroll
                    for (int q = 0; q < NQ16; ++q) {
                        const int c = q * 64 + lane;
                        const int r = c / (WN / 8), cq = c % (WN / 8);
                        const int64_t i = row_at(32 * rb + NR * h + r);
                        if (i < 0) continue;
                        if (row0_bad) {
                            bool absent = false;
                            for (int t = 0; t < kTaps; ++t) absent |= nbr[(int64_t)t * n + i] == (int32_t)n;
                            if (absent) {
                                constexpr uint32_t kNaN2 = ODT == TSP_BF16 ? 0x7FC07FC0u : 0x7E007E00u;
                                v16[q] = u32x4_t{kNaN2, kNaN2, kNaN2, kNaN2};
                            }
                        }
                        *reinterpret_cast<u32x4_t*>(reinterpret_cast<uint16_t*>(out) + i * co + c0 + cq * 8) = v16[q];
                    }
                }
            }
            return;
        }
#pragma unroll
        for (int rb = 0; rb < RB; ++rb) {
#pragma unroll
            for (int h = 0; h < 32 / NR; ++h) {
#pragma unroll
                for (int cb = 0; cb < CB; ++cb)
#pragma unroll
                    for (int j = 16 * h * NR / 32; j < 16 * (h + 1) * NR / 32; ++j) {
                        const int r = 8 * (j / 4) + 4 * g + (j % 4) - NR * h;
                        *reinterpret_cast<float*>(stage + r * RS + (cb * 32 + r32) * 4) = acc[rb][cb][j] + bv[cb];
                    }
                // NR rows x WN/CH chunks: all LDS reads first (one wait), then the stores
                f32x4_t vs[NQ][CH / 4];
#pragma unroll
                for (int q = 0; q < NQ; ++q) {
                    const int c = q * 64 + lane;
                    const char* p = stage + (c / (WN / CH)) * RS + (c % (WN / CH)) * (CH * 4);
#pragma unroll
                    for (int e = 0; e < CH / 4; ++e) vs[q][e] = *reinterpret_cast<const f32x4_t*>(p + 16 * e);
                }
                if constexpr (EPI == 2) {
                    constexpr int NH = 32 / NR;
                    if (h + 1 < NH) skip_vals(rb, h + 1, sv_nxt);
                    else if (rb + 1 < RB) skip_vals(rb + 1, 0, sv_nxt);
                }
#pragma unroll
                for (int q = 0; q < NQ; ++q) {
                    const int c = q * 64 + lane;
                    const int r = c / (WN / CH), cq = c % (WN / CH);
                    const int64_t i = row_at(32 * rb + NR * h + r);
                    int64_t o = i * co + c0 + cq * CH;
                    bool keep = i >= 0;
                    if (row0_bad && keep) {
                        bool absent = false;
                        for (int t = 0; t < kTaps; ++t) absent |= nbr[(int64_t)t * n + i] == (int32_t)n;
                        if (absent) {
#pragma unroll
                            for (int e = 0; e < CH / 4; ++e) vs[q][e] = f32x4_t{NAN, NAN, NAN, NAN};
                        }
                    }
                    if constexpr (EPI == 4) {
                        // the child row's norm (its WN channels: the WN / CH lanes of this row) + SiLU
                        static_assert(EPI != 4 || (ODT != TSP_F32 && WN / CH == 8), "one row per 8 lanes");
                        float sum = 0.f;
#pragma unroll
                        for (int e = 0; e < CH / 4; ++e)
#pragma unroll
                            for (int k = 0; k < 4; ++k) sum += vs[q][e][k];
                        const float mean = group_sum<WN / CH>(sum) / (float)WN;
                        float sq = 0.f;
#pragma unroll
                        for (int e = 0; e < CH / 4; ++e)
#pragma unroll
                            for (int k = 0; k < 4; ++k) {
                                const float d = vs[q][e][k] - mean;
                                sq += d * d;
                            }
                        const float rstd = 1.0f / sqrtf(group_sum<WN / CH>(sq) / (float)WN + osc.norm_eps);
#pragma unroll
                        for (int e = 0; e < CH / 4; ++e)
#pragma unroll
                            for (int k = 0; k < 4; ++k) {
                                // (hardware exp and reciprocal: the value is rounded to 16 bits next)
                                const float y = (vs[q][e][k] - mean) * rstd;
                                vs[q][e][k] = y * __builtin_amdgcn_rcpf(1.0f + __expf(-y));
                            }
                    }
                    if constexpr (EPI == 1 || EPI == 4) {
                        // parent row lr of the wave: its child of octant oct (or -1)
                        const int lr = 32 * rb + NR * h + r;
                        const int a = __shfl(child2[0], lr >> 1, 64), b = __shfl(child2[1], lr >> 1, 64);
                        const int child = (lr & 1) ? b : a;
                        keep = keep && child >= 0;
                        o = (int64_t)child * osc.cout + ocol + cq * CH;
                    }
                    if constexpr (EPI == 2) {
                        // child row: + x[gidx / 8][(gidx % 8) K + c / R]
#pragma unroll
                        for (int e = 0; e < 4; ++e) vs[q][0][e] += sv_cur[q];
                    }
                    if (keep) {
                        if constexpr (ODT == TSP_F32) {
                            *reinterpret_cast<f32x4_t*>(reinterpret_cast<float*>(out) + o) = vs[q][0];
                            if constexpr (EPI == 2) {
                                if (skip.out16) {
                                    const f32x4_t v = vs[q][0];
                                    const uint2 w16 = skip.out16_bf16
                                        ? uint2{f32x2_to_bf16x2_bits(v[0], v[1]), f32x2_to_bf16x2_bits(v[2], v[3])}
                                        : uint2{f32_to_f16_bits(v[0]) | ((uint32_t)f32_to_f16_bits(v[1]) << 16),
                                                f32_to_f16_bits(v[2]) | ((uint32_t)f32_to_f16_bits(v[3]) << 16)};
                                    *reinterpret_cast<uint2*>(static_cast<uint16_t*>(skip.out16) + o) = w16;
                                }
                            }
                        } else {
                            uint32_t w[4];
#pragma unroll
                            for (int e = 0; e < 4; ++e) {
                                const float lo = vs[q][e / 2][(2 * e) % 4], hi = vs[q][e / 2][(2 * e) % 4 + 1];
                                w[e] = (ODT == TSP_BF16) ? f32x2_to_bf16x2_bits(lo, hi)
                                                         : f32_to_f16_bits(lo) | ((uint32_t)f32_to_f16_bits(hi) << 16);
                            }
                            *reinterpret_cast<u32x4_t*>(reinterpret_cast<uint16_t*>(out) + o) =
                                u32x4_t{w[0], w[1], w[2], w[3]};
                        }
                    }
                }
                if constexpr (EPI == 2) {
#pragma unroll
                    for (int q = 0; q < NQ; ++q) sv_cur[q] = sv_nxt[q];
                }
            }
        }
    };

    // ---- row-norm epilogue (EPI 3: co == BN, so the workgroup holds every channel of its rows):
    // in rounds of 16 rows of each row group, both column waves stage their halves of the rows
    // (f32, + bias) in sH1 as whole rows; then each wave normalises 8 of the rows, 16 lanes a row
    // (BN / 16 consecutive channels each), with the row's sums reduced over those lanes: the mean,
    // then the mean square deviation, rstd = 1 / sqrt(var + eps), y = (x - mean) rstd w + b,
    // stored in the 16-bit output type, one contiguous row segment per lane.
    auto epilogue_ln = [&](f32x16_t (&acc)[RB][CB], int64_t tile) {
        constexpr int RR = 16;                   // rows per round and row group
        constexpr int RSW = BN * 4 + 16;         // staged row stride in bytes
        constexpr int CPL = BN / 16;             // channels per lane
        constexpr bool RN = EPI == 3 || EPI == 5;
        static_assert(!RN || (NCG == 2 && RB == 4 && NRG * RR * RSW <= (int)sizeof(sH1)), "row-norm staging");
        static_assert(!RN || ODT == TSP_BF16 || ODT == TSP_F16, "row norm stores 16-bit rows");
        char* stage = reinterpret_cast<char*>(&sH1[0][0][0]) + rg * RR * RSW;
        const int cg = wave / NRG;
        int vrow[2];
#pragma unroll
        for (int k = 0; k < 2; ++k) vrow[k] = plan.vox[tile * HB_M + 32 * RB * rg + 2 * lane + k];
        auto row_at = [&](int lr) {
            const int a = __shfl(vrow[0], lr >> 1, 64), b = __shfl(vrow[1], lr >> 1, 64);
            return (lr & 1) ? b : a;
        };
        const int lc = (lane & 15) * CPL;        // this lane's first channel
        float gw[CPL], gb[CPL];
#pragma unroll
        for (int e = 0; e < CPL; ++e) {
            gw[e] = EPI == 5 ? 1.f : ln.w[lc + e];   // (EPI 5: no affine)
            gb[e] = EPI == 5 ? 0.f : ln.b[lc + e];
        }
#pragma unroll
        for (int rb = 0; rb < RB; ++rb) {
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                // element j of a block holds row 8 (j / 4) + 4 g + j % 4: rows 16 h .. 16 h + 15
#pragma unroll
                for (int cb = 0; cb < CB; ++cb)
#pragma unroll
                    for (int j = 8 * h; j < 8 * h + 8; ++j) {
                        const int r = 8 * (j / 4) + 4 * g + (j % 4) - 16 * h;
                        *reinterpret_cast<float*>(stage + r * RSW + (cg * WN + cb * 32 + r32) * 4) =
                            acc[rb][cb][j] + bv[cb];
                    }
                __syncthreads();
#pragma unroll
                for (int bt = 0; bt < 2; ++bt) {
                    const int r = 8 * cg + 4 * bt + (lane >> 4);          // row of the round
                    float v[CPL];
#pragma unroll
                    for (int e = 0; e < CPL; e += 4) {
                        const f32x4_t q = *reinterpret_cast<const f32x4_t*>(stage + r * RSW + (lc + e) * 4);
#pragma unroll
                        for (int k = 0; k < 4; ++k) v[e + k] = q[k];
                    }
                    float sum = 0.f;
#pragma unroll
                    for (int e = 0; e < CPL; ++e) sum += v[e];
                    const float mean = group_sum<16>(sum) / (float)BN;
                    float sq = 0.f;
#pragma unroll
                    for (int e = 0; e < CPL; ++e) {
                        const float d = v[e] - mean;
                        sq += d * d;
                    }
                    const float rstd = 1.0f / sqrtf(group_sum<16>(sq) / (float)BN + (EPI == 5 ? osc.norm_eps : ln.eps));
                    float y[CPL];
#pragma unroll
                    for (int e = 0; e < CPL; ++e) y[e] = (v[e] - mean) * rstd * gw[e] + gb[e];
                    if constexpr (EPI == 5) {
#pragma unroll
                        for (int e = 0; e < CPL; ++e) y[e] = y[e] * __builtin_amdgcn_rcpf(1.0f + __expf(-y[e]));
                    }
                    const int64_t i = row_at(32 * rb + 16 * h + r);
                    // the stored row: i, or (EPI 5) the child of octant oct of parent i, or none
                    int64_t drow = i;
                    if constexpr (EPI == 5) {
                        drow = -1;
                        if (i >= 0) {
                            constexpr uint64_t kLow7 = 0x7f7f7f7f7f7f7f7full;
                            const uint64_t mw = *reinterpret_cast<const uint64_t*>(osc.mask + 8 * i);
                            const uint64_t kept = (((mw & kLow7) + kLow7) | mw) & ~kLow7;
                            if ((kept >> (8 * oct + 7)) & 1)
                                drow = osc.mstart[i] + __popcll(kept & ((1ull << (8 * oct)) - 1));
                        }
                    }
                    if (row0_bad && i >= 0) {
                        bool absent = false;
                        for (int t = 0; t < kTaps; ++t) absent |= nbr[(int64_t)t * n + i] == (int32_t)n;
                        if (absent) {
#pragma unroll
                            for (int e = 0; e < CPL; ++e) y[e] = NAN;
                        }
                    }
                    if (drow >= 0) {
                        uint32_t wd[CPL / 2];
#pragma unroll
                        for (int e = 0; e < CPL / 2; ++e)
                            wd[e] = (ODT == TSP_BF16) ? f32x2_to_bf16x2_bits(y[2 * e], y[2 * e + 1])
                                                      : f32_to_f16_bits(y[2 * e]) |
                                                            ((uint32_t)f32_to_f16_bits(y[2 * e + 1]) << 16);
                        uint16_t* dst = reinterpret_cast<uint16_t*>(out) + drow * (EPI == 5 ? osc.cout : co) + lc;
                        if constexpr (CPL == 8)
                            *reinterpret_cast<u32x4_t*>(dst) = u32x4_t{wd[0], wd[1], wd[2], wd[3]};
                        else
                            *reinterpret_cast<uint2*>(dst) = uint2{wd[0], wd[1]};
                    }
                }
                __syncthreads();                 // the next round overwrites the staging
            }
        }
    };
    auto finish = [&](auto nr_c, f32x16_t (&acc)[RB][CB], int64_t tile) {
        if constexpr (EPI == 3 || EPI == 5) epilogue_ln(acc, tile);
        else epilogue(nr_c, acc, tile);
    };

    // Vector-memory loads return in issue order, so waiting for a weight load also waits for
    // every slice piece issued before it: the weights run PD taps ahead and the slice pieces go
    // out every SP-th tap, which leaves each piece >= PD+1 taps to land. The weight ring has
    // PD+1 slots indexed by tap; PD+1 must divide 2 x 27 so that the ring index continues
    // across slice pairs with compile-time register indices.
    static_assert((2 * kTaps) % (PD + 1) == 0, "weight ring must divide 2 x 27 taps");
    static_assert(PIECES * SP <= kTaps, "slice pieces must fit in one slice's taps");
    static_assert((PIECES - 1) * SP + STG < kTaps, "every staged piece is written within its slice");

    // The tile loop, once with cross-tile pipelining and once without: two loops rather than a
    // branch per tile, so that the weight ring carried from one tile to the next is live only in
    // the loop that carries it (across a per-tile branch the register allocator spilled it at
    // every tile).
    auto tile_loop = [&](auto pipe_c) {
    constexpr bool PIPE = decltype(pipe_c)::value;
    // prologue state: the current tile's plan is in sL, its first slice in sH0 and the weights
    // of its first PD taps in the ring (set by the previous tile's last slice when pipelined)
    bool pre = false;
    int H = 0;
    bool direct = false;
    u32x4_t bR[PD + 1][CB];

    for (int64_t lin = lin0; lin < xhi; lin += stride) {
        asm volatile("" : "+v"(lane), "+v"(r32), "+v"(g), "+v"(rg), "+v"(plane));
#pragma unroll
        for (int cb = 0; cb < CB; ++cb) asm volatile("" : "+v"(boff[cb]));
        const int64_t tile = lin / n_ctiles;
        const int64_t row0 = tile * HB_M;
        if (!pre) {
            // ---- tile plan: slot table in LDS, rows of this thread's slice pieces in registers
            int32_t prow[PIECES];
            if constexpr (PLANNED) {
                // Header, slot table and piece rows are independent loads (every tile has a
                // full-size slot table and row list in the plan), issued together so the
                // prologue pays one memory round trip for them instead of two.
                const int32_t* hdr = plan.hdr + tile * 4;
                const int32_t h0 = hdr[0], h1 = hdr[1];
                const char* src = reinterpret_cast<const char*>(plan.slots + tile * HB_SLOT_TABLE);
                for (int p = wave; p < HB_SLOT_TABLE * 2 / 1024; p += WAVES)   // 27 x 1 KiB
                    __builtin_amdgcn_global_load_lds(
                        src + p * 1024 + lane * 16,
                        (__attribute__((address_space(3))) void*)(reinterpret_cast<char*>(&sL[0][0][0][0]) + p * 1024),
                        16, 0, 0);
                const int32_t* ro = plan.rowof + tile * HB_SLOTS;
#pragma unroll
                for (int j = 0; j < PIECES; ++j) prow[j] = ro[piece_slot(j) + (lane >> 1)];
                H = h0;
                direct = h1 != 0;
                load_act(tile, ab);
                ob = load_ob(tile);
            } else {
                tile_plan<NT>(nbr, n, row0, sL, reinterpret_cast<int32_t*>(&sH0[0][0][0]),
                              reinterpret_cast<uint32_t*>(&sH1[0][0][0]), sRed, H, direct);
                const int32_t* sRowOf = reinterpret_cast<const int32_t*>(&sH0[0][0][0]);
#pragma unroll
                for (int j = 0; j < PIECES; ++j) prow[j] = direct ? 0 : sRowOf[(piece_slot(j) + (lane >> 1)) % HB_SLOTS];
                __syncthreads();     // sH0 is overwritten by the first slice below
            }
            if (!direct) {
                set_poff(prow, H);
                zero_slot(sH0);
                zero_slot(sH1);
#pragma unroll
                for (int j = 0; j < PIECES; ++j) {
                    u32x4_t r;
                    fetch_piece(0, j, r);
                    put_piece(sH0, j, r);
                }
#pragma unroll
                for (int q = 0; q < PD; ++q) load_b(q, 0, bR[q]);
                wait_vmcnt0();
                __syncthreads();
            }
        }
        if (!direct) {
            // Slice pieces go through registers: a 16-byte global load per lane at tap t, its
            // LDS write at tap t + STG. (A direct-to-LDS DMA would be hidden from the compiler's
            // wait counting -- it then waits for each DMA right after issuing it, because it
            // cannot tell the DMA's LDS store from the reads that follow -- while plain loads are
            // counted exactly and the slice boundary need not wait for the weight loads still in
            // flight.) The zero slot lies past the loaded slots and is never overwritten.
            u32x4_t stg[NSTG];

            // one slice: all 27 taps on `cur` while slice kcn streams into `nxt`
            // R0: the weight ring's slot of this slice's tap 0 (slices go in pairs, so a ring
            // size that divides 2 x 27 keeps every register index static). With LAST, the piece
            // ring, once idle, loads the next tile's slot table (this wave's 1 KiB blocks).
            auto run_slice = [&](f32x16_t (&acc)[RB][CB], auto ring0, auto last_c,
                                 const uint16_t (*cur)[HB_ROWS][8], uint16_t (*nxt)[HB_ROWS][8], int kc,
                                 int kcn, const uint16_t* nslots) {
                constexpr int R0 = decltype(ring0)::value;
                constexpr bool LAST = decltype(last_c)::value;
                u32x4_t aC[RB], aN[RB];
                load_a(cur, 0, aC);
                // all 27 taps unrolled: register rings stay static and every wait is exact
#pragma unroll
                for (int t = 0; t < kTaps; ++t) {
                    // The higher issue priority on alternate taps, so that waves at different
                    // taps of the slice are not served alike: at 128 output channels even and
                    // odd waves alternate it (neighbouring SIMDs in turn), at 64 every wave takes
                    // it on the odd taps. Against equal priorities, 3.5 % faster at 128 and the
                    // same at 64. (At 128 the wave-uniform branch also keeps the scheduler from
                    // interleaving taps: the every-wave-alike form there doubles the spills and
                    // runs 2.3 % slower; at 64, with no spills, it is 1 % faster.)
                    if ((BN == 128 ? t + wave_s : t) & 1) __builtin_amdgcn_s_setprio(1);
                    else __builtin_amdgcn_s_setprio(0);
                    // weights PD taps ahead (the first taps of the next slice at the end)
                    if (t + PD < kTaps) load_b(t + PD, kc, bR[(R0 + t + PD) % (PD + 1)]);
                    else load_b(t + PD - kTaps, kcn, bR[(R0 + t + PD) % (PD + 1)]);
                    if (t % SP == 0 && t / SP < PIECES) fetch_piece(kcn, t / SP, stg[(t / SP) % NSTG]);
                    if (t >= STG && (t - STG) % SP == 0 && (t - STG) / SP < PIECES)
                        put_piece(nxt, (t - STG) / SP, stg[((t - STG) / SP) % NSTG]);
                    if constexpr (LAST) {
                        if (t == T_FREE) {
                            // blocks wave + WAVES k of the next tile's slot table (the last
                            // block again where this wave has fewer)
#pragma unroll
                            for (int k = 0; k < SLOT_BLOCKS; ++k) {
                                const int p = min(wave + WAVES * k, HB_SLOT_TABLE * 2 / 1024 - 1);
                                stg[k] = *reinterpret_cast<const u32x4_t*>(
                                    reinterpret_cast<const char*>(nslots) + p * 1024 + lane * 16);
                            }
                        }
                    }
                    // This tap's MFMAs, block by block (a block whose act bit is clear is
                    // skipped), with the next tap's A reads placed between them: each skip test
                    // ends a basic block, so the interleaving is written out here rather than
                    // left to the scheduler, and the reads' latency stays behind MFMAs.
                    const uint32_t on = tap_bits(t);
                    auto mfma_block = [&](int rb) {
                        if (__builtin_expect((on >> rb) & 1u, 1)) {
#pragma unroll
                            for (int cb = 0; cb < CB; ++cb)
                                acc[rb][cb] = mfma32x32x16<BF16>(aC[rb], bR[(R0 + t) % (PD + 1)][cb], acc[rb][cb]);
                        }
                    };
                    mfma_block(0);
                    uint2 sl{};
                    if (t + 1 < kTaps) sl = *reinterpret_cast<const uint2*>(&sL[t + 1][rg][r32][0]);
                    mfma_block(1);
                    if (t + 1 < kTaps) {
                        aN[0] = *reinterpret_cast<const u32x4_t*>(&cur[g][sl.x & 0xffffu][0]);
                        aN[1] = *reinterpret_cast<const u32x4_t*>(&cur[g][sl.x >> 16][0]);
                    }
                    mfma_block(2);
                    if (t + 1 < kTaps) {
                        aN[2] = *reinterpret_cast<const u32x4_t*>(&cur[g][sl.y & 0xffffu][0]);
                        aN[3] = *reinterpret_cast<const u32x4_t*>(&cur[g][sl.y >> 16][0]);
                    }
                    mfma_block(3);
#pragma unroll
                    for (int rb = 0; rb < RB; ++rb) aC[rb] = aN[rb];
                    // keep each tap's loads in its tap: unconstrained, the scheduler gathers the
                    // slice loads at the end of the slice, where their latency is fully exposed
                    __builtin_amdgcn_sched_barrier(0);
                }
                // The accumulators are final here: without this use, the compiler may sink a
                // slice's MFMA chains past the barrier toward the epilogue that reads them,
                // keeping every tap's A operands alive (and spilled) until then. (An input
                // operand only: redefining the registers here would hide from the hazard
                // recognizer that the epilogue's reads follow MFMA writes.)
#pragma unroll
                for (int rb = 0; rb < RB; ++rb)
#pragma unroll
                    for (int cb = 0; cb < CB; ++cb) asm volatile("" ::"v"(acc[rb][cb]));
                __syncthreads();
            };
            using I0 = std::integral_constant<int, 0>;
            using I1 = std::integral_constant<int, kTaps % (PD + 1)>;
            using NO = std::false_type;
            if constexpr (PIPE) {
                f32x16_t acc[RB][CB];
                zero(acc);
                for (int kc = 0; kc + 2 < nkc; kc += 2) {
                    run_slice(acc, I0{}, NO{}, sH0, sH1, kc, kc + 1, nullptr);
                    run_slice(acc, I1{}, NO{}, sH1, sH0, kc + 1, kc + 2, nullptr);
                }
                // the next tile of this workgroup (this one again after the last: its loads are
                // then only unused copies)
                const int64_t nlin = lin + stride < xhi ? lin + stride : lin;
                const int64_t ntile = nlin / n_ctiles;
                const int32_t* nhdr = plan.hdr + ntile * 4;
                const int32_t nH = nhdr[0], ndirect = nhdr[1];
                int32_t nrow[PIECES];
                const int32_t* nro = plan.rowof + ntile * HB_SLOTS;
#pragma unroll
                for (int j = 0; j < PIECES; ++j) nrow[j] = nro[piece_slot(j) + (lane >> 1)];
                uint32_t nab[HB_ACT_WORDS];
                load_act(ntile, nab);
                const uint32_t nob = load_ob(ntile);
                run_slice(acc, I0{}, NO{}, sH0, sH1, nkc - 2, nkc - 1, nullptr);
                // the last slice streams the next tile's slice 0 (rows clamped to 0 where the
                // plan holds none, e.g. a direct tile) and the first taps of its weights
                set_poff(nrow, ndirect ? 0 : nH);
                run_slice(acc, I1{}, std::true_type{}, sH1, sH0, nkc - 1, 0, plan.slots + ntile * HB_SLOT_TABLE);
                // every wave is past its last read of sL and sH1
#pragma unroll
                for (int k = 0; k < SLOT_BLOCKS; ++k) {
                    const int p = wave + WAVES * k;
                    if (p < HB_SLOT_TABLE * 2 / 1024)
                        *reinterpret_cast<u32x4_t*>(reinterpret_cast<char*>(&sL[0][0][0][0]) + p * 1024 + lane * 16) = stg[k];
                }
                finish(std::integral_constant<int, 16>{}, acc, tile);
                __syncthreads();       // the next tile's slot table; every wave's staging is done
                zero_slot(sH1);        // the staging covered it; first read after the next barrier
                pre = nlin != lin && !ndirect;
                H = nH;
                direct = ndirect != 0;
#pragma unroll
                for (int k = 0; k < HB_ACT_WORDS; ++k) ab[k] = nab[k];
                ob = nob;
            } else {
                f32x16_t acc[RB][CB];
                zero(acc);
                // the last slice re-loads itself into the idle buffer, so there is no branch
                for (int kc = 0; kc < nkc; kc += 2) {
                    const int k1 = kc + 1 < nkc ? kc + 1 : kc;
                    run_slice(acc, I0{}, NO{}, sH0, sH1, kc, k1, nullptr);
                    if (kc + 1 < nkc)
                        run_slice(acc, I1{}, NO{}, sH1, sH0, kc + 1, kc + 2 < nkc ? kc + 2 : kc + 1, nullptr);
                }
                finish(std::integral_constant<int, 32>{}, acc, tile);
                __syncthreads();       // staging reads end before the next tile's loads
                pre = false;
            }
        } else {
            // the weight ring is dead here (the next tile's prologue reloads it)
#pragma unroll
            for (int q = 0; q <= PD; ++q)
#pragma unroll
                for (int cb = 0; cb < CB; ++cb) asm volatile("" : "=v"(bR[q][cb]));
            f32x16_t acc[RB][CB];
            zero(acc);
            // ---- direct path: A gathered from global memory
            for (int kc = 0; kc < nkc; ++kc)
                for (int t = 0; t < kTaps; ++t) {
                    u32x4_t bq[CB];
                    load_b(t, kc, bq);
                    u32x4_t a[RB];
#pragma unroll
                    for (int rb = 0; rb < RB; ++rb) {
                        const int p = 32 * RB * rg + 32 * rb + r32;   // tile position
                        int64_t i = row0 + p;
                        if constexpr (PLANNED) i = plan.vox[tile * HB_M + p];
                        const int32_t v = (i >= 0 && i < n) ? nbr[(int64_t)t * n + i] : (int32_t)n;
                        a[rb] = u32x4_t{0, 0, 0, 0};
                        if ((uint32_t)v < (uint32_t)n)
                            a[rb] = *reinterpret_cast<const u32x4_t*>(feats + (int64_t)v * ci +
                                                                      kc * HB_KC + g * 8);
                    }
#pragma unroll
                    for (int rb = 0; rb < RB; ++rb)
#pragma unroll
                        for (int cb = 0; cb < CB; ++cb)
                            acc[rb][cb] = mfma32x32x16<BF16>(a[rb], bq[cb], acc[rb][cb]);
                }
            finish(std::integral_constant<int, 32>{}, acc, tile);
            __syncthreads();           // staging reads end before the next tile's loads
            pre = false;
        }
    }
    };
    if constexpr (CAN_PIPE) {
        if (nkc % 2 == 0) {
            tile_loop(std::true_type{});
            return;
        }
    }
    tile_loop(std::false_type{});
}

// Compute units of the current device (cached per device).
int cu_count() {
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

template <bool BF16, int BN, int ODT, bool PLANNED>
int launch(const void* feats, int64_t n, int ci, const int32_t* nbr, const void* plan,
           const void* weight, const float* bias, int co, void* out, hipStream_t s, OctantScatter osc,
           SkipAdd skip, PadRow pad, RowNorm ln, TileRange tr) {
    const int64_t all_tiles = ceil_div(n, HB_M);
    // a stored plan's tiles [t0, t0 + n_tiles): its per-tile arrays (and the octant block words)
    // start at tile t0, and the kernel's tile indices count from there
    const int64_t t0 = PLANNED ? tr.t0 : 0;
    const int64_t n_tiles = PLANNED && tr.nt >= 0 ? tr.nt : all_tiles - t0;
    if (t0 < 0 || n_tiles < 0 || t0 + n_tiles > all_tiles) {
        set_error("MFMA conv: tiles [%lld, %lld) outside the plan's %lld", (long long)t0,
                  (long long)(t0 + n_tiles), (long long)all_tiles);
        return TSP_ERR_INVALID;
    }
    if (n_tiles == 0) return TSP_OK;
    const int n_ctiles = co / BN;
    const int64_t total = n_tiles * n_ctiles;
    const int64_t per_xcd = ceil_div(total, 8);
    PlanView pv{};
    if (plan) {
        pv = carve_plan(const_cast<void*>(plan), all_tiles);
        pv.hdr += t0 * 4;
        pv.rowof += t0 * HB_SLOTS;
        pv.slots += t0 * HB_SLOT_TABLE;
        pv.vox += t0 * HB_M;
        pv.act += t0 * 4 * HB_ACT_WORDS;
    }
    if (osc.blocks) osc.blocks += t0 * 4;
    // 8 waves of 128 voxels x BN/2 channels; weights 2 taps ahead (5 at BN = 64, whose waves
    // have the registers for it: 3 % faster there, while at BN = 128 the deeper ring spills);
    // a slice piece every other tap, written to LDS 6 taps after its load
    constexpr int RB = 4, CB = BN / 64, PD = BN == 128 ? 2 : 5, SP = 2, STG = 6;
    // With a plan: one workgroup per CU (the LDS of one fills a CU), a multiple of n_ctiles per
    // XCD. Without: one per (tile, column tile), each building its own plan.
    int64_t per_xcd_wg = per_xcd;
    if (PLANNED) {
        const int64_t fit = std::max<int64_t>(1, cu_count() / 8 / n_ctiles) * n_ctiles;
        per_xcd_wg = std::min(per_xcd, fit);
    }
    const dim3 grid((unsigned)(per_xcd_wg * 8)), block(hb_waves<BN, RB, CB>() * 64);
    const uint16_t* f16 = reinterpret_cast<const uint16_t*>(feats);
    const uint16_t* w16 = reinterpret_cast<const uint16_t*>(weight);
    if constexpr (PLANNED && ODT == TSP_F32) {
        if (osc.cout) {
            hipLaunchKernelGGL((k_conv_halo_octants<BF16, BN, RB, CB, PD, SP, STG>), grid, block, 0, s,
                               f16, n, ci, nbr, pv, w16, bias, co, out, n_tiles, n_ctiles, per_xcd, osc, pad);
            TSP_CHECK_LAUNCH();
            return TSP_OK;
        }
        if (skip.cin) {
            hipLaunchKernelGGL((k_conv_halo_skip<BF16, BN, RB, CB, PD, SP, STG>), grid, block, 0, s,
                               f16, n, ci, nbr, pv, w16, bias, co, out, n_tiles, n_ctiles, per_xcd, skip, pad);
            TSP_CHECK_LAUNCH();
            return TSP_OK;
        }
    }
    if constexpr (PLANNED && ODT == (BF16 ? TSP_BF16 : TSP_F16)) {
        if constexpr (CB == 2) {
            if (osc.cout && osc.norm_silu && osc.cout == 32 * CB) {
                hipLaunchKernelGGL((k_conv_halo_octants_norm<BF16, BN, RB, CB, PD, SP, STG>), grid, block, 0, s,
                                   f16, n, ci, nbr, pv, w16, bias, co, out, n_tiles, n_ctiles, per_xcd, osc, pad);
                TSP_CHECK_LAUNCH();
                return TSP_OK;
            }
            if (osc.cout && osc.norm_silu && osc.cout == BN) {
                hipLaunchKernelGGL((k_conv_halo_octants_rownorm<BF16, BN, RB, CB, PD, SP, STG>), grid, block, 0, s,
                                   f16, n, ci, nbr, pv, w16, bias, co, out, n_tiles, n_ctiles, per_xcd, osc, pad);
                TSP_CHECK_LAUNCH();
                return TSP_OK;
            }
        }
        if (ln.w) {
            hipLaunchKernelGGL((k_conv_halo_ln<BF16, BN, RB, CB, PD, SP, STG>), grid, block, 0, s,
                               f16, n, ci, nbr, pv, w16, bias, co, out, n_tiles, n_ctiles, per_xcd, pad, ln);
            TSP_CHECK_LAUNCH();
            return TSP_OK;
        }
    }
    if (osc.cout || skip.cin || ln.w) {
        set_error("MFMA conv: octant stores and the skip add write f32 from a stored plan, a row norm "
                  "the feature type");
        return TSP_ERR_UNSUPPORTED;
    }
    hipLaunchKernelGGL((k_conv_halo<BF16, BN, ODT, PLANNED, RB, CB, PD, SP, STG>), grid, block, 0, s,
                       f16, n, ci, nbr, pv, w16, bias, co, out, n_tiles, n_ctiles, per_xcd, pad);
    TSP_CHECK_LAUNCH();
    return TSP_OK;
}

template <bool BF16, int BN, int ODT>
int launch_planned(bool planned, const void* feats, int64_t n, int ci, const int32_t* nbr,
                   const void* plan, const void* weight, const float* bias, int co, void* out,
                   hipStream_t s, OctantScatter osc, SkipAdd skip, PadRow pad, RowNorm ln, TileRange tr) {
    if (planned)
        return launch<BF16, BN, ODT, true>(feats, n, ci, nbr, plan, weight, bias, co, out, s, osc, skip, pad, ln, tr);
    return launch<BF16, BN, ODT, false>(feats, n, ci, nbr, nullptr, weight, bias, co, out, s, osc, skip, pad, ln,
                                        TileRange{});
}

template <bool BF16, int BN>
int launch_out(int odt, bool planned, const void* feats, int64_t n, int ci, const int32_t* nbr,
               const void* plan, const void* weight, const float* bias, int co, void* out,
               hipStream_t s, OctantScatter osc, SkipAdd skip, PadRow pad, RowNorm ln, TileRange tr) {
    if (odt == TSP_F32)
        return launch_planned<BF16, BN, TSP_F32>(planned, feats, n, ci, nbr, plan, weight, bias, co, out, s, osc, skip,
                                                 pad, ln, tr);
    if (BF16 && odt == TSP_BF16)
        return launch_planned<BF16, BN, TSP_BF16>(planned, feats, n, ci, nbr, plan, weight, bias, co, out, s, osc,
                                                  skip, pad, ln, tr);
    if (!BF16 && odt == TSP_F16)
        return launch_planned<BF16, BN, TSP_F16>(planned, feats, n, ci, nbr, plan, weight, bias, co, out, s, osc, skip,
                                                 pad, ln, tr);
    set_error("MFMA conv writes f32 or the feature dtype, not %d", odt);
    return TSP_ERR_UNSUPPORTED;
}

}  // namespace

// One instantiation family each (conv_halo_bf16_128.hip, ...): the planned or unplanned conv with
// output dtype odt, octant or skip stores when given.
#define TSP_HALO_LAUNCH_ARGS int odt, bool planned, const void* feats, int64_t n, int ci, const int32_t* nbr, \
    const void* plan, const void* weight, const float* bias, int co, void* out, hipStream_t s, OctantScatter osc, \
    SkipAdd skip, PadRow pad, RowNorm ln, TileRange tr
int halo_launch_bf16_128(TSP_HALO_LAUNCH_ARGS);
int halo_launch_bf16_64(TSP_HALO_LAUNCH_ARGS);
int halo_launch_f16_128(TSP_HALO_LAUNCH_ARGS);
int halo_launch_f16_64(TSP_HALO_LAUNCH_ARGS);

}  // namespace tsp
