// MFMA submanifold conv with each tile's neighbour rows staged in LDS.
//
// A workgroup owns HB_M = 512 consecutive output voxels x BN output channels and runs 8 waves,
// two per SIMD: wave w owns voxels [128 (w%4), +128) x channels [(w/4) BN/2, +BN/2) (the
// kernel is written for any split of RB 32-row x CB 32-column MFMA blocks per wave). On
// sorted surface sets those 512 voxels reference only ~1700 distinct input rows (against
// ~9600 (voxel, tap) pairs), so instead of gathering every pair from L2 the tile gathers each
// distinct row once:
//   * tile plan: mark every referenced row in a two-level bitmap over [lo, hi] (the range of
//     the tile's table entries), exclusive-scan the popcounts, and give each (tap, voxel) its
//     rank in the set -- its slot. Slots are sorted by row, so consecutive voxels at one tap
//     mostly get consecutive slots. Absent taps get the zero slot. The plan depends only on
//     the neighbour table, so it is built once and reused by every conv on that table (the
//     reference shares one table across a decoder stage, shape_decoder.cpp:93-103); without a
//     stored plan the kernel builds it in LDS itself.
//   * the distinct rows stream through LDS 16 channels at a time (two buffers, each a separate
//     LDS object), the next slice loading while the current one runs all 27 taps: each lane
//     loads its 16-byte pieces into registers and writes them to LDS a few taps later. Each
//     buffer holds the two 8-channel halves of a row in separate planes, so the 32 lanes that
//     feed one MFMA operand read 32 consecutive 16-byte words when the slots are consecutive;
//     absent taps read a zero slot kept past the loaded ones.
//   * per tap, A operands are read from LDS by slot and B operands (weights) come from L2 two
//     taps ahead. Packed weights ([co/32][ci/16][27][64 lanes][8]) make every weight load one
//     contiguous 1 KiB per wave. All 27 taps are unrolled and slices go in pairs, so every
//     register ring index is static and the compiler's load waits are exact.
//   * the epilogue stages 32-row blocks of the accumulators in LDS and writes whole rows.
// A tile whose row range or distinct-row count does not fit (scattered or unsorted inputs)
// takes the direct path: the same MFMA loop with A gathered straight from global memory.
#include <algorithm>
#include <type_traits>

#include "conv_internal.hpp"

namespace tsp {
namespace {

constexpr int HB_PLAN_NT = 256;            // threads of a plan-build workgroup
constexpr int HB_KC = 16;                  // channels per LDS slice
constexpr int HB_SLOTS = 2048;             // slots per slice buffer
constexpr int HB_ZERO = HB_SLOTS;          // slot that always holds zeros (absent taps)
constexpr int HB_ROWS = HB_SLOTS + 1;      // rows of a slice buffer plane: the slots + zero
constexpr int HB_SLOT_TABLE = kTaps * HB_M;                    // uint16 slots per tile
constexpr int HB_PLAN_SCRATCH = 5 * HB_SLOTS;                  // tile_plan scratch words
constexpr int64_t HB_MAXSPAN = (int64_t)HB_SLOTS * 32 * 32;    // 2^21 rows

__device__ __forceinline__ void wait_vmcnt0() { __builtin_amdgcn_s_waitcnt(0x0070 | 0x0f00); }

__device__ __forceinline__ int wave_min(int v) {
    for (int off = 32; off > 0; off >>= 1) v = min(v, __shfl_xor(v, off, 64));
    return v;
}
__device__ __forceinline__ int wave_max(int v) {
    for (int off = 32; off > 0; off >>= 1) v = max(v, __shfl_xor(v, off, 64));
    return v;
}

// Plan layout: [n_tiles][4] int32 header {H, direct, 0, 0} | [n_tiles][HB_SLOTS] int32 row of each
// slot | [n_tiles][27][4][32][4] uint16 slot of each (tap, voxel/128, voxel%32, voxel/32%4).
struct PlanView {
    int32_t* hdr;
    int32_t* rowof;
    uint16_t* slots;
};
inline size_t align256(size_t b) { return (b + 255) & ~size_t(255); }
__host__ __device__ inline PlanView carve_plan(void* p, int64_t n_tiles) {
    char* c = reinterpret_cast<char*>(p);
    PlanView v;
    v.hdr = reinterpret_cast<int32_t*>(c);
    c += align256((size_t)n_tiles * 16);
    v.rowof = reinterpret_cast<int32_t*>(c);
    c += align256((size_t)n_tiles * HB_SLOTS * 4);
    v.slots = reinterpret_cast<uint16_t*>(c);
    return v;
}

// ---- tile plan (all NT threads of the block) -----------------------------------------------
// Exclusive scan of the popcounts of words[0..nwords) (nwords <= HB_SLOTS) into pre[];
// returns the total. sRed: NT/64 ints of scratch.
template <int NT>
__device__ int scan_popcounts(const uint32_t* words, int nwords, int32_t* pre, int* sRed) {
    constexpr int WPT = HB_SLOTS / NT;
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    int cnt[WPT];
    int mine = 0;
#pragma unroll
    for (int k = 0; k < WPT; ++k) {
        const int w = tid * WPT + k;
        cnt[k] = (w < nwords) ? __popc(words[w]) : 0;
        mine += cnt[k];
    }
    int x = mine;
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
        const int y = __shfl_up(x, off, 64);
        if (lane >= off) x += y;
    }
    if (lane == 63) sRed[wave] = x;
    __syncthreads();
    int base = 0, total = 0;
#pragma unroll
    for (int w = 0; w < NT / 64; ++w) {
        if (w < wave) base += sRed[w];
        total += sRed[w];
    }
    base += x - mine;
#pragma unroll
    for (int k = 0; k < WPT; ++k) {
        pre[tid * WPT + k] = base;
        base += cnt[k];
    }
    __syncthreads();
    return total;
}

// Fills sL with the slot of every (tap, voxel) of tile row0 and sRowOf with the row of every
// slot; returns H (number of distinct rows) and whether the tile must take the direct path.
// The set of referenced rows is ranked with a two-level bitmap over [lo, hi]: a coarse bit per
// 32-row block (spans up to 2^21 rows), then one fine word per non-empty block; slot = fine
// prefix of the block + rank inside the block's word.
// scratch: HB_PLAN_SCRATCH words; sRed: 2 * NT/64 ints.
template <int NT>
__device__ void tile_plan(const int32_t* __restrict__ nbr, int64_t n, int64_t row0,
                          uint16_t (*sL)[4][32][4], int32_t* sRowOf, uint32_t* scratch,
                          int* sRed, int& H_out, bool& direct_out) {
    constexpr int VPT = HB_M / NT;         // voxels per thread
    constexpr int WPT = HB_SLOTS / NT;     // bitmap words per thread
    constexpr int NW = NT / 64;
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    uint32_t* coarse = scratch;                                       // bit per 32-row block
    int32_t* cpre = reinterpret_cast<int32_t*>(scratch + HB_SLOTS);   // block rank of a word
    uint32_t* fine = scratch + 2 * HB_SLOTS;                          // rows of each block
    int32_t* fpre = reinterpret_cast<int32_t*>(scratch + 3 * HB_SLOTS);
    int32_t* block_of = reinterpret_cast<int32_t*>(scratch + 4 * HB_SLOTS);   // rank -> block
    // this thread's table entries (voxels tid + NT h, all taps), loaded once and without
    // branches so all loads are in flight together; absent taps / voxels past n -> -1
    int32_t nv[kTaps][VPT];
    {
        int64_t ic[VPT];
        bool in[VPT];
#pragma unroll
        for (int h = 0; h < VPT; ++h) {
            const int64_t i = row0 + tid + NT * h;
            in[h] = i < n;
            ic[h] = in[h] ? i : n - 1;
        }
#pragma unroll
        for (int t = 0; t < kTaps; ++t)
#pragma unroll
            for (int h = 0; h < VPT; ++h) nv[t][h] = nbr[(int64_t)t * n + ic[h]];
#pragma unroll
        for (int t = 0; t < kTaps; ++t)
#pragma unroll
            for (int h = 0; h < VPT; ++h)
                nv[t][h] = (in[h] && (uint32_t)nv[t][h] < (uint32_t)n) ? nv[t][h] : -1;
    }
    int lo = INT32_MAX, hi = -1;
#pragma unroll
    for (int t = 0; t < kTaps; ++t)
#pragma unroll
        for (int h = 0; h < VPT; ++h)
            if (nv[t][h] >= 0) { lo = min(lo, nv[t][h]); hi = max(hi, nv[t][h]); }
    lo = wave_min(lo);
    hi = wave_max(hi);
    if (lane == 0) { sRed[wave] = lo; sRed[NW + wave] = hi; }
    __syncthreads();
    lo = INT32_MAX;
    hi = -1;
#pragma unroll
    for (int w = 0; w < NW; ++w) { lo = min(lo, sRed[w]); hi = max(hi, sRed[NW + w]); }
    __syncthreads();
    bool direct = hi >= 0 && (int64_t)hi - lo + 1 > HB_MAXSPAN;
    int H = 0, nblocks = 0;

    if (!direct && hi >= 0) {
#pragma unroll
        for (int k = 0; k < WPT; ++k) {
            coarse[tid * WPT + k] = 0u;
            fine[tid * WPT + k] = 0u;
        }
        __syncthreads();
        // level 1: which 32-row blocks are referenced
#pragma unroll
        for (int t = 0; t < kTaps; ++t)
#pragma unroll
            for (int h = 0; h < VPT; ++h) {
                const int32_t v = nv[t][h];
                if (v >= 0) {
                    const int d = v - lo;
                    atomicOr(&coarse[d >> 10], 1u << ((d >> 5) & 31));
                }
            }
        __syncthreads();
        nblocks = scan_popcounts<NT>(coarse, HB_SLOTS, cpre, sRed);
        direct = nblocks > HB_ZERO;        // every block holds a row: too many rows for LDS
        if (!direct) {
            // level 2: rows within each referenced block
#pragma unroll
            for (int t = 0; t < kTaps; ++t)
#pragma unroll
                for (int h = 0; h < VPT; ++h) {
                    const int32_t v = nv[t][h];
                    if (v >= 0) {
                        const int d = v - lo, cw = d >> 10, cb = (d >> 5) & 31;
                        const int blk = cpre[cw] + __popc(coarse[cw] & ((1u << cb) - 1u));
                        atomicOr(&fine[blk], 1u << (d & 31));
                    }
                }
            // rank -> block id
#pragma unroll
            for (int k = 0; k < WPT; ++k) {
                const int w = tid * WPT + k;
                uint32_t bits = coarse[w];
                int r = cpre[w];
                while (bits) {
                    const int bit = __builtin_ctz(bits);
                    bits &= bits - 1u;
                    block_of[r++] = w * 32 + bit;
                }
            }
            __syncthreads();
            H = scan_popcounts<NT>(fine, nblocks, fpre, sRed);
            direct = H > HB_ZERO;
        }
    }
    if (!direct) {
        // slot of every (tap, voxel)
#pragma unroll
        for (int t = 0; t < kTaps; ++t)
#pragma unroll
            for (int h = 0; h < VPT; ++h) {
                const int rr = tid + NT * h;                   // voxel within the tile
                const int32_t v = nv[t][h];
                int slot = HB_ZERO;
                if (v >= 0) {
                    const int d = v - lo, cw = d >> 10, cb = (d >> 5) & 31;
                    const int blk = cpre[cw] + __popc(coarse[cw] & ((1u << cb) - 1u));
                    slot = fpre[blk] + __popc(fine[blk] & ((1u << (d & 31)) - 1u));
                }
                sL[t][rr >> 7][rr & 31][(rr >> 5) & 3] = (uint16_t)slot;
            }
        // row of every slot
#pragma unroll
        for (int k = 0; k < WPT; ++k) {
            const int w = tid * WPT + k;
            if (w < nblocks) {
                uint32_t bits = fine[w];
                int s = fpre[w];
                const int base = lo + block_of[w] * 32;
                while (bits) {
                    const int bit = __builtin_ctz(bits);
                    bits &= bits - 1u;
                    sRowOf[s++] = base + bit;
                }
            }
        }
    }
    __syncthreads();
    H_out = H;
    direct_out = direct;
}

__global__ __launch_bounds__(HB_PLAN_NT) void k_plan_build(const int32_t* __restrict__ nbr,
                                                           int64_t n, int64_t n_tiles,
                                                           PlanView plan) {
    __shared__ __attribute__((aligned(16))) uint16_t sL[kTaps][4][32][4];
    __shared__ int32_t sRowOf[HB_SLOTS];
    __shared__ uint32_t sScratch[HB_PLAN_SCRATCH];
    __shared__ int sRed[2 * HB_PLAN_NT / 64];
    const int64_t tile = blockIdx.x;
    int H;
    bool direct;
    tile_plan<HB_PLAN_NT>(nbr, n, tile * HB_M, sL, sRowOf, sScratch, sRed, H, direct);
    const int tid = threadIdx.x;
    if (tid == 0) {
        int32_t* h = plan.hdr + tile * 4;
        h[0] = H; h[1] = direct ? 1 : 0; h[2] = 0; h[3] = 0;
    }
    if (direct) return;
    int32_t* ro = plan.rowof + tile * HB_SLOTS;
    for (int s = tid; s < H; s += HB_PLAN_NT) ro[s] = sRowOf[s];
    const u32x4_t* src = reinterpret_cast<const u32x4_t*>(&sL[0][0][0][0]);
    u32x4_t* dst = reinterpret_cast<u32x4_t*>(plan.slots + tile * HB_SLOT_TABLE);
    for (int p = tid; p < HB_SLOT_TABLE / 8; p += HB_PLAN_NT) dst[p] = src[p];
}

// packed[((c32 * nkc + kc) * 27 + t) * 64 + lane][0..7] = W[32 c32 + lane%32][t][16 kc + 8 (lane/32) ..]
__global__ void k_weight_pack(const uint16_t* __restrict__ w, int ci, int co,
                              uint16_t* __restrict__ packed) {
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
}

// ---- the conv ---------------------------------------------------------------------------------
// WAVES = 4 (one wave per SIMD, each owning 128 voxels x all BN channels, accumulators in the
// upper register file, weights PD taps ahead) or 8 (two per SIMD, each 128 voxels x BN/2).
template <int BN, int RB, int CB>
constexpr int hb_waves() { return (HB_M / (32 * RB)) * (BN / (32 * CB)); }

template <bool BF16, int BN, int ODT, bool PLANNED, int RB, int CB, int PD, int SP, int STG>
__device__ __forceinline__ void conv_tile(
    const uint16_t* __restrict__ feats, int64_t n, int ci, const int32_t* __restrict__ nbr,
    PlanView plan, const uint16_t* __restrict__ weight, const float* __restrict__ bias, int co,
    void* __restrict__ out, int n_ctiles, int64_t lin, uint16_t (&sH0)[2][HB_ROWS][8],
    uint16_t (&sH1)[2][HB_ROWS][8], uint16_t (&sL)[kTaps][4][32][4], int* sRed);

template <bool BF16, int BN, int ODT, bool PLANNED, int RB, int CB, int PD, int SP, int STG>
__global__ __launch_bounds__((hb_waves<BN, RB, CB>() * 64), 1) void k_conv_halo(
    const uint16_t* __restrict__ feats, int64_t n, int ci, const int32_t* __restrict__ nbr,
    PlanView plan, const uint16_t* __restrict__ weight, const float* __restrict__ bias, int co,
    void* __restrict__ out, int64_t n_tiles, int n_ctiles, int64_t per_xcd) {
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
    const int64_t total = n_tiles * n_ctiles;
    const int xcd = (int)(blockIdx.x % 8);
    const int64_t xlo = xcd * per_xcd, xhi = xlo + per_xcd < total ? xlo + per_xcd : total;
    const int64_t lin = xlo + blockIdx.x / 8;
    if (lin >= xhi) return;
    conv_tile<BF16, BN, ODT, PLANNED, RB, CB, PD, SP, STG>(
        feats, n, ci, nbr, plan, weight, bias, co, out, n_ctiles, lin, sH0, sH1, sL, sRed);
}

// One (tile, column tile) of the conv: the whole tile pipeline, run by all the workgroup's waves.
template <bool BF16, int BN, int ODT, bool PLANNED, int RB, int CB, int PD, int SP, int STG>
__device__ __forceinline__ void conv_tile(
    const uint16_t* __restrict__ feats, int64_t n, int ci, const int32_t* __restrict__ nbr,
    PlanView plan, const uint16_t* __restrict__ weight, const float* __restrict__ bias, int co,
    void* __restrict__ out, int n_ctiles, int64_t lin, uint16_t (&sH0)[2][HB_ROWS][8],
    uint16_t (&sH1)[2][HB_ROWS][8], uint16_t (&sL)[kTaps][4][32][4], int* sRed) {
    constexpr int NRG = HB_M / (32 * RB), NCG = BN / (32 * CB);
    constexpr int WAVES = NRG * NCG;
    constexpr int NT = WAVES * 64;
    constexpr int WN = 32 * CB;              // output channels per wave
    constexpr int PIECES = 2 * HB_SLOTS / 64 / WAVES;   // slice loads per wave and slice
    const int64_t tile = lin / n_ctiles;
    const int64_t row0 = tile * HB_M;

    const int tid = threadIdx.x;
    const int wave = tid >> 6, lane = tid & 63;
    const int r32 = lane & 31, g = lane >> 5;
    const int rg = wave % NRG;               // row group: voxels [32 RB rg, +32 RB)
    const int c0 = (int)(lin % n_ctiles) * BN + (wave / NRG) * WN;   // first channel of wave
    const int nkc = ci / HB_KC;
    // slice DMA: wave w streams plane (w & 1), 64-slot blocks (w >> 1) + (WAVES/2) j
    const int plane = wave & 1;
    auto piece_slot = [&](int j) { return 64 * ((wave >> 1) + (WAVES / 2) * j); };

    // ---- tile plan: slot table in LDS, rows of this thread's slice pieces in registers
    int H;
    bool direct;
    // byte offset (from feats) of the 8 channels this lane copies for each slice piece at
    // slice 0: row * ci * 2 + plane * 16; slots past H copy row 0 into an unused slot
    uint32_t poff[PIECES];
    int32_t prow[PIECES];
    // the bias of this lane's output channels, fetched now so the epilogue does not wait for it
    float bv[CB];
#pragma unroll
    for (int cb = 0; cb < CB; ++cb) bv[cb] = bias[c0 + cb * 32 + r32];
    if constexpr (PLANNED) {
        // Header, slot table and piece rows are independent loads (every tile has a full-size
        // slot table and row list in the plan), issued together so the prologue pays one
        // memory round trip for them instead of two.
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
        for (int j = 0; j < PIECES; ++j) prow[j] = ro[piece_slot(j) + lane];
        H = h0;
        direct = h1 != 0;
        if (!direct) {
#pragma unroll
            for (int j = 0; j < PIECES; ++j)
                if (piece_slot(j) + lane >= H) prow[j] = 0;
#pragma unroll
            for (int j = 0; j < PIECES; ++j) poff[j] = (uint32_t)prow[j] * (uint32_t)ci * 2u + plane * 16u;
        }
    } else {
        tile_plan<NT>(nbr, n, row0, sL, reinterpret_cast<int32_t*>(&sH0[0][0][0]),
                         reinterpret_cast<uint32_t*>(&sH1[0][0][0]), sRed, H, direct);
        if (!direct) {
            const int32_t* sRowOf = reinterpret_cast<const int32_t*>(&sH0[0][0][0]);
#pragma unroll
            for (int j = 0; j < PIECES; ++j) {
                const int slot = piece_slot(j) + lane;
                prow[j] = slot < H ? sRowOf[slot] : 0;
                poff[j] = (uint32_t)prow[j] * (uint32_t)ci * 2u + plane * 16u;
            }
            __syncthreads();     // sH0 is overwritten by the first slice below
        }
    }

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

    // ---- epilogue: each wave stages 32-row blocks of its accumulators (fp32, + bias) in its own
    // 32 RS bytes of the slice buffers, then writes whole row segments, 4 channels per lane. The
    // row stride WN*4+32 bytes puts the two 32-lane halves of a staging write on disjoint banks.
    // (The slice buffers are idle: every wave passed the last barrier of the main loop, or
    // never used them on the direct path.)
    auto epilogue = [&](f32x16_t (&acc)[RB][CB]) {
        constexpr int RS = WN * 4 + 32;
        static_assert((WAVES / 2) * 32 * RS <= (int)sizeof(sH0), "staging must fit a slice buffer");
        char* stage = reinterpret_cast<char*>(wave < WAVES / 2 ? &sH0[0][0][0] : &sH1[0][0][0]) +
                      (wave % (WAVES / 2)) * 32 * RS;
        const bool full = row0 + HB_M <= n;   // no row of the tile is past n (uniform)
#pragma unroll
        for (int rb = 0; rb < RB; ++rb) {
#pragma unroll
            for (int cb = 0; cb < CB; ++cb)
#pragma unroll
                for (int j = 0; j < 16; ++j) {
                    const int r = 8 * (j / 4) + 4 * g + (j % 4);
                    *reinterpret_cast<float*>(stage + r * RS + (cb * 32 + r32) * 4) = acc[rb][cb][j] + bv[cb];
                }
            // 32 rows x WN/4 chunks of 4 channels: all LDS reads first (one wait), then the stores
            f32x4_t vs[WN / 8];
#pragma unroll
            for (int q = 0; q < WN / 8; ++q) {
                const int c = q * 64 + lane;
                vs[q] = *reinterpret_cast<const f32x4_t*>(stage + (c / (WN / 4)) * RS + (c % (WN / 4)) * 16);
            }
#pragma unroll
            for (int q = 0; q < WN / 8; ++q) {
                const int c = q * 64 + lane;
                const int r = c / (WN / 4), cq = c % (WN / 4);
                const f32x4_t v = vs[q];
                const int64_t i = row0 + 32 * RB * rg + 32 * rb + r;
                if (full || i < n) {
                    const int64_t o = i * co + c0 + cq * 4;
                    if constexpr (ODT == TSP_F32) {
                        *reinterpret_cast<f32x4_t*>(reinterpret_cast<float*>(out) + o) = v;
                    } else {
                        uint16_t h[4];
#pragma unroll
                        for (int e = 0; e < 4; ++e)
                            h[e] = (ODT == TSP_BF16) ? f32_to_bf16_bits(v[e]) : f32_to_f16_bits(v[e]);
                        *reinterpret_cast<uint2*>(reinterpret_cast<uint16_t*>(out) + o) =
                            uint2{(uint32_t)h[0] | ((uint32_t)h[1] << 16), (uint32_t)h[2] | ((uint32_t)h[3] << 16)};
                    }
                }
            }
        }
    };

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

    if (!direct) {
        f32x16_t acc[RB][CB];
        zero(acc);
        // Slice pieces go through registers: a 16-byte global load per lane at tap t, its LDS
        // write at tap t + STG. (A direct-to-LDS DMA would be hidden from the compiler's wait
        // counting -- it then waits for each DMA right after issuing it, because it cannot tell
        // the DMA's LDS store from the reads that follow -- while plain loads are counted exactly
        // and the slice boundary need not wait for the weight loads still in flight.) The zero
        // slot lies past the loaded slots and is never overwritten.
        constexpr int NSTG = (STG + SP - 1) / SP + 1;   // pieces in flight
        u32x4_t stg[NSTG];
        auto fetch_piece = [&](int kc, int j, u32x4_t& r) {
            r = *reinterpret_cast<const u32x4_t*>(reinterpret_cast<const char*>(feats) + poff[j] +
                                                  (uint32_t)kc * (HB_KC * 2));
        };
        auto put_piece = [&](uint16_t (*dst)[HB_ROWS][8], int j, const u32x4_t& r) {
            *reinterpret_cast<u32x4_t*>(&dst[plane][piece_slot(j) + lane][0]) = r;
        };
        // A operands of tap t: per 128 voxels one 8-byte read of four slots, then one 16-byte
        // read per 32-row block
        auto load_a = [&](const uint16_t (*cur)[HB_ROWS][8], int t, u32x4_t* a) {
#pragma unroll
            for (int q = 0; q < RB / 4; ++q) {
                const uint2 sl = *reinterpret_cast<const uint2*>(&sL[t][(RB / 4) * rg + q][r32][0]);
                const int slots[4] = {(int)(sl.x & 0xffffu), (int)(sl.x >> 16),
                                      (int)(sl.y & 0xffffu), (int)(sl.y >> 16)};
#pragma unroll
                for (int k = 0; k < 4; ++k)
                    a[4 * q + k] = *reinterpret_cast<const u32x4_t*>(&cur[g][slots[k]][0]);
            }
        };

        // Vector-memory loads return in issue order, so waiting for a weight load also waits
        // for every slice DMA issued before it: the weights run PD taps ahead and the slice
        // pieces go out every SP-th tap, which leaves each piece >= PD+1 taps to land. The
        // weight ring has PD+1 slots indexed by tap; PD+1 must divide 27 so that the ring
        // index continues across slices with compile-time register indices.
        static_assert((2 * kTaps) % (PD + 1) == 0, "weight ring must divide 2 x 27 taps");
        static_assert(PIECES * SP <= kTaps, "slice pieces must fit in one slice's taps");
        static_assert((PIECES - 1) * SP + STG < kTaps, "every staged piece is written within its slice");
        // zero slot of both buffers and planes (the barrier below publishes it)
        if (tid < 4) {
            u32x4_t z{0, 0, 0, 0};
            asm volatile("" : "+v"(z));   // made here, not held in registers across tiles
            *reinterpret_cast<u32x4_t*>(tid < 2 ? &sH0[tid & 1][HB_ZERO][0] : &sH1[tid & 1][HB_ZERO][0]) = z;
        }
#pragma unroll
        for (int j = 0; j < PIECES; ++j) {
            u32x4_t r;
            fetch_piece(0, j, r);
            put_piece(sH0, j, r);
        }
        u32x4_t bR[PD + 1][CB];
#pragma unroll
        for (int q = 0; q < PD; ++q) load_b(q, 0, bR[q]);
        wait_vmcnt0();
        __syncthreads();

        // one slice: all 27 taps on `cur` while slice kcn streams into `nxt` (the last slice
        // re-loads itself into the idle buffer, so there is no branch here either)
        // R0: the weight ring's slot of this slice's tap 0 (slices go in pairs, so a ring size
        // that divides 2 x 27 keeps every register index static)
        auto run_slice = [&](auto ring0, const uint16_t (*cur)[HB_ROWS][8], uint16_t (*nxt)[HB_ROWS][8],
                             int kc, int kcn) {
            constexpr int R0 = decltype(ring0)::value;
            u32x4_t aC[RB], aN[RB];
            load_a(cur, 0, aC);
            // all 27 taps unrolled: register rings stay static and every wait is exact
#pragma unroll
            for (int t = 0; t < kTaps; ++t) {
                // weights PD taps ahead (the first taps of the next slice at the end)
                if (t + PD < kTaps) load_b(t + PD, kc, bR[(R0 + t + PD) % (PD + 1)]);
                else load_b(t + PD - kTaps, kcn, bR[(R0 + t + PD) % (PD + 1)]);
                if (t % SP == 0 && t / SP < PIECES) fetch_piece(kcn, t / SP, stg[(t / SP) % NSTG]);
                if (t >= STG && (t - STG) % SP == 0 && (t - STG) / SP < PIECES)
                    put_piece(nxt, (t - STG) / SP, stg[((t - STG) / SP) % NSTG]);
                if (t + 1 < kTaps) load_a(cur, t + 1, aN);
#pragma unroll
                for (int rb = 0; rb < RB; ++rb)
#pragma unroll
                    for (int cb = 0; cb < CB; ++cb)
                        acc[rb][cb] = mfma32x32x16<BF16>(aC[rb], bR[(R0 + t) % (PD + 1)][cb], acc[rb][cb]);
#pragma unroll
                for (int rb = 0; rb < RB; ++rb) aC[rb] = aN[rb];
                // keep each tap's loads in its tap: unconstrained, the scheduler gathers the
                // slice DMAs at the end of the slice, where their latency is fully exposed
                __builtin_amdgcn_sched_barrier(0);
            }
            __syncthreads();
        };
        for (int kc = 0; kc < nkc; kc += 2) {
            const int k1 = kc + 1 < nkc ? kc + 1 : kc;
            run_slice(std::integral_constant<int, 0>{}, sH0, sH1, kc, k1);
            if (kc + 1 < nkc)
                run_slice(std::integral_constant<int, kTaps % (PD + 1)>{}, sH1, sH0, kc + 1,
                          kc + 2 < nkc ? kc + 2 : kc + 1);
        }
        epilogue(acc);
    } else {
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
                    const int64_t i = row0 + 32 * RB * rg + 32 * rb + r32;
                    const int32_t v = (i < n) ? nbr[(int64_t)t * n + i] : (int32_t)n;
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
        epilogue(acc);
    }
}

template <bool BF16, int BN, int ODT, bool PLANNED>
int launch(const void* feats, int64_t n, int ci, const int32_t* nbr, const void* plan,
           const void* weight, const float* bias, int co, void* out, hipStream_t s) {
    const int64_t n_tiles = ceil_div(n, HB_M);
    const int n_ctiles = co / BN;
    const int64_t total = n_tiles * n_ctiles;
    const int64_t per_xcd = ceil_div(total, 8);
    PlanView pv{};
    if (plan) pv = carve_plan(const_cast<void*>(plan), n_tiles);
    // 8 waves of 128 voxels x BN/2 channels; weights 2 taps ahead; a slice piece every other
    // tap, written to LDS 6 taps after its load
    constexpr int RB = 4, CB = BN / 64, PD = 2, SP = 2, STG = 6;
    hipLaunchKernelGGL((k_conv_halo<BF16, BN, ODT, PLANNED, RB, CB, PD, SP, STG>),
                       dim3((unsigned)(per_xcd * 8)), dim3(hb_waves<BN, RB, CB>() * 64), 0, s,
                       reinterpret_cast<const uint16_t*>(feats), n, ci,
                       nbr, pv, reinterpret_cast<const uint16_t*>(weight), bias, co, out, n_tiles,
                       n_ctiles, per_xcd);
    TSP_CHECK_LAUNCH();
    return TSP_OK;
}

template <bool BF16, int BN, int ODT>
int launch_planned(bool planned, const void* feats, int64_t n, int ci, const int32_t* nbr,
                   const void* plan, const void* weight, const float* bias, int co, void* out,
                   hipStream_t s) {
    if (planned) return launch<BF16, BN, ODT, true>(feats, n, ci, nbr, plan, weight, bias, co, out, s);
    return launch<BF16, BN, ODT, false>(feats, n, ci, nbr, nullptr, weight, bias, co, out, s);
}

template <bool BF16, int BN>
int launch_out(int odt, bool planned, const void* feats, int64_t n, int ci, const int32_t* nbr,
               const void* plan, const void* weight, const float* bias, int co, void* out,
               hipStream_t s) {
    if (odt == TSP_F32)
        return launch_planned<BF16, BN, TSP_F32>(planned, feats, n, ci, nbr, plan, weight, bias, co, out, s);
    if (BF16 && odt == TSP_BF16)
        return launch_planned<BF16, BN, TSP_BF16>(planned, feats, n, ci, nbr, plan, weight, bias, co, out, s);
    if (!BF16 && odt == TSP_F16)
        return launch_planned<BF16, BN, TSP_F16>(planned, feats, n, ci, nbr, plan, weight, bias, co, out, s);
    set_error("MFMA conv writes f32 or the feature dtype, not %d", odt);
    return TSP_ERR_UNSUPPORTED;
}

}  // namespace

bool halo_fits(int64_t n, int ci) { return n * (int64_t)ci * 2 < ((int64_t)1 << 32); }

size_t halo_plan_bytes(int64_t n) {
    const int64_t n_tiles = std::max<int64_t>(1, ceil_div(n, HB_M));
    return align256((size_t)n_tiles * 16) + align256((size_t)n_tiles * HB_SLOTS * 4) +
           align256((size_t)n_tiles * HB_SLOT_TABLE * 2);
}

int halo_plan_build(const int32_t* nbr, int64_t n, void* plan, hipStream_t s) {
    const int64_t n_tiles = ceil_div(n, HB_M);
    if (n_tiles == 0) return TSP_OK;
    hipLaunchKernelGGL(k_plan_build, dim3((unsigned)n_tiles), dim3(HB_PLAN_NT), 0, s, nbr, n,
                       n_tiles, carve_plan(plan, n_tiles));
    TSP_CHECK_LAUNCH();
    return TSP_OK;
}

int halo_weight_pack(const void* w, int ci, int co, void* packed, hipStream_t s) {
    const int64_t blocks = (int64_t)(co / 32) * (ci / HB_KC) * kTaps;
    if (blocks == 0) return TSP_OK;
    hipLaunchKernelGGL(k_weight_pack, dim3((unsigned)blocks), dim3(64), 0, s,
                       reinterpret_cast<const uint16_t*>(w), ci, co,
                       reinterpret_cast<uint16_t*>(packed));
    TSP_CHECK_LAUNCH();
    return TSP_OK;
}

int halo_conv_launch(int fdt, int odt, const void* feats, int64_t n, int ci, const int32_t* nbr,
                     const void* plan, const void* weight, const float* bias, int co, void* out,
                     hipStream_t s) {
    const bool planned = plan != nullptr;
    const bool bn128 = co % 128 == 0;
    // the slice DMA addresses feature rows with 32-bit byte offsets
    if (!halo_fits(n, ci)) {
        set_error("MFMA conv: n * ci * 2 = %lld bytes of features exceed the 4 GiB the LDS-staged "
                  "kernel addresses", (long long)(n * ci * 2));
        return TSP_ERR_UNSUPPORTED;
    }
    if (fdt == TSP_BF16)
        return bn128 ? launch_out<true, 128>(odt, planned, feats, n, ci, nbr, plan, weight, bias, co, out, s)
                     : launch_out<true, 64>(odt, planned, feats, n, ci, nbr, plan, weight, bias, co, out, s);
    return bn128 ? launch_out<false, 128>(odt, planned, feats, n, ci, nbr, plan, weight, bias, co, out, s)
                 : launch_out<false, 64>(odt, planned, feats, n, ci, nbr, plan, weight, bias, co, out, s);
}

}  // namespace tsp
