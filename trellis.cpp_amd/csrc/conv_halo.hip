// MFMA submanifold conv with each tile's neighbour rows staged in LDS.
//
// A workgroup owns HB_M = 512 consecutive output voxels x BN output channels and runs 8 waves,
// two per SIMD: wave w owns voxels [128 (w%4), +128) x channels [(w/4) BN/2, +BN/2). On
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
//   * the distinct rows stream through LDS 16 channels at a time (two buffers, DMA straight
//     from global memory to LDS), the next slice loading while the current one runs all 27
//     taps. Each buffer holds the two 8-channel halves of a row in separate planes, so the 32
//     lanes that feed one MFMA operand read 32 consecutive 16-byte words: conflict-free.
//   * per tap, A operands are read from LDS by slot and B operands (weights) come from L2 two
//     taps ahead. Packed weights ([co/32][ci/16][27][64 lanes][8]) make every weight load one
//     contiguous 1 KiB per wave.
//   * the epilogue stages 32-row blocks of the accumulators in LDS and writes whole rows.
// A tile whose row range or distinct-row count does not fit (scattered or unsorted inputs)
// takes the direct path: the same MFMA loop with A gathered straight from global memory.
#include <algorithm>

#include "conv_internal.hpp"

namespace tsp {
namespace {

constexpr int HB_NT = 512;                 // threads of a conv workgroup (8 waves)
constexpr int HB_PLAN_NT = 256;            // threads of a plan-build workgroup
constexpr int HB_KC = 16;                  // channels per LDS slice
constexpr int HB_SLOTS = 2048;             // slots per slice buffer
constexpr int HB_ZERO = HB_SLOTS - 1;      // slot that always holds zeros (absent taps)
constexpr int HB_PIECES = 2 * HB_SLOTS / 64 / (HB_NT / 64);   // slice DMA ops per wave (8)
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

// Plan layout: [n_tiles][4] int32 header {H, direct, 0, 0} | [n_tiles][HB_SLOTS] int32 row of
// each slot | [n_tiles][27][4][32][4] uint16 slot of each (tap, voxel/128, voxel%32,
// voxel/32%4).
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
template <bool BF16, int BN, int ODT, bool PLANNED>
__global__ __launch_bounds__(HB_NT, 1) void k_conv_halo(
    const uint16_t* __restrict__ feats, int64_t n, int ci, const int32_t* __restrict__ nbr,
    PlanView plan, const uint16_t* __restrict__ weight, const float* __restrict__ bias, int co,
    void* __restrict__ out, int64_t n_tiles, int n_ctiles, int64_t per_xcd) {
    constexpr int WN = BN / 2;               // output channels per wave
    constexpr int CB = WN / 32;              // 32-wide column blocks per wave
    // slice buffers [buffer][half][slot][8 ch] and the slot table [tap][row block][voxel%32][rb]
    __shared__ __attribute__((aligned(16))) uint16_t sH[2][2][HB_SLOTS][8];
    __shared__ __attribute__((aligned(16))) uint16_t sL[kTaps][4][32][4];
    __shared__ int sRed[2 * HB_NT / 64];

    // XCD-aware order: workgroup ids go round-robin over the 8 XCDs, so each XCD gets one
    // contiguous range of (tile, column-tile) pairs and gathers from rows its L2 already holds.
    const int64_t b = blockIdx.x;
    const int64_t lin = (b % 8) * per_xcd + b / 8;
    if (lin >= n_tiles * n_ctiles) return;
    const int64_t tile = lin / n_ctiles;
    const int64_t row0 = tile * HB_M;

    const int tid = threadIdx.x;
    const int wave = tid >> 6, lane = tid & 63;
    const int r32 = lane & 31, g = lane >> 5;
    const int wm = wave & 3;                 // 128-voxel row block of this wave
    const int c0 = (int)(lin % n_ctiles) * BN + (wave >> 2) * WN;   // first channel of wave
    const int nkc = ci / HB_KC;
    // slice DMA: wave w streams plane (w & 1), 64-slot blocks (w >> 1) + 4 j
    const int plane = wave & 1;

    // ---- tile plan: slot table in LDS, rows of this thread's slice pieces in registers
    int H;
    bool direct;
    int32_t prow[HB_PIECES];
    if constexpr (PLANNED) {
        const int32_t* hdr = plan.hdr + tile * 4;
        H = hdr[0];
        direct = hdr[1] != 0;
        if (!direct) {
            const char* src = reinterpret_cast<const char*>(plan.slots + tile * HB_SLOT_TABLE);
            for (int p = wave; p < HB_SLOT_TABLE * 2 / 1024; p += HB_NT / 64)   // 27 x 1 KiB
                __builtin_amdgcn_global_load_lds(
                    src + p * 1024 + lane * 16,
                    (__attribute__((address_space(3))) void*)(reinterpret_cast<char*>(&sL[0][0][0][0]) + p * 1024),
                    16, 0, 0);
            const int32_t* ro = plan.rowof + tile * HB_SLOTS;
#pragma unroll
            for (int j = 0; j < HB_PIECES; ++j) {
                const int slot = 64 * ((wave >> 1) + 4 * j) + lane;
                prow[j] = slot < H ? ro[slot] : 0;
            }
        }
    } else {
        tile_plan<HB_NT>(nbr, n, row0, sL, reinterpret_cast<int32_t*>(&sH[0][0][0][0]),
                         reinterpret_cast<uint32_t*>(&sH[1][0][0][0]), sRed, H, direct);
        if (!direct) {
            const int32_t* sRowOf = reinterpret_cast<const int32_t*>(&sH[0][0][0][0]);
#pragma unroll
            for (int j = 0; j < HB_PIECES; ++j) {
                const int slot = 64 * ((wave >> 1) + 4 * j) + lane;
                prow[j] = slot < H ? sRowOf[slot] : 0;
            }
            __syncthreads();     // sH[0] is overwritten by the first slice below
        }
    }

    f32x16_t acc[4][CB];
#pragma unroll
    for (int rb = 0; rb < 4; ++rb)
#pragma unroll
        for (int cb = 0; cb < CB; ++cb)
#pragma unroll
            for (int j = 0; j < 16; ++j) acc[rb][cb][j] = 0.f;

    // weights of (tap t, slice kc), column block cb of this wave
    uint32_t boff[CB];
#pragma unroll
    for (int cb = 0; cb < CB; ++cb) {
        if constexpr (PLANNED)   // packed: block ((co/32 index) * nkc + kc) * 27 + t, 1 KiB each
            boff[cb] = (uint32_t)((((c0 >> 5) + cb) * nkc * kTaps * 64 + lane) * 16u);
        else                     // [co][27][ci]
            boff[cb] = (uint32_t)(((uint32_t)(c0 + cb * 32 + r32) * (uint32_t)(kTaps * ci) + g * 8) * 2u);
    }
    auto load_b = [&](int t, int kc, u32x4_t* dst) {
        const char* wt;
        if constexpr (PLANNED) wt = reinterpret_cast<const char*>(weight) + ((int64_t)kc * kTaps + t) * 1024;
        else wt = reinterpret_cast<const char*>(weight + (t * ci + kc * HB_KC));
#pragma unroll
        for (int cb = 0; cb < CB; ++cb) dst[cb] = *reinterpret_cast<const u32x4_t*>(wt + boff[cb]);
    };

    if (!direct) {
        // zero slot of both buffers and planes (slice loads only write slots < H <= HB_ZERO)
        if (tid < 4) *reinterpret_cast<u32x4_t*>(&sH[tid >> 1][tid & 1][HB_ZERO][0]) = u32x4_t{0, 0, 0, 0};

        // slice kc -> buffer buf: this thread's piece j (DMA straight to LDS)
        auto load_slice_part = [&](int kc, int buf, int j) {
            const int s0 = 64 * ((wave >> 1) + 4 * j);
            if (s0 < H) {
                if (s0 + lane < H) {
                    const uint16_t* src = feats + (int64_t)prow[j] * ci + kc * HB_KC + plane * 8;
                    __builtin_amdgcn_global_load_lds(
                        src, (__attribute__((address_space(3))) void*)(&sH[buf][plane][s0][0]),
                        16, 0, 0);
                }
            }
        };
        // A operands of tap t: one 8-byte read of the four slots, four 16-byte reads
        auto load_a = [&](int buf, int t, u32x4_t* a) {
            const uint2 sl = *reinterpret_cast<const uint2*>(&sL[t][wm][r32][0]);
            const int slots[4] = {(int)(sl.x & 0xffffu), (int)(sl.x >> 16),
                                  (int)(sl.y & 0xffffu), (int)(sl.y >> 16)};
#pragma unroll
            for (int rb = 0; rb < 4; ++rb)
                a[rb] = *reinterpret_cast<const u32x4_t*>(&sH[buf][g][slots[rb]][0]);
        };

        // Vector-memory loads return in issue order, so waiting for a weight load also waits
        // for every slice DMA issued before it: the weights run PD taps ahead and the slice
        // pieces go out every SP-th tap, which leaves each piece >= PD+1 taps to land. The
        // weight ring has PD+1 slots indexed by tap; PD+1 must divide 27 so that the ring
        // index continues across slices with compile-time register indices.
        constexpr int PD = 2, SP = 2;
        static_assert(kTaps % (PD + 1) == 0, "weight ring must divide the 27 taps");
        static_assert(HB_PIECES * SP <= kTaps, "slice pieces must fit in one slice's taps");
#pragma unroll
        for (int j = 0; j < HB_PIECES; ++j) load_slice_part(0, 0, j);
        u32x4_t bR[PD + 1][CB];
#pragma unroll
        for (int q = 0; q < PD; ++q) load_b(q, 0, bR[q]);
        wait_vmcnt0();
        __syncthreads();

        for (int kc = 0; kc < nkc; ++kc) {
            const int buf = kc & 1;
            const bool next = kc + 1 < nkc;
            const int kcn = next ? kc + 1 : kc;
            u32x4_t aC[4], aN[4];
            load_a(buf, 0, aC);
            // all 27 taps unrolled: register rings stay static and every wait is exact
#pragma unroll
            for (int t = 0; t < kTaps; ++t) {
                // weights PD taps ahead (the first taps of the next slice at the end)
                if (t + PD < kTaps) load_b(t + PD, kc, bR[(t + PD) % (PD + 1)]);
                else load_b(t + PD - kTaps, kcn, bR[(t + PD) % (PD + 1)]);
                if (next && t % SP == 0 && t / SP < HB_PIECES) load_slice_part(kc + 1, buf ^ 1, t / SP);
                if (t + 1 < kTaps) load_a(buf, t + 1, aN);
#pragma unroll
                for (int rb = 0; rb < 4; ++rb)
#pragma unroll
                    for (int cb = 0; cb < CB; ++cb)
                        acc[rb][cb] = mfma32x32x16<BF16>(aC[rb], bR[t % (PD + 1)][cb], acc[rb][cb]);
#pragma unroll
                for (int rb = 0; rb < 4; ++rb) aC[rb] = aN[rb];
            }
            wait_vmcnt0();
            __syncthreads();
        }
    } else {
        // ---- direct path: A gathered from global memory
        for (int kc = 0; kc < nkc; ++kc)
            for (int t = 0; t < kTaps; ++t) {
                u32x4_t bq[CB];
                load_b(t, kc, bq);
                u32x4_t a[4];
#pragma unroll
                for (int rb = 0; rb < 4; ++rb) {
                    const int64_t i = row0 + 128 * wm + 32 * rb + r32;
                    const int32_t v = (i < n) ? nbr[(int64_t)t * n + i] : (int32_t)n;
                    a[rb] = u32x4_t{0, 0, 0, 0};
                    if ((uint32_t)v < (uint32_t)n)
                        a[rb] = *reinterpret_cast<const u32x4_t*>(feats + (int64_t)v * ci +
                                                                  kc * HB_KC + g * 8);
                }
#pragma unroll
                for (int rb = 0; rb < 4; ++rb)
#pragma unroll
                    for (int cb = 0; cb < CB; ++cb)
                        acc[rb][cb] = mfma32x32x16<BF16>(a[rb], bq[cb], acc[rb][cb]);
            }
    }

    // ---- epilogue: each wave stages 32-row blocks of its accumulators (fp32, + bias) in its own
    // 16 KiB of the slice buffers, then writes whole row segments, 4 channels per lane. The row
    // stride WN*4+32 bytes puts the two 32-lane halves of a staging write on disjoint banks.
    // (The slice buffers are idle: every wave passed the last barrier of the main loop, or of
    // the plan on the direct path.)
    constexpr int RS = WN * 4 + 32;
    char* stage = reinterpret_cast<char*>(&sH[0][0][0][0]) + wave * 16384;
    float bv[CB];
#pragma unroll
    for (int cb = 0; cb < CB; ++cb) bv[cb] = bias[c0 + cb * 32 + r32];
#pragma unroll
    for (int rb = 0; rb < 4; ++rb) {
#pragma unroll
        for (int cb = 0; cb < CB; ++cb)
#pragma unroll
            for (int j = 0; j < 16; ++j) {
                const int r = 8 * (j / 4) + 4 * g + (j % 4);
                *reinterpret_cast<float*>(stage + r * RS + (cb * 32 + r32) * 4) = acc[rb][cb][j] + bv[cb];
            }
#pragma unroll
        for (int q = 0; q < WN / 8; ++q) {           // 32 rows x WN/4 chunks of 4 channels
            const int c = q * 64 + lane;
            const int r = c / (WN / 4), cq = c % (WN / 4);
            const f32x4_t v = *reinterpret_cast<const f32x4_t*>(stage + r * RS + cq * 16);
            const int64_t i = row0 + 128 * wm + 32 * rb + r;
            if (i < n) {
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
    hipLaunchKernelGGL((k_conv_halo<BF16, BN, ODT, PLANNED>), dim3((unsigned)(per_xcd * 8)),
                       dim3(HB_NT), 0, s, reinterpret_cast<const uint16_t*>(feats), n, ci,
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
    if (fdt == TSP_BF16)
        return bn128 ? launch_out<true, 128>(odt, planned, feats, n, ci, nbr, plan, weight, bias, co, out, s)
                     : launch_out<true, 64>(odt, planned, feats, n, ci, nbr, plan, weight, bias, co, out, s);
    return bn128 ? launch_out<false, 128>(odt, planned, feats, n, ci, nbr, plan, weight, bias, co, out, s)
                 : launch_out<false, 64>(odt, planned, feats, n, ci, nbr, plan, weight, bias, co, out, s);
}

}  // namespace tsp
