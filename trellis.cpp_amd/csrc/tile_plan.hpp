// Conv tile plans: which input rows a tile of HB_M output voxels reads, and where each (tap, voxel)
// finds its row once those rows are staged in LDS. Shared by the plan build (plan.hip) and the conv
// kernel that builds its plan in LDS when no stored plan is given (conv_halo.hip).
#pragma once
#include "conv_internal.hpp"

namespace tsp {

constexpr int HB_PLAN_NT = 512;            // threads of a plan-build workgroup (one per voxel)
constexpr int HB_KC = 16;                  // channels per LDS slice
constexpr int HB_SLOTS = 2048;             // slots per slice buffer
constexpr int HB_ZERO = HB_SLOTS;          // slot that always holds zeros (absent taps)
constexpr int HB_ROWS = HB_SLOTS + 1;      // rows of a slice buffer plane: the slots + zero
constexpr int HB_SLOT_TABLE = kTaps * HB_M;                    // uint16 slots per tile
constexpr int HB_GAP_BUCKETS = 256;                            // buckets of a wide row range
constexpr int HB_PLAN_SCRATCH = 5 * HB_SLOTS + HB_GAP_BUCKETS / 32 + HB_GAP_BUCKETS;   // words
constexpr int64_t HB_MAXSPAN = (int64_t)HB_SLOTS * 32 * 32;    // 2^21 rows

__device__ __forceinline__ int wave_min(int v) {
    for (int off = 32; off > 0; off >>= 1) v = min(v, __shfl_xor(v, off, 64));
    return v;
}
__device__ __forceinline__ int wave_max(int v) {
    for (int off = 32; off > 0; off >>= 1) v = max(v, __shfl_xor(v, off, 64));
    return v;
}

// A stored plan, per tile of HB_M voxels:
//   hdr   int32 [4]            {H = distinct rows, direct (1: rows do not fit LDS), 0, 0}
//   rowof int32 [HB_SLOTS]     input row of each slot (slots sorted by row)
//   slots uint16 [27][4][32][4] slot of each (tap, position / 128, position % 32, position / 32 % 4)
//   vox   int32 [HB_M]         output row at each tile position, -1 for none
//   act   uint32 [4][4]        per row group g: bit 4 t + b set when some voxel of MFMA block b of
//                              the group has tap t (HB_ACT_WORDS words per group)
// Position p of a tile is row p % 32 of MFMA block (p / 32) % 4 of row group p / 128. The tiles
// partition the voxels in an order chosen by the build (compact regions of space when coordinates
// are given); inside a tile the voxels are grouped by which corner taps they have, so that a 32-row
// block often has a tap absent for all its rows (act bit clear: the conv skips that block's MFMAs
// when the weights are finite), and the blocks are dealt to the four row groups so that each
// group has about the same number of present (tap, block) pairs.
constexpr int HB_ACT_WORDS = 4;            // act words per row group: 27 taps x 4 blocks <= 128 bits
struct PlanView {
    int32_t* hdr;
    int32_t* rowof;
    uint16_t* slots;
    int32_t* vox;
    uint32_t* act;
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
    c += align256((size_t)n_tiles * HB_SLOT_TABLE * 2);
    v.vox = reinterpret_cast<int32_t*>(c);
    c += align256((size_t)n_tiles * HB_M * 4);
    v.act = reinterpret_cast<uint32_t*>(c);
    return v;
}
// bytes of the tile records (without the build's sort scratch)
inline size_t plan_tile_bytes(int64_t n_tiles) {
    return align256((size_t)n_tiles * 16) + align256((size_t)n_tiles * HB_SLOTS * 4) +
           align256((size_t)n_tiles * HB_SLOT_TABLE * 2) + align256((size_t)n_tiles * HB_M * 4) +
           align256((size_t)n_tiles * 4 * HB_ACT_WORDS * 4);
}

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

// The tile's distinct referenced rows and the slot of every (tap, voxel). Thread tid holds the
// table entries nv[t][h] of VPT voxels (-1 where a tap is absent or there is no voxel) and their
// tile positions pos[h]. Fills sL with the slot of every (tap, position) and sRowOf with the row of
// every slot; returns H (number of distinct rows) and whether the tile must take the direct path.
// The set of referenced rows is ranked with a bitmap over their offsets from lo: one fine word
// per 32 rows when the span is at most 32 * HB_SLOTS rows, otherwise two levels -- a coarse bit
// per 32-row block (spans up to 2^21 rows), then one fine word per non-empty block. slot =
// prefix of the fine word + rank inside the word, so slots are sorted by row; absent taps get
// HB_ZERO. A wider span (a tile whose voxels lie in two distant parts of the row range) is first
// cut into HB_GAP_BUCKETS buckets of 2^bs rows and the offsets renumbered over the occupied
// buckets only, which removes the empty stretches between the parts.
// scratch: HB_PLAN_SCRATCH words; sRed: 2 * NT/64 ints.
template <int NT, int VPT>
__device__ void tile_plan_core(int32_t (&nv)[kTaps][VPT], const int (&pos)[VPT],
                               uint16_t (*sL)[4][32][4], int32_t* sRowOf, uint32_t* scratch,
                               int* sRed, int& H_out, bool& direct_out) {
    constexpr int WPT = HB_SLOTS / NT;     // bitmap words per thread
    constexpr int NW = NT / 64;
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    uint32_t* coarse = scratch;                                       // bit per 32-row block
    int32_t* cpre = reinterpret_cast<int32_t*>(scratch + HB_SLOTS);   // block rank of a word
    uint32_t* fine = scratch + 2 * HB_SLOTS;                          // rows of each block
    int32_t* fpre = reinterpret_cast<int32_t*>(scratch + 3 * HB_SLOTS);
    int32_t* block_of = reinterpret_cast<int32_t*>(scratch + 4 * HB_SLOTS);   // rank -> block
    uint32_t* gmask = scratch + 5 * HB_SLOTS;                          // occupied gap buckets
    int32_t* gbucket = reinterpret_cast<int32_t*>(gmask + HB_GAP_BUCKETS / 32);   // rank -> bucket
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
    // from here on entries are offsets from lo (renumbered over occupied buckets when wide)
    const int row_lo = lo;
    int bs = -1;   // bucket shift when the offsets were renumbered
    if (hi >= 0 && (int64_t)hi - lo + 1 > HB_MAXSPAN) {
        bs = 0;
        while (((int64_t)HB_GAP_BUCKETS << bs) < (int64_t)hi - lo + 1) ++bs;
        if (tid < HB_GAP_BUCKETS / 32) gmask[tid] = 0u;
        __syncthreads();
#pragma unroll
        for (int t = 0; t < kTaps; ++t)
#pragma unroll
            for (int h = 0; h < VPT; ++h)
                if (nv[t][h] >= 0) {
                    const int b = (nv[t][h] - lo) >> bs;
                    atomicOr(&gmask[b >> 5], 1u << (b & 31));
                }
        __syncthreads();
        // occupied bucket ranks: rank(b) = occupied buckets below b
        auto brank = [&](int b) {
            int r = __popc(gmask[b >> 5] & ((1u << (b & 31)) - 1u));
            for (int w = 0; w < (b >> 5); ++w) r += __popc(gmask[w]);
            return r;
        };
        if (tid < HB_GAP_BUCKETS && ((gmask[tid >> 5] >> (tid & 31)) & 1u)) gbucket[brank(tid)] = tid;
        int nocc = 0;
        for (int w = 0; w < HB_GAP_BUCKETS / 32; ++w) nocc += __popc(gmask[w]);
        const int lmask = (1 << bs) - 1;
#pragma unroll
        for (int t = 0; t < kTaps; ++t)
#pragma unroll
            for (int h = 0; h < VPT; ++h)
                if (nv[t][h] >= 0) {
                    const int d = nv[t][h] - lo;
                    nv[t][h] = (brank(d >> bs) << bs) | (d & lmask);
                }
        lo = 0;
        hi = (int)(((int64_t)nocc << bs) - 1);
        __syncthreads();   // gbucket is read when the rows of the slots are written
    } else if (hi >= 0) {
#pragma unroll
        for (int t = 0; t < kTaps; ++t)
#pragma unroll
            for (int h = 0; h < VPT; ++h)
                if (nv[t][h] >= 0) nv[t][h] -= lo;
        hi -= lo;
        lo = 0;
    }
    // the input row of offset d
    auto row_of = [&](int d) {
        return bs < 0 ? row_lo + d : row_lo + ((gbucket[d >> bs] << bs) | (d & ((1 << bs) - 1)));
    };
    bool direct = hi >= 0 && (int64_t)hi - lo + 1 > HB_MAXSPAN;
    // One level when the rows span at most 32 * HB_SLOTS (the usual case for sorted sets: a
    // tile's neighbours lie in a few x-planes): the fine word of row d is d >> 5 directly.
    const bool one = hi >= 0 && (int64_t)hi - lo + 1 <= 32 * HB_SLOTS;
    int H = 0, nfine = 0;
    // fine word of row offset d (two levels: the rank of d's 32-row block among the referenced ones)
    auto fine_word = [&](int d) -> int {
        if (one) return d >> 5;
        const int cw = d >> 10, cb = (d >> 5) & 31;
        return cpre[cw] + (int)__popc(coarse[cw] & ((1u << cb) - 1u));
    };

    if (!direct && hi >= 0) {
#pragma unroll
        for (int k = 0; k < WPT; ++k) {
            coarse[tid * WPT + k] = 0u;
            fine[tid * WPT + k] = 0u;
        }
        __syncthreads();
        if (one) {
            nfine = HB_SLOTS;
        } else {
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
            nfine = scan_popcounts<NT>(coarse, HB_SLOTS, cpre, sRed);
            direct = nfine > HB_ZERO;      // every block holds a row: too many rows for LDS
            if (!direct) {
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
            }
        }
        if (!direct) {
            // level 2: rows within each referenced block
#pragma unroll
            for (int t = 0; t < kTaps; ++t)
#pragma unroll
                for (int h = 0; h < VPT; ++h) {
                    const int32_t v = nv[t][h];
                    if (v >= 0) {
                        const int d = v - lo;
                        atomicOr(&fine[fine_word(d)], 1u << (d & 31));
                    }
                }
            __syncthreads();
            H = scan_popcounts<NT>(fine, nfine, fpre, sRed);
            direct = H > HB_ZERO;
        }
    }
    if (!direct) {
        // slot of every (tap, voxel), stored at the voxel's tile position
#pragma unroll
        for (int t = 0; t < kTaps; ++t)
#pragma unroll
            for (int h = 0; h < VPT; ++h) {
                const int rr = pos[h];
                const int32_t v = nv[t][h];
                int slot = HB_ZERO;
                if (v >= 0) {
                    const int d = v - lo, fw = fine_word(d);
                    slot = fpre[fw] + __popc(fine[fw] & ((1u << (d & 31)) - 1u));
                }
                sL[t][rr >> 7][rr & 31][(rr >> 5) & 3] = (uint16_t)slot;
            }
        // row of every slot
#pragma unroll
        for (int k = 0; k < WPT; ++k) {
            const int w = tid * WPT + k;
            if (w < nfine) {
                uint32_t bits = fine[w];
                int s = fpre[w];
                const int base = (one ? w : block_of[w]) * 32;
                while (bits) {
                    const int bit = __builtin_ctz(bits);
                    bits &= bits - 1u;
                    sRowOf[s++] = row_of(base + bit);
                }
            }
        }
    }
    __syncthreads();
    H_out = H;
    direct_out = direct;
}

// The table entries of voxel i (-1 for absent taps, or for every tap when i < 0).
template <int VPT>
__device__ __forceinline__ void load_entries(const int32_t* __restrict__ nbr, int64_t n,
                                             const int64_t (&i)[VPT], int32_t (&nv)[kTaps][VPT]) {
    int64_t ic[VPT];
#pragma unroll
    for (int h = 0; h < VPT; ++h) ic[h] = i[h] >= 0 ? i[h] : 0;
    // loaded without branches so that all loads are in flight together
#pragma unroll
    for (int t = 0; t < kTaps; ++t)
#pragma unroll
        for (int h = 0; h < VPT; ++h) nv[t][h] = nbr[(int64_t)t * n + ic[h]];
#pragma unroll
    for (int t = 0; t < kTaps; ++t)
#pragma unroll
        for (int h = 0; h < VPT; ++h)
            nv[t][h] = (i[h] >= 0 && (uint32_t)nv[t][h] < (uint32_t)n) ? nv[t][h] : -1;
}

}  // namespace tsp
