// Conv plans (tsp_conv_plan_build, tsp_conv_plan_build_ordered).
//
// A plan splits the output voxels into tiles of HB_M and records, per tile, the input rows its
// table entries reference and the LDS slot of every (tap, voxel) (tile_plan.hpp). Which voxels
// share a tile decides how many rows a tile stages: with coordinates, voxels are ordered by the
// Morton code of their 8^3 cell (a stable radix sort, so voxels of one cell keep their row order)
// and each run of HB_M voxels is a tile -- a compact patch of the surface, whose neighbours are
// ~1.7 distinct rows per voxel on thin shells instead of ~3.3 for HB_M consecutive rows of an
// x-major set. Without coordinates tiles are consecutive rows. Inside a tile the voxels are
// grouped by which corner taps they have (see k_plan_build). The conv's results do not depend on
// the grouping: every output row sums the same products in the same order wherever it sits (a
// skipped absent tap would only have added exact zeros).
#include <algorithm>

#include "tile_plan.hpp"

namespace tsp {
namespace {

// ---- Morton order of 8^3 cells: stable LSD radix sort, 8-bit digits -----------------------------
constexpr int RS_NT = 512;                  // threads per sort workgroup
constexpr int RS_ROUNDS = 16;               // items per thread and pass
constexpr int RS_TILE = RS_NT * RS_ROUNDS;  // items per sort workgroup
constexpr int RS_BINS = 256;
constexpr int RS_PASSES = 3;                // 24-bit keys
constexpr int RS_SCAN_NT = 256;

// bits of v (8 used) spread to every third position
__device__ __forceinline__ uint32_t spread3(uint32_t v) {
    uint32_t r = 0;
#pragma unroll
    for (int b = 0; b < 8; ++b) r |= ((v >> b) & 1u) << (3 * b);
    return r;
}

// key = Morton code of the voxel's 8^3 cell (8 bits per axis, x most significant; coordinates past
// 2^11 wrap, which only costs locality), value = row
__global__ void k_order_keys(const int32_t* __restrict__ coords, int64_t n, uint32_t* __restrict__ keys,
                             int32_t* __restrict__ vals) {
    const int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
    if (i >= n) return;
    const uint32_t x = (uint32_t)coords[3 * i] >> 3, y = (uint32_t)coords[3 * i + 1] >> 3,
                   z = (uint32_t)coords[3 * i + 2] >> 3;
    keys[i] = (spread3(x & 255u) << 2) | (spread3(y & 255u) << 1) | spread3(z & 255u);
    vals[i] = (int32_t)i;
}

// digit counts of each workgroup's RS_TILE keys: hist[digit * nblk + workgroup]
__global__ __launch_bounds__(RS_NT) void k_rs_hist(const uint32_t* __restrict__ kin, int64_t n, int shift,
                                                   int32_t* __restrict__ hist, int nblk) {
    __shared__ int sH[RS_BINS];
    const int tid = threadIdx.x;
    if (tid < RS_BINS) sH[tid] = 0;
    __syncthreads();
    const int64_t base = (int64_t)blockIdx.x * RS_TILE;
    for (int r = 0; r < RS_ROUNDS; ++r) {
        const int64_t i = base + r * RS_NT + tid;
        if (i < n) atomicAdd(&sH[(kin[i] >> shift) & (RS_BINS - 1)], 1);
    }
    __syncthreads();
    if (tid < RS_BINS) hist[(int64_t)tid * nblk + blockIdx.x] = sH[tid];
}

// Exclusive prefix sum of one digit's row hist[digit * nblk + 0 .. nblk) in place (a workgroup per
// digit), its total into tot[digit]. The digits' bases are added by the scatter.
__global__ __launch_bounds__(RS_SCAN_NT) void k_rs_scan_rows(int32_t* __restrict__ hist, int nblk,
                                                             int32_t* __restrict__ tot) {
    __shared__ int sW[RS_SCAN_NT / 64];
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    int32_t* a = hist + (int64_t)blockIdx.x * nblk;
    int carry = 0;
    for (int t0 = 0; t0 < nblk; t0 += RS_SCAN_NT) {
        const int i = t0 + tid;
        const int v = i < nblk ? a[i] : 0;
        int x = v;   // inclusive scan over the wave
#pragma unroll
        for (int off = 1; off < 64; off <<= 1) {
            const int y = __shfl_up(x, off, 64);
            if (lane >= off) x += y;
        }
        if (lane == 63) sW[wave] = x;
        __syncthreads();
        int before = 0, total = 0;
#pragma unroll
        for (int w = 0; w < RS_SCAN_NT / 64; ++w) {
            before += w < wave ? sW[w] : 0;
            total += sW[w];
        }
        if (i < nblk) a[i] = carry + before + x - v;
        carry += total;
        __syncthreads();   // sW is rewritten by the next round
    }
    if (tid == 0) tot[blockIdx.x] = carry;
}

// Stable scatter of each workgroup's RS_TILE (key, value) pairs to their digit's range. Pairs are
// ranked in index order: round by round (RS_NT consecutive pairs), wave by wave, lane by lane. A
// lane's rank among its wave's lanes of the same digit comes from ballots of the digit's 8 bits.
__global__ __launch_bounds__(RS_NT) void k_rs_scatter(const uint32_t* __restrict__ kin,
                                                      const int32_t* __restrict__ vin, int64_t n, int shift,
                                                      const int32_t* __restrict__ off, const int32_t* __restrict__ tot,
                                                      int nblk, uint32_t* __restrict__ kout,
                                                      int32_t* __restrict__ vout) {
    constexpr int NW = RS_NT / 64;
    static_assert(RS_BINS == 4 * 64 && NW >= 4, "digit bases: four waves of 64 digits");
    __shared__ int sCnt[NW][RS_BINS];   // a round's count (then first rank) per (wave, digit)
    __shared__ int sRun[RS_BINS];       // pairs of each digit placed by earlier rounds
    __shared__ int sGlob[RS_BINS];      // the workgroup's first position per digit
    __shared__ int sTot[4];
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    // the digit's base (exclusive scan of the digit totals) + this workgroup's offset in its row
    int dbase = 0;
    if (tid < RS_BINS) {
        const int t = tot[tid];
        int x = t;
#pragma unroll
        for (int o = 1; o < 64; o <<= 1) {
            const int y = __shfl_up(x, o, 64);
            if (lane >= o) x += y;
        }
        if (lane == 63) sTot[wave] = x;
        dbase = x - t;
    }
    __syncthreads();
    if (tid < RS_BINS) {
        for (int w = 0; w < wave; ++w) dbase += sTot[w];
        sRun[tid] = 0;
        sGlob[tid] = dbase + off[(int64_t)tid * nblk + blockIdx.x];
    }
    const int64_t base = (int64_t)blockIdx.x * RS_TILE;
    const uint64_t below = (1ull << lane) - 1ull;
    for (int r = 0; r < RS_ROUNDS; ++r) {
        for (int k = tid; k < NW * RS_BINS; k += RS_NT) (&sCnt[0][0])[k] = 0;
        __syncthreads();
        const int64_t i = base + r * RS_NT + tid;
        const bool valid = i < n;
        const uint32_t key = valid ? kin[i] : 0u;
        const int32_t val = valid ? vin[i] : 0;
        const int d = (int)((key >> shift) & (RS_BINS - 1));
        uint64_t peers = __ballot(valid);
#pragma unroll
        for (int b = 0; b < 8; ++b) {
            const uint64_t set = __ballot((d >> b) & 1);
            peers &= ((d >> b) & 1) ? set : ~set;
        }
        const int rank = __popcll(peers & below);
        if (valid && rank == 0) sCnt[wave][d] = __popcll(peers);
        __syncthreads();
        if (tid < RS_BINS) {
            int run = sRun[tid];
#pragma unroll
            for (int w = 0; w < NW; ++w) {
                const int c = sCnt[w][tid];
                sCnt[w][tid] = run;
                run += c;
            }
            sRun[tid] = run;
        }
        __syncthreads();
        if (valid) {
            const int64_t pos = (int64_t)sGlob[d] + sCnt[wave][d] + rank;
            kout[pos] = key;
            vout[pos] = val;
        }
        __syncthreads();   // sCnt is cleared by the next round
    }
}

struct SortScratch {
    uint32_t* keys[2];
    int32_t* vals[2];
    int32_t* hist;
    int32_t* tot;
    int nblk;
};
size_t sort_scratch_bytes(int64_t n) {
    const int64_t nblk = ceil_div(std::max<int64_t>(n, 1), RS_TILE);
    return 4 * align256((size_t)n * 4) + align256((size_t)nblk * RS_BINS * 4) + align256(RS_BINS * 4);
}
SortScratch carve_sort(void* p, int64_t n) {
    char* c = reinterpret_cast<char*>(p);
    SortScratch s;
    for (int b = 0; b < 2; ++b) {
        s.keys[b] = reinterpret_cast<uint32_t*>(c);
        c += align256((size_t)n * 4);
        s.vals[b] = reinterpret_cast<int32_t*>(c);
        c += align256((size_t)n * 4);
    }
    s.hist = reinterpret_cast<int32_t*>(c);
    s.nblk = (int)ceil_div(std::max<int64_t>(n, 1), RS_TILE);
    c += align256((size_t)s.nblk * RS_BINS * 4);
    s.tot = reinterpret_cast<int32_t*>(c);
    return s;
}

// Voxel rows in Morton order of their 8^3 cells; returns the buffer holding them.
int morton_order(const int32_t* coords, int64_t n, const SortScratch& ss, hipStream_t s,
                 const int32_t** order) {
    hipLaunchKernelGGL(k_order_keys, dim3((unsigned)ceil_div(n, 256)), dim3(256), 0, s, coords, n,
                       ss.keys[0], ss.vals[0]);
    TSP_CHECK_LAUNCH();
    int cur = 0;
    for (int pass = 0; pass < RS_PASSES; ++pass, cur ^= 1) {
        const int shift = 8 * pass;
        hipLaunchKernelGGL(k_rs_hist, dim3(ss.nblk), dim3(RS_NT), 0, s, ss.keys[cur], n, shift, ss.hist, ss.nblk);
        TSP_CHECK_LAUNCH();
        hipLaunchKernelGGL(k_rs_scan_rows, dim3(RS_BINS), dim3(RS_SCAN_NT), 0, s, ss.hist, ss.nblk, ss.tot);
        TSP_CHECK_LAUNCH();
        hipLaunchKernelGGL(k_rs_scatter, dim3(ss.nblk), dim3(RS_NT), 0, s, ss.keys[cur], ss.vals[cur], n, shift,
                           ss.hist, ss.tot, ss.nblk, ss.keys[cur ^ 1], ss.vals[cur ^ 1]);
        TSP_CHECK_LAUNCH();
    }
    *order = ss.vals[cur];
    return TSP_OK;
}

// ---- the plan of one tile per workgroup (HB_PLAN_NT threads, one voxel each) ------------------------
// Positions inside the tile: the voxels grouped by which of the 8 corner taps they have (a stable
// counting sort of 9-bit digits in LDS: voxels with the same corners mostly share their other
// taps too, so a tap is often absent from all 32 rows of an MFMA block and costs no MFMA there);
// then the 16 blocks are dealt to the 4 row groups (one per SIMD) so that the groups' MFMA counts
// stay close.
__global__ __launch_bounds__(HB_PLAN_NT) void k_plan_build(const int32_t* __restrict__ nbr, int64_t n,
                                                           const int32_t* __restrict__ order,
                                                           int64_t n_tiles, PlanView plan) {
    static_assert(HB_PLAN_NT == HB_M, "one thread per tile position");
    constexpr int NB = HB_M / 32;                 // MFMA row blocks of a tile
    constexpr int NW = HB_PLAN_NT / 64;
    constexpr int ND = 257;                       // digits: corner sets 0..255, 256 = no voxel
    __shared__ __attribute__((aligned(16))) uint16_t sL[kTaps][4][32][4];
    __shared__ __attribute__((aligned(16))) int32_t sRowOf[HB_SLOTS];
    __shared__ uint32_t sScratch[HB_PLAN_SCRATCH];
    __shared__ int sRed[2 * HB_PLAN_NT / 64];
    __shared__ uint32_t sBlk[NB];                 // present taps of each sorted block
    __shared__ int sBase[NB];                     // first position of each sorted block
    __shared__ uint32_t sAct[4 * HB_ACT_WORDS];   // the tile's act words
    // Until tile_plan_core, sRowOf holds the taps and the thread of each sorted index and the
    // position of each thread, and the scratch the sort's counts.
    static_assert(HB_SLOTS * 4 >= HB_M * 4 + HB_M * 2 + HB_M * 2, "sort records fit the row list");
    static_assert(HB_PLAN_SCRATCH >= NW * ND + ND + 64, "sort counts fit the scratch");
    uint32_t* sTaps = reinterpret_cast<uint32_t*>(sRowOf);
    uint16_t* sTid = reinterpret_cast<uint16_t*>(sTaps + HB_M);
    uint16_t* sPos = sTid + HB_M;
    int* sCnt = reinterpret_cast<int*>(sScratch);            // [NW][ND]: count, then first rank
    int* sDig = sCnt + NW * ND;                               // [ND]: first sorted index of a digit
    int* sWsum = sDig + ND;                                   // scan of the digit totals

    const int64_t tile = blockIdx.x;
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int64_t q = tile * HB_M + tid;
    int64_t i[1] = {q < n ? (order ? (int64_t)order[q] : q) : -1};
    int32_t nv[kTaps][1];
    load_entries<1>(nbr, n, i, nv);
    uint32_t taps = 0;
#pragma unroll
    for (int t = 0; t < kTaps; ++t) taps |= (nv[t][0] >= 0 ? 1u : 0u) << t;
    constexpr int kCorner[8] = {0, 2, 6, 8, 18, 20, 24, 26};   // taps (+-1, +-1, +-1)
    int d = 0;
#pragma unroll
    for (int k = 0; k < 8; ++k) d |= ((taps >> kCorner[k]) & 1u) << k;
    if (i[0] < 0) d = ND - 1;                     // empty positions sort last
    for (int k = tid; k < NW * ND; k += HB_PLAN_NT) sCnt[k] = 0;
    if (tid < 4 * HB_ACT_WORDS) sAct[tid] = 0u;
    // rank among this wave's lanes with the same digit (lanes in order)
    uint64_t peers = ~0ull;
#pragma unroll
    for (int b = 0; b < 9; ++b) {
        const uint64_t set = __ballot((d >> b) & 1);
        peers &= ((d >> b) & 1) ? set : ~set;
    }
    const int rank = __popcll(peers & ((1ull << lane) - 1ull));
    __syncthreads();
    if (rank == 0) sCnt[wave * ND + d] = __popcll(peers);
    __syncthreads();
    // per digit: counts of the waves before, and the digit's total
    int tot = 0;
    if (tid < ND) {
#pragma unroll
        for (int w = 0; w < NW; ++w) {
            const int c = sCnt[w * ND + tid];
            sCnt[w * ND + tid] = tot;
            tot += c;
        }
    }
    // exclusive scan of the digit totals (digits tid < ND, waves 0..4)
    int x = tot;
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
        const int y = __shfl_up(x, off, 64);
        if (lane >= off) x += y;
    }
    if (lane == 63) sWsum[wave] = x;
    __syncthreads();
    if (tid < ND) {
        int before = 0;
        for (int w = 0; w < wave; ++w) before += sWsum[w];
        sDig[tid] = before + x - tot;
    }
    __syncthreads();
    const int sidx = sDig[d] + sCnt[wave * ND + d] + rank;   // this voxel's sorted index
    sTaps[sidx] = i[0] >= 0 ? taps : 0u;
    sTid[sidx] = (uint16_t)tid;
    __syncthreads();
    // thread tid now stands for sorted index tid: the present taps of its 32-row block
    uint32_t bt = sTaps[tid];
#pragma unroll
    for (int off = 1; off < 32; off <<= 1) bt |= __shfl_xor(bt, off, 64);
    if ((lane & 31) == 0) sBlk[tid >> 5] = bt;
    __syncthreads();
    // The blocks, ranked by present taps (most first; ties: sorted order), are dealt to the row
    // groups in snake order (ranks 0-3 to groups 0-3, 4-7 to groups 3-0, ...; slot = rank / 4),
    // which keeps the groups' MFMA counts close; each block ORs its act bits into its group's words.
    if (tid < NB) {
        const uint32_t blk = sBlk[tid];
        const int c = __popc(blk);
        int r = 0;
#pragma unroll
        for (int j = 0; j < NB; ++j) {
            const int cj = __popc(sBlk[j]);
            r += (cj > c) || (cj == c && j < tid);
        }
        const int slot = r >> 2, g = (slot & 1) ? 3 - (r & 3) : (r & 3);
        sBase[tid] = g * 128 + slot * 32;
        // word w of row group g: bit 4 t + slot (t in [8 w, 8 w + 8)) = tap t present in the block
#pragma unroll
        for (int w = 0; w < HB_ACT_WORDS; ++w) {
            uint32_t v = (blk >> (8 * w)) & 0xffu;   // the 8 tap bits spread to every fourth bit
            v = (v | (v << 12)) & 0x000F000Fu;
            v = (v | (v << 6)) & 0x03030303u;
            v = (v | (v << 3)) & 0x11111111u;
            if (v) atomicOr(&sAct[g * HB_ACT_WORDS + w], v << slot);
        }
    }
    __syncthreads();
    if (tid < 4 * HB_ACT_WORDS) plan.act[tile * 4 * HB_ACT_WORDS + tid] = sAct[tid];
    sPos[sTid[tid]] = (uint16_t)(sBase[tid >> 5] + (tid & 31));
    __syncthreads();
    int pos[1] = {sPos[tid]};
    plan.vox[tile * HB_M + pos[0]] = (int32_t)i[0];
    __syncthreads();   // sRowOf and the scratch are the planner's from here on

    int H;
    bool direct;
    tile_plan_core<HB_PLAN_NT, 1>(nv, pos, sL, sRowOf, sScratch, sRed, H, direct);
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

}  // namespace

size_t halo_plan_bytes(int64_t n) {
    const int64_t n_tiles = std::max<int64_t>(1, ceil_div(n, HB_M));
    return plan_tile_bytes(n_tiles) + sort_scratch_bytes(n);
}

int halo_plan_build(const int32_t* nbr, const int32_t* coords, int64_t n, void* plan, hipStream_t s) {
    const int64_t n_tiles = ceil_div(n, HB_M);
    if (n_tiles == 0) return TSP_OK;
    const int32_t* order = nullptr;
    if (coords) {
        const SortScratch ss = carve_sort(static_cast<char*>(plan) + plan_tile_bytes(n_tiles), n);
        const int st = morton_order(coords, n, ss, s, &order);
        if (st != TSP_OK) return st;
    }
    hipLaunchKernelGGL(k_plan_build, dim3((unsigned)n_tiles), dim3(HB_PLAN_NT), 0, s, nbr, n, order, n_tiles,
                       carve_plan(plan, n_tiles));
    TSP_CHECK_LAUNCH();
    return TSP_OK;
}

}  // namespace tsp
