// Conv plans (tsp_conv_plan_build, tsp_conv_plan_build_ordered).
//
// A plan splits the output voxels into tiles of HB_M and records, per tile, the input rows its
// table entries reference and the LDS slot of every (tap, voxel) (tile_plan.hpp). Which voxels
// share a tile decides how many rows a tile stages: with coordinates, the plan builds a cell grid
// of the voxels (grid.hpp), lists them in Morton order of their 8^3 cells (then x, y, z inside a
// cell) and each run of HB_M voxels is a tile -- a compact patch of the surface, whose neighbours
// are ~1.7 distinct rows per voxel on thin shells instead of ~3.3 for HB_M consecutive rows of an
// x-major set -- and the tiles read their neighbours from the grid, where a Morton-ordered tile's
// neighbourhood is a few cells, instead of gathering them from the tap-major table. Without
// coordinates, or when the grid does not fit, tiles are consecutive rows. Inside a tile the voxels are
// grouped by which corner taps they have (see k_plan_build). The conv's results do not depend on
// the grouping: every output row sums the same products in the same order wherever it sits (a
// skipped absent tap would only have added exact zeros).
#include <algorithm>

#include "brick_hash.hpp"
#include "grid.hpp"
#include "tile_plan.hpp"

namespace tsp {
namespace {

// ---- Morton order from the cell grid -----------------------------------------------------------
// The cell walk lists the voxels block by block (blocks are numbered in Morton order of their
// cells), each block's voxels in x, y, z order inside the cell; then the voxels that hold no
// block word -- duplicates of a coordinate other than its largest row, and coordinates out of
// range -- in row order. Two launches: counts, then the stores.
constexpr int WK_NT = 256;

__device__ __forceinline__ int wave_sum_i(int v) {
    for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
    return v;
}

// voxel i holds no block word
__device__ __forceinline__ bool left_out(const int32_t* __restrict__ coords, const GridRef& g, int64_t i) {
    const int32_t x = coords[3 * i], y = coords[3 * i + 1], z = coords[3 * i + 2];
    if (!coords_ok(x, y, z)) return true;
    const int32_t blk = grid_block(g, x >> 3, y >> 3, z >> 3);
    return g.blocks[(int64_t)blk * GRID_BLOCK_WORDS + cell_word(x, y, z)] != (int32_t)(i + 1);
}

// coordinates packed 21 bits each (all ones: out of range)
__device__ __forceinline__ uint64_t pack_xyz(int32_t x, int32_t y, int32_t z) {
    return (uint64_t)x | ((uint64_t)y << 21) | ((uint64_t)z << 42);
}

// Workgroup p: the voxel counts of blocks [p bchunk, +bchunk) into counts[] and their sum into
// parts[p]; each block's presence bitmap (byte (x & 7) * 8 + (y & 7) holds the z bits of that
// column) into pres[64 b ..]; the left-out voxels of rows [p vchunk, +vchunk) into
// parts[GRID_PARTS + p]. A wave takes a block, a lane a column.
__global__ __launch_bounds__(WK_NT) void k_walk_count(const int32_t* __restrict__ coords, int64_t n,
                                                      const int32_t* __restrict__ dir, const GridHdr* __restrict__ hdr,
                                                      int32_t* __restrict__ counts, uint8_t* __restrict__ pres,
                                                      int32_t* __restrict__ parts) {
    __shared__ int sW[WK_NT / 64];
    __shared__ int sB[WK_NT / 64];
    if (hdr->mode != GRID_MODE_CELLS) return;
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const GridRef g = grid_ref(dir, hdr);
    const int64_t nb = hdr->nblocks, bchunk = (nb + GRID_PARTS - 1) / GRID_PARTS;
    const int64_t b0 = blockIdx.x * bchunk, b1 = min(nb, b0 + bchunk);
    int bsum = 0;
    for (int64_t b = b0 + wave; b < b1; b += WK_NT / 64) {
        const int32_t* col = g.blocks + b * GRID_BLOCK_WORDS + lane * GRID_COL_WORDS + 1;
        uint32_t byte = 0;
#pragma unroll
        for (int k = 0; k < 8; ++k) byte |= (col[k] != 0 ? 1u : 0u) << k;
        pres[b * 64 + lane] = (uint8_t)byte;
        const int k = wave_sum_i(__popc(byte));
        if (lane == 0) counts[b] = k;
        bsum += k;
    }
    const int64_t vchunk = (n + GRID_PARTS - 1) / GRID_PARTS;
    const int64_t v0 = blockIdx.x * vchunk, v1 = min(n, v0 + vchunk);
    int lc = 0;
    for (int64_t i = v0 + tid; i < v1; i += WK_NT) lc += left_out(coords, g, i);
    lc = wave_sum_i(lc);
    if (lane == 0) { sW[wave] = lc; sB[wave] = bsum; }
    __syncthreads();
    if (tid == 0) {
        int tb = 0, tl = 0;
        for (int w = 0; w < WK_NT / 64; ++w) { tb += sB[w]; tl += sW[w]; }
        parts[blockIdx.x] = tb;
        parts[GRID_PARTS + blockIdx.x] = tl;
    }
}

// The stores of the walk: the row (order) and packed coordinates (wc) of every voxel -- block
// voxels from their block's start, column by column, then the left-out voxels after all block
// voxels. Every workgroup sums the partials before it (and all block partials) itself.
// Workgroups from GRID_PARTS on carry the neighbour-table probe (pj), when asked for: the walk is
// latency-bound and the probe bound by its table stores, so the two share the launch (2-3 % off
// the table + plan call, against the probe as a launch of its own; a third of the probe on the
// count launch instead measured the same).
__global__ __launch_bounds__(WK_NT) void k_walk_emit(const int32_t* __restrict__ coords, int64_t n,
                                                     const int32_t* __restrict__ dir, const GridHdr* __restrict__ hdr,
                                                     const int32_t* __restrict__ counts, const uint8_t* __restrict__ pres,
                                                     const int32_t* __restrict__ cell_of,
                                                     const int32_t* __restrict__ parts, int32_t* __restrict__ order,
                                                     uint64_t* __restrict__ wc, int32_t* __restrict__ list_n,
                                                     ProbeJob pj) {
    __shared__ int sW[WK_NT / 64];
    __shared__ int sS[3][WK_NT / 64];
    __shared__ int sStart[WK_NT];
    if (blockIdx.x >= GRID_PARTS) {
        const int64_t i = pj.v0 + (int64_t)(blockIdx.x - GRID_PARTS) * WK_NT + threadIdx.x;
        if (i < pj.v1) probe_voxel(coords, n, i, dir, hdr, pj.hash, pj.nbr);
        return;
    }
    if (blockIdx.x == 0 && threadIdx.x == 0) *list_n = 0;   // the plan kernels' list of table tiles
    if (hdr->mode != GRID_MODE_CELLS) return;
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const GridRef g = grid_ref(dir, hdr);
    const int64_t nb = hdr->nblocks, bchunk = (nb + GRID_PARTS - 1) / GRID_PARTS;
    const int64_t b0 = blockIdx.x * bchunk, b1 = min(nb, b0 + bchunk);
    int base = 0, placed = 0, lbase = 0;
    {
        constexpr int PPT = GRID_PARTS / WK_NT;
        int bb = 0, ball = 0, lb = 0;
#pragma unroll
        for (int k = 0; k < PPT; ++k) {
            const int p = tid * PPT + k;
            const int vb = parts[p], vl = parts[GRID_PARTS + p];
            ball += vb;
            if (p < (int)blockIdx.x) { bb += vb; lb += vl; }
        }
        bb = wave_sum_i(bb); ball = wave_sum_i(ball); lb = wave_sum_i(lb);
        if (lane == 0) { sS[0][wave] = bb; sS[1][wave] = ball; sS[2][wave] = lb; }
        __syncthreads();
        for (int w = 0; w < WK_NT / 64; ++w) { base += sS[0][w]; placed += sS[1][w]; lbase += sS[2][w]; }
        lbase += placed;
    }
    for (int64_t r0 = b0; r0 < b1; r0 += WK_NT) {
        const int64_t b = r0 + tid;
        int total;
        const int pre = block_exclusive_scan<WK_NT>(b < b1 ? counts[b] : 0, sW, total);
        sStart[tid] = base + pre;
        base += total;
        __syncthreads();
        const int nr = (int)min<int64_t>(WK_NT, b1 - r0);
        for (int j = wave; j < nr; j += WK_NT / 64) {
            const int64_t blk = r0 + j;
            const uint32_t m = (uint32_t)cell_of[blk];
            const int32_t cx = (int32_t)compact3_10(m >> 2) + g.clo[0], cy = (int32_t)compact3_10(m >> 1) + g.clo[1],
                          cz = (int32_t)compact3_10(m) + g.clo[2];
            const uint32_t byte = pres[blk * 64 + lane];
            const int cnt = __popc(byte);
            int x = cnt;   // inclusive scan of the columns' counts
#pragma unroll
            for (int off = 1; off < 64; off <<= 1) {
                const int y = __shfl_up(x, off, 64);
                if (lane >= off) x += y;
            }
            int at = sStart[j] + x - cnt;
            const int32_t* col = g.blocks + blk * GRID_BLOCK_WORDS + lane * GRID_COL_WORDS + 1;
            const int32_t vx = cx * 8 + (lane >> 3), vy = cy * 8 + (lane & 7);
#pragma unroll
            for (int k = 0; k < 8; ++k)
                if ((byte >> k) & 1u) {
                    order[at] = col[k] - 1;
                    wc[at] = pack_xyz(vx, vy, cz * 8 + k);
                    ++at;
                }
        }
        __syncthreads();   // sStart is rewritten by the next round
    }
    const int64_t vchunk = (n + GRID_PARTS - 1) / GRID_PARTS;
    const int64_t v0 = blockIdx.x * vchunk, v1 = min(n, v0 + vchunk);
    for (int64_t r0 = v0; r0 < v1; r0 += WK_NT) {
        const int64_t i = r0 + tid;
        const bool out = i < v1 && left_out(coords, g, i);
        int total;
        const int pre = block_exclusive_scan<WK_NT>(out ? 1 : 0, sW, total);
        if (out) {
            const int32_t x = coords[3 * i], y = coords[3 * i + 1], z = coords[3 * i + 2];
            order[lbase + pre] = (int32_t)i;
            wc[lbase + pre] = coords_ok(x, y, z) ? pack_xyz(x, y, z) : ~0ull;
        }
        lbase += total;
    }
}

struct PlanScratch {
    int32_t* order;
    uint64_t* wc;
    int32_t* counts;
    int32_t* cell_of;
    uint8_t* pres;
    void* tail;
    void* region;
    size_t region_bytes;
};
// the grid may use 32 bytes per voxel + 16 MiB (surface-like sets need ~25-30 bytes per voxel)
size_t grid_region_bytes(int64_t n) { return align256((size_t)n * 32 + ((size_t)16 << 20)); }
}  // namespace

// Blocks the per-block scratch (counts, cell_of: 4 bytes each; presence bitmaps: 64 bytes each)
// holds: every block that fits the larger of the plan's own grid region and the neighbour
// table's workspace (whose grid the planned table build shares), and at least one entry per tile
// (counts is reused as the list of table tiles). A grid with more blocks is not built
// (grid_build's block_cap), so no block index runs past these arrays.
int64_t plan_block_cap(int64_t n) {
    const size_t region = std::max(grid_region_bytes(n), (size_t)table_capacity(n) * kBucketWords * 4);
    return std::max<int64_t>(std::max<int64_t>(ceil_div(n, HB_M), 1),
                             (int64_t)(region / (4 * GRID_BLOCK_WORDS)) + 1);
}

namespace {
size_t plan_scratch_bytes(int64_t n) {
    const size_t n1 = (size_t)std::max<int64_t>(n, 1), cap = (size_t)plan_block_cap(n);
    return align256(n1 * 4) + align256(n1 * 8) + 2 * align256(cap * 4) + align256(cap * 64) +
           GRID_TAIL + grid_region_bytes(n);
}
PlanScratch carve_scratch(void* p, int64_t n) {
    const size_t n1 = (size_t)std::max<int64_t>(n, 1), cap = (size_t)plan_block_cap(n);
    char* c = static_cast<char*>(p);
    PlanScratch s;
    s.order = reinterpret_cast<int32_t*>(c);
    c += align256(n1 * 4);
    s.wc = reinterpret_cast<uint64_t*>(c);
    c += align256(n1 * 8);
    s.counts = reinterpret_cast<int32_t*>(c);
    c += align256(cap * 4);
    s.cell_of = reinterpret_cast<int32_t*>(c);
    c += align256(cap * 4);
    s.pres = reinterpret_cast<uint8_t*>(c);
    c += align256(cap * 64);
    s.tail = c;
    c += GRID_TAIL;
    s.region = c;
    s.region_bytes = grid_region_bytes(n);
    return s;
}

// ---- the plan of one tile per workgroup (HB_PLAN_NT threads, one voxel each) ------------------------
// Positions inside the tile: the voxels grouped by which of the 8 corner taps they have (a stable
// counting sort of 9-bit digits in LDS: voxels with the same corners mostly share their other
// taps too, so a tap is often absent from all 32 rows of an MFMA block and costs no MFMA there);
// then the 16 blocks are dealt to the 4 row groups (one per SIMD) so that the groups' MFMA counts
// stay close.
//
// Distinct rows and slots, two kernels:
//   * k_plan_window (cell grid, the tile's voxels within a box of at most WIN_COLS columns of
//     <= 64 voxels in z, with a voxel of margin): a bitmap over the box, one 64-bit word of z bits
//     per (x, y) column. The tile's voxels are marked (one LDS OR each), dilated by one voxel along
//     every axis with word shifts and ORs of the neighbouring columns, and ANDed with the grid's
//     presence bits: the set bits are exactly the distinct rows the tile's taps reference. Their
//     ranks in (x, y, z) order are the slots -- row order for coordinate-sorted sets -- and a
//     voxel's 27 taps are 9 column reads (3 z bits each). No table entries are read; the box's
//     cells are looked up once (a block number per cell in LDS). Its LDS (~42 KiB) lets three
//     workgroups share a CU, which hides the grid reads' latency.
//   * k_plan_table (no grid, or the tiles k_plan_window listed as spread too wide): the table's 27
//     entries of each voxel, ranked by tile_plan_core.
// With a grid tile q holds voxels order[512 q ..] of the cell walk (their coordinates in
// wc[512 q ..]); otherwise rows 512 q ...
constexpr int WIN_COLS = 1280;     // columns of a window
constexpr int WIN_CELLS = 1536;    // cells of a window's box
constexpr int WIN_SEGS = 4;        // windows a tile may take
constexpr int PL_NB = HB_M / 32;   // MFMA row blocks of a tile
constexpr int PL_NW = HB_PLAN_NT / 64;
constexpr int PL_ND = 257;         // digits: corner sets 0..255, 256 = no voxel
constexpr int PL_ORDER_WORDS = PL_NW * PL_ND + PL_ND + 64 + HB_M + HB_M / 2 + HB_M / 2;

// Exclusive scan of the popcounts of the 64-bit words[0..nw) (nw <= WIN_COLS) into pre[];
// returns the total. sRed: NT / 64 ints.
template <int NT>
__device__ int scan_popcounts64(const uint64_t* words, int nw, int32_t* pre, int* sRed) {
    constexpr int CPT = (WIN_COLS + NT - 1) / NT;
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    int cnt[CPT], mine = 0;
#pragma unroll
    for (int k = 0; k < CPT; ++k) {
        const int c = tid * CPT + k;
        cnt[k] = c < nw ? __popcll(words[c]) : 0;
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
    for (int k = 0; k < CPT; ++k) {
        const int c = tid * CPT + k;
        if (c < nw) pre[c] = base;
        base += cnt[k];
    }
    __syncthreads();
    return total;
}

// The tile's positions (see above) from each voxel's 27-bit tap set; writes the tile's act words
// and its vox record and returns this thread's position. `lds`: PL_ORDER_WORDS words; sBlk, sBase,
// sAct: PL_NB, PL_NB, 4 HB_ACT_WORDS. Every thread calls it.
__device__ int tile_positions(uint32_t taps, int64_t i, int64_t tile, uint32_t* lds, uint32_t* sBlk, int* sBase,
                              uint32_t* sAct, PlanView plan) {
    constexpr int NW = PL_NW, ND = PL_ND, NB = PL_NB;
    int* sCnt = reinterpret_cast<int*>(lds);                  // [NW][ND]: count, then first rank
    int* sDig = sCnt + NW * ND;                               // [ND]: first sorted index of a digit
    int* sWsum = sDig + ND;                                   // scan of the digit totals
    uint32_t* sTaps = reinterpret_cast<uint32_t*>(sWsum + 64);   // taps of each sorted index
    uint16_t* sTid = reinterpret_cast<uint16_t*>(sTaps + HB_M);  // thread of each sorted index
    uint16_t* sPos = sTid + HB_M;                                // position of each thread
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    constexpr int kCorner[8] = {0, 2, 6, 8, 18, 20, 24, 26};   // taps (+-1, +-1, +-1)
    int d = 0;
#pragma unroll
    for (int k = 0; k < 8; ++k) d |= ((taps >> kCorner[k]) & 1u) << k;
    if (i < 0) d = ND - 1;                        // empty positions sort last
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
    int xs = tot;
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
        const int yv = __shfl_up(xs, off, 64);
        if (lane >= off) xs += yv;
    }
    if (lane == 63) sWsum[wave] = xs;
    __syncthreads();
    if (tid < ND) {
        int before = 0;
        for (int w = 0; w < wave; ++w) before += sWsum[w];
        sDig[tid] = before + xs - tot;
    }
    __syncthreads();
    const int sidx = sDig[d] + sCnt[wave * ND + d] + rank;   // this voxel's sorted index
    sTaps[sidx] = i >= 0 ? taps : 0u;
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
        const int slot = r >> 2, grp = (slot & 1) ? 3 - (r & 3) : (r & 3);
        sBase[tid] = grp * 128 + slot * 32;
        // word w of row group grp: bit 4 t + slot (t in [8 w, 8 w + 8)) = tap t present in the block
#pragma unroll
        for (int w = 0; w < HB_ACT_WORDS; ++w) {
            uint32_t v = (blk >> (8 * w)) & 0xffu;   // the 8 tap bits spread to every fourth bit
            v = (v | (v << 12)) & 0x000F000Fu;
            v = (v | (v << 6)) & 0x03030303u;
            v = (v | (v << 3)) & 0x11111111u;
            if (v) atomicOr(&sAct[grp * HB_ACT_WORDS + w], v << slot);
        }
    }
    __syncthreads();
    if (tid < 4 * HB_ACT_WORDS) plan.act[tile * 4 * HB_ACT_WORDS + tid] = sAct[tid];
    sPos[sTid[tid]] = (uint16_t)(sBase[tid >> 5] + (tid & 31));
    __syncthreads();
    const int pos = sPos[tid];
    plan.vox[tile * HB_M + pos] = (int32_t)i;
    __syncthreads();   // the LDS is the caller's again
    return pos;
}

// Tiles of the cell walk, in windows; tiles of more than WIN_SEGS windows are appended to list
// (count in *list_n) for k_plan_table, and every tile is when the grid fell back.
// (three workgroups a CU, as their LDS allows: at most 80 registers)
__global__ __launch_bounds__(HB_PLAN_NT) __attribute__((amdgpu_waves_per_eu(6))) void k_plan_window(int64_t n, const int32_t* __restrict__ order,
                                                            const uint64_t* __restrict__ wc,
                                                            const int32_t* __restrict__ dir,
                                                            const uint8_t* __restrict__ pres,
                                                            const GridHdr* __restrict__ hdr, PlanView plan,
                                                            int32_t* __restrict__ list, int32_t* __restrict__ list_n) {
    static_assert(HB_PLAN_NT == HB_M, "one thread per tile position");
    static_assert(2 * 2 * WIN_COLS >= PL_ORDER_WORDS, "the order step's records fit the dead bitmaps");
    constexpr int NW = PL_NW;
    __shared__ __attribute__((aligned(16))) uint64_t sA[2 * WIN_COLS];   // wT, wPres; then the order step
    __shared__ __attribute__((aligned(16))) uint64_t wP[WIN_COLS];       // referenced and present
    __shared__ int32_t wPre[WIN_COLS];                                    // slot of a column's first bit
    __shared__ int32_t wCell[WIN_CELLS];                                  // block of each cell of the box
    __shared__ int sRed[2 * NW];
    __shared__ int sBox[6][NW];
    __shared__ int sSeg[6];
    __shared__ int sEnd;
    __shared__ uint32_t sBlk[PL_NB];
    __shared__ int sBase[PL_NB];
    __shared__ uint32_t sAct[4 * HB_ACT_WORDS];
    uint64_t* wT = sA;
    uint64_t* wPres = sA + WIN_COLS;

    const int64_t tile = blockIdx.x;
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    if (hdr->mode != GRID_MODE_CELLS) {
        if (tid == 0) list[atomicAdd(list_n, 1)] = (int32_t)tile;
        return;
    }
    const int64_t q = tile * HB_M + tid;
    const int64_t i = q < n ? (int64_t)order[q] : -1;
    const GridRef g = grid_ref(dir, hdr);
    int32_t x = 0, y = 0, z = 0;
    bool valid = false;
    if (i >= 0) {
        const uint64_t p = wc[q];
        x = (int32_t)(p & 0x1fffff); y = (int32_t)((p >> 21) & 0x1fffff); z = (int32_t)((p >> 42) & 0x1fffff);
        valid = coords_ok(x, y, z);
    }
    // The tile's voxels (walk order) in segments: runs whose box fits a window, found with a prefix
    // box over the positions. Each segment's window ranks its own dilated set; the slots of later
    // segments follow those of earlier ones (a row two segments reference gets a slot in each,
    // which only stages it twice). A tile of more than WIN_SEGS segments goes to k_plan_table.
    uint32_t taps = 0;
    // the voxel's 27 slots, two 16-bit slots a register (tap 2 k low, 2 k + 1 high)
    uint32_t wsl[(kTaps + 1) / 2];
#pragma unroll
    for (int k = 0; k < (kTaps + 1) / 2; ++k) wsl[k] = HB_ZERO | (HB_ZERO << 16);
    auto set_slot = [&](int t, int v) {
        wsl[t >> 1] = (t & 1) ? ((wsl[t >> 1] & 0xffffu) | ((uint32_t)v << 16)) : ((wsl[t >> 1] & 0xffff0000u) | (uint32_t)v);
    };
    int H = 0, seg0 = 0, nseg = 0;
    while (seg0 < HB_M) {
        // inclusive prefix box over positions seg0 .. tid (lo xyz by min, hi xyz by max)
        const bool in = valid && tid >= seg0;
        int b[6] = {in ? x : INT32_MAX, in ? y : INT32_MAX, in ? z : INT32_MAX, in ? x : -1, in ? y : -1, in ? z : -1};
#pragma unroll
        for (int off = 1; off < 64; off <<= 1) {
#pragma unroll
            for (int a = 0; a < 6; ++a) {
                const int u = __shfl_up(b[a], off, 64);
                if (lane >= off) b[a] = a < 3 ? min(b[a], u) : max(b[a], u);
            }
        }
        if (lane == 63) {
#pragma unroll
            for (int a = 0; a < 6; ++a) sBox[a][wave] = b[a];
        }
        if (tid == 0) sEnd = HB_M;
        __syncthreads();
        for (int w = 0; w < wave; ++w) {
#pragma unroll
            for (int a = 0; a < 6; ++a) b[a] = a < 3 ? min(b[a], sBox[a][w]) : max(b[a], sBox[a][w]);
        }
        // the segment ends at the first position whose prefix box does not fit
        bool fits = true;
        if (b[3] >= 0) {
            const int64_t WX = (int64_t)b[3] - b[0] + 3, WYl = (int64_t)b[4] - b[1] + 3, WZ = (int64_t)b[5] - b[2] + 3;
            const int64_t CX = ((b[3] + 1) >> 3) - ((b[0] - 1) >> 3) + 1, CYl = ((b[4] + 1) >> 3) - ((b[1] - 1) >> 3) + 1,
                          CZl = ((b[5] + 1) >> 3) - ((b[2] - 1) >> 3) + 1;
            fits = WZ <= 64 && WX * WYl <= WIN_COLS && CX * CYl * CZl <= WIN_CELLS;
        }
        const uint64_t bad = __ballot(tid >= seg0 && !fits);
        if (lane == 0 && bad) atomicMin(&sEnd, wave * 64 + (int)__builtin_ctzll(bad));
        __syncthreads();
        const int end = sEnd;   // > seg0: a box of one voxel always fits
        if (tid == end - 1) {
#pragma unroll
            for (int a = 0; a < 6; ++a) sSeg[a] = b[a];
        }
        __syncthreads();
        int sb[6];
#pragma unroll
        for (int a = 0; a < 6; ++a) sb[a] = sSeg[a];
        const bool member = valid && tid >= seg0 && tid < end;
        if (sb[3] >= 0) {
            const int wx0 = sb[0] - 1, wy0 = sb[1] - 1, wz0 = sb[2] - 1;
            const int WX = sb[3] - sb[0] + 3, WY = sb[4] - sb[1] + 3, WZ = sb[5] - sb[2] + 3;
            const int ox = wx0 >> 3, oy = wy0 >> 3, oz = wz0 >> 3;
            const int CY = ((wy0 + WY - 1) >> 3) - oy + 1, CZ = ((wz0 + WZ - 1) >> 3) - oz + 1;
            const int ncol = WX * WY, ncell = (((wx0 + WX - 1) >> 3) - ox + 1) * CY * CZ;
            // the block of every cell of the box
            for (int k = tid; k < ncell; k += HB_PLAN_NT)
                wCell[k] = grid_block(g, ox + k / (CY * CZ), oy + (k / CZ) % CY, oz + k % CZ);
            __syncthreads();
            // presence words of the columns, from the blocks' presence bytes
            const uint64_t zmask = WZ == 64 ? ~0ull : ((1ull << WZ) - 1ull);
            for (int c = tid; c < ncol; c += HB_PLAN_NT) {
                const int cx = wx0 + c / WY, cy = wy0 + c % WY;
                const int32_t* cc = wCell + ((cx >> 3) - ox) * CY * CZ + ((cy >> 3) - oy) * CZ;
                const int po = (cx & 7) * 8 + (cy & 7);
                uint64_t word = 0;
#pragma unroll
                for (int k = 0; k < 9; ++k) {
                    if (k >= CZ) break;
                    const int32_t blk = cc[k];
                    const uint64_t byte = blk >= 0 ? pres[(int64_t)blk * 64 + po] : 0u;
                    const int sh = (oz + k) * 8 - wz0;
                    word |= sh >= 0 ? byte << sh : byte >> -sh;
                }
                wPres[c] = word & zmask;
                wT[c] = 0ull;
            }
            __syncthreads();
            if (member)
                atomicOr(reinterpret_cast<unsigned long long*>(&wT[(x - wx0) * WY + (y - wy0)]), 1ull << (z - wz0));
            __syncthreads();
            // dilate by one voxel, keep the present ones
            for (int c = tid; c < ncol; c += HB_PLAN_NT) {
                const int cx = c / WY, cy = c % WY;
                uint64_t d = 0;
#pragma unroll
                for (int dx = -1; dx <= 1; ++dx)
#pragma unroll
                    for (int dy = -1; dy <= 1; ++dy) {
                        const int ax = cx + dx, ay = cy + dy;
                        if (ax < 0 || ay < 0 || ax >= WX || ay >= WY) continue;
                        const uint64_t t = wT[ax * WY + ay];
                        d |= t | (t << 1) | (t >> 1);
                    }
                wP[c] = d & wPres[c];
            }
            __syncthreads();
            const int Hs = scan_popcounts64<HB_PLAN_NT>(wP, ncol, wPre, sRed);
            // the row of every slot H + s of the segment: column = the last one whose first slot is
            // <= s, then the (s - first)-th set bit of its word
            int32_t* ro = plan.rowof + tile * HB_SLOTS;
            for (int sl = tid; sl < Hs && H + sl < HB_SLOTS; sl += HB_PLAN_NT) {
                int lo = 0, hi = ncol - 1;
                while (lo < hi) {
                    const int mid = (lo + hi + 1) >> 1;
                    if (wPre[mid] <= sl) lo = mid; else hi = mid - 1;
                }
                uint64_t bits = wP[lo];
                for (int k = sl - wPre[lo]; k > 0; --k) bits &= bits - 1ull;
                const int cx = wx0 + lo / WY, cy = wy0 + lo % WY, cz = wz0 + __builtin_ctzll(bits);
                const int32_t blk = wCell[((cx >> 3) - ox) * CY * CZ + ((cy >> 3) - oy) * CZ + ((cz >> 3) - oz)];
                ro[H + sl] = g.blocks[(int64_t)blk * GRID_BLOCK_WORDS + cell_word(cx, cy, cz)] - 1;
            }
            // taps and slots of the segment's voxels: 3 z bits of each of the 9 neighbouring columns
            if (member) {
                const int zz = z - wz0;   // in [1, WZ - 2]
#pragma unroll
                for (int dx = 0; dx < 3; ++dx)
#pragma unroll
                    for (int dy = 0; dy < 3; ++dy) {
                        const int c = (x - wx0 + dx - 1) * WY + (y - wy0 + dy - 1);
                        const uint64_t w = wP[c];
                        const uint32_t b3 = (uint32_t)(w >> (zz - 1)) & 7u;
                        const int base = H + wPre[c] + __popcll(w & ((1ull << (zz - 1)) - 1ull));
                        const int t0 = dx * 9 + dy * 3;
                        taps |= b3 << t0;
                        const int b0 = b3 & 1u, b1 = (b3 >> 1) & 1u;
                        if (b3 & 1u) set_slot(t0, base);
                        if (b3 & 2u) set_slot(t0 + 1, base + b0);
                        if (b3 & 4u) set_slot(t0 + 2, base + b0 + b1);
                    }
            }
            H += Hs;
            __syncthreads();   // the window's arrays are the next segment's
        }
        seg0 = end;
        if (++nseg == WIN_SEGS && seg0 < HB_M) {
            if (tid == 0) list[atomicAdd(list_n, 1)] = (int32_t)tile;
            return;
        }
    }
    const bool direct = H > HB_ZERO;
    __syncthreads();   // the bitmaps are dead: sA is the order step's
    const int pos = tile_positions(taps, i, tile, reinterpret_cast<uint32_t*>(sA), sBlk, sBase, sAct, plan);
    if (tid == 0) {
        int32_t* h = plan.hdr + tile * 4;
        h[0] = H; h[1] = direct ? 1 : 0; h[2] = 0; h[3] = 0;
    }
    if (direct) return;
    // slot table [tap][position / 128][position % 32][position / 32 % 4], straight to memory
    uint16_t* sl = plan.slots + tile * HB_SLOT_TABLE + (pos >> 7) * 128 + (pos & 31) * 4 + ((pos >> 5) & 3);
#pragma unroll
    for (int t = 0; t < kTaps; ++t) sl[t * HB_M] = (uint16_t)(wsl[t >> 1] >> (16 * (t & 1)));
}

// Tiles ranked from the table's entries: tiles list[0 .. *list_n) (cell walk order when the grid is
// in cell mode), or, without a list, tiles 0 .. n_tiles of consecutive rows. A workgroup takes
// tiles blockIdx.x, + gridDim.x, ...
// (two workgroups a CU, as their LDS allows: at most 128 registers)
__global__ __launch_bounds__(HB_PLAN_NT) __attribute__((amdgpu_waves_per_eu(4))) void k_plan_table(const int32_t* __restrict__ nbr, int64_t n,
                                                           const int32_t* __restrict__ order,
                                                           const GridHdr* __restrict__ hdr,
                                                           const int32_t* __restrict__ list,
                                                           const int32_t* __restrict__ list_n, int64_t n_tiles,
                                                           PlanView plan) {
    static_assert(HB_PLAN_SCRATCH >= PL_ORDER_WORDS, "the order step fits the scratch");
    __shared__ __attribute__((aligned(16))) uint16_t sL[kTaps][4][32][4];
    __shared__ __attribute__((aligned(16))) int32_t sRowOf[HB_SLOTS];
    __shared__ __attribute__((aligned(16))) uint32_t sScratch[HB_PLAN_SCRATCH];
    __shared__ int sRed[2 * PL_NW];
    __shared__ uint32_t sBlk[PL_NB];
    __shared__ int sBase[PL_NB];
    __shared__ uint32_t sAct[4 * HB_ACT_WORDS];
    const int tid = threadIdx.x;
    const bool walk = order != nullptr && hdr->mode == GRID_MODE_CELLS;
    const int64_t count = list ? (int64_t)*list_n : n_tiles;
    for (int64_t k = blockIdx.x; k < count; k += gridDim.x) {
        const int64_t tile = list ? (int64_t)list[k] : k;
        const int64_t q = tile * HB_M + tid;
        int64_t i[1] = {q < n ? (walk ? (int64_t)order[q] : q) : -1};
        int32_t nv[kTaps][1];
        load_entries<1>(nbr, n, i, nv);
        uint32_t taps = 0;
#pragma unroll
        for (int t = 0; t < kTaps; ++t) taps |= (nv[t][0] >= 0 ? 1u : 0u) << t;
        int pos[1] = {tile_positions(taps, i[0], tile, sScratch, sBlk, sBase, sAct, plan)};
        int H;
        bool direct;
        tile_plan_core<HB_PLAN_NT, 1>(nv, pos, sL, sRowOf, sScratch, sRed, H, direct);
        if (tid == 0) {
            int32_t* h = plan.hdr + tile * 4;
            h[0] = H; h[1] = direct ? 1 : 0; h[2] = 0; h[3] = 0;
        }
        if (!direct) {
            int32_t* ro = plan.rowof + tile * HB_SLOTS;
            for (int s = tid; s < H; s += HB_PLAN_NT) ro[s] = sRowOf[s];
            const u32x4_t* src = reinterpret_cast<const u32x4_t*>(&sL[0][0][0][0]);
            u32x4_t* dst = reinterpret_cast<u32x4_t*>(plan.slots + tile * HB_SLOT_TABLE);
            for (int p = tid; p < HB_SLOT_TABLE / 8; p += HB_PLAN_NT) dst[p] = src[p];
        }
        __syncthreads();   // the LDS is the next tile's
    }
}

}  // namespace

size_t halo_plan_bytes(int64_t n) {
    const int64_t n_tiles = std::max<int64_t>(1, ceil_div(n, HB_M));
    return plan_tile_bytes(n_tiles) + plan_scratch_bytes(n);
}

// The cell walk and the tiles on a grid built from coords (dir = its region, tail = its tail).
static int plan_on_grid(const int32_t* nbr, const int32_t* coords, int64_t n, void* plan, const int32_t* dir,
                        void* tail, hipStream_t s, const ProbeJob* probe) {
    const int64_t n_tiles = ceil_div(n, HB_M);
    const PlanScratch ps = carve_scratch(static_cast<char*>(plan) + plan_tile_bytes(n_tiles), n);
    const GridTail gt = carve_grid_tail(tail);
    int32_t* list_n = gt.parts + 5 * GRID_PARTS;   // zeroed by k_walk_emit
    int32_t* list = ps.counts;                     // free once k_walk_emit has read the counts
    const PlanView pv = carve_plan(plan, n_tiles);
    // the table probe, when asked for, rides on the walk's emit launch
    ProbeJob pj;
    int64_t ge = GRID_PARTS;
    if (probe && probe->nbr) {
        pj = *probe;
        pj.v0 = 0;
        pj.v1 = n;
        ge += ceil_div(n, WK_NT);
    }
    hipLaunchKernelGGL(k_walk_count, dim3(GRID_PARTS), dim3(WK_NT), 0, s, coords, n, dir, gt.hdr, ps.counts,
                       ps.pres, gt.parts);
    TSP_CHECK_LAUNCH();
    hipLaunchKernelGGL(k_walk_emit, dim3((unsigned)ge), dim3(WK_NT), 0, s, coords, n, dir, gt.hdr, ps.counts,
                       ps.pres, ps.cell_of, gt.parts, ps.order, ps.wc, list_n, pj);
    TSP_CHECK_LAUNCH();
    hipLaunchKernelGGL(k_plan_window, dim3((unsigned)n_tiles), dim3(HB_PLAN_NT), 0, s, n, ps.order, ps.wc, dir,
                       ps.pres, gt.hdr, pv, list, list_n);
    TSP_CHECK_LAUNCH();
    const unsigned grid = (unsigned)std::min<int64_t>(n_tiles, 512);
    hipLaunchKernelGGL(k_plan_table, dim3(grid), dim3(HB_PLAN_NT), 0, s, nbr, n, ps.order, gt.hdr, list, list_n,
                       n_tiles, pv);
    TSP_CHECK_LAUNCH();
    return TSP_OK;
}

// With coordinates: the cell grid (in the plan's scratch), the cell walk, then the tiles (which
// fall back to row tiles and the table on the device when the grid did not fit its space).
int halo_plan_build(const int32_t* nbr, const int32_t* coords, int64_t n, void* plan, hipStream_t s) {
    const int64_t n_tiles = ceil_div(n, HB_M);
    if (n_tiles == 0) return TSP_OK;
    if (coords) {
        const PlanScratch ps = carve_scratch(static_cast<char*>(plan) + plan_tile_bytes(n_tiles), n);
        const int st = grid_build(coords, n, ps.region, ps.region_bytes, ps.tail, nullptr, HashView{nullptr, 0},
                                  ps.cell_of, plan_block_cap(n), s);
        if (st != TSP_OK) return st;
        return plan_on_grid(nbr, coords, n, plan, static_cast<const int32_t*>(ps.region), ps.tail, s, nullptr);
    }
    hipLaunchKernelGGL(k_plan_table, dim3((unsigned)n_tiles), dim3(HB_PLAN_NT), 0, s, nbr, n, nullptr, nullptr,
                       nullptr, nullptr, n_tiles, carve_plan(plan, n_tiles));
    TSP_CHECK_LAUNCH();
    return TSP_OK;
}

int32_t* plan_cell_of(void* plan, int64_t n) {
    return carve_scratch(static_cast<char*>(plan) + plan_tile_bytes(std::max<int64_t>(1, ceil_div(n, HB_M))), n).cell_of;
}

int halo_plan_build_on_grid(const int32_t* nbr, const int32_t* coords, int64_t n, void* plan,
                            const void* region, void* tail, hipStream_t s, const ProbeJob* probe) {
    if (n == 0) return TSP_OK;
    return plan_on_grid(nbr, coords, n, plan, static_cast<const int32_t*>(region), tail, s, probe);
}

}  // namespace tsp
