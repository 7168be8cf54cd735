// Cell grid: the map from voxel coordinates to rows used by the neighbour-table and plan builds
// when the voxels' bounding box is compact (surfaces, bands, dense blocks).
//
// Space is cut into cells of 8^3 voxels. A directory, indexed by the Morton code of a cell
// relative to the bounding box's first cell, holds for each occupied cell the index of its block
// (+1, 0 = empty); blocks are numbered in Morton order of their cells. A block holds the cell's
// 64 (x, y) columns, column (x & 7) * 8 + (y & 7) as 10 words: the voxel below the cell (the
// z-neighbouring cell's top voxel), the cell's 8 voxels, the voxel above. A word holds row + 1
// (0 = absent; the largest row for duplicated coordinates, as the reference's map keeps the last
// insert). With the two halo words a voxel's three z-neighbours in any column are three
// consecutive words of one block, read together. A cell directly above or below an occupied
// cell's top or bottom voxel gets a block (holding only halo words if it has no voxel), so that
// the halo word has somewhere to live.
//
// The build runs on the device without a host round trip; when the directory or the blocks would
// not fit the space the caller gave (scattered or far-flung voxels), the header's mode says so
// and the caller's other path runs instead (kernels of both paths are launched; each returns
// at once when the mode is not its own).
#pragma once
#include "common.hpp"

namespace tsp {

constexpr int32_t kCoordMax = (1 << 21) - 3;   // voxel coordinates in [0, kCoordMax]
constexpr int GRID_PARTS = 1024;               // workgroups of the grid's scans
constexpr int GRID_MAX_BITS = 10;              // directory of at most 2^30 cells
constexpr size_t GRID_TAIL = 32768;            // bytes: header + GRID_PARTS * 7 partials
constexpr int GRID_MODE_CELLS = 0, GRID_MODE_FALLBACK = 1;

struct GridHdr {
    int32_t mode;           // GRID_MODE_CELLS or GRID_MODE_FALLBACK
    int32_t bits;           // Morton bits per axis of the directory
    int32_t clo[3];         // first cell of the bounding box
    int32_t nblocks;        // occupied cells
    int32_t ascending;      // rows strictly ascending in (x, y, z): no coordinate repeats
    int32_t pad1;
    int64_t dir_n;          // directory words: 8^bits
    int64_t blocks_off;     // words from the directory to the first block
    int64_t region_words;   // words available for directory + blocks
};
static_assert(sizeof(GridHdr) <= 256, "header fits its slot");

// The tail (GRID_TAIL bytes, 16-byte aligned): the header, then int32 partials [7 GRID_PARTS]
// (the bounding-box pass's 6 per workgroup, then its ascending flags).
struct GridTail {
    GridHdr* hdr;
    int32_t* parts;
};
inline GridTail carve_grid_tail(void* p) {
    char* c = static_cast<char*>(p);
    return GridTail{reinterpret_cast<GridHdr*>(c), reinterpret_cast<int32_t*>(c + 256)};
}
static_assert(256 + 4 * 7 * GRID_PARTS <= GRID_TAIL, "tail layout");

// Exclusive scan of one value per thread over a workgroup of NT threads; total = the sum.
// sW: NT / 64 ints of LDS. Every thread must call it.
template <int NT>
__device__ __forceinline__ int block_exclusive_scan(int v, int* sW, int& total) {
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    int x = v;
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
        const int y = __shfl_up(x, off, 64);
        if (lane >= off) x += y;
    }
    __syncthreads();
    if (lane == 63) sW[wave] = x;
    __syncthreads();
    int before = 0;
    total = 0;
#pragma unroll
    for (int w = 0; w < NT / 64; ++w) {
        if (w < wave) before += sW[w];
        total += sW[w];
    }
    return before + x - v;
}

__device__ __forceinline__ bool coords_ok(int32_t x, int32_t y, int32_t z) {
    return x >= 0 && y >= 0 && z >= 0 && x <= kCoordMax && y <= kCoordMax && z <= kCoordMax;
}

// bits 0..9 of v moved to bits 0, 3, 6, ..., 27
__device__ __forceinline__ uint32_t spread3_10(uint32_t v) {
    uint32_t r = 0;
#pragma unroll
    for (int b = 0; b < GRID_MAX_BITS; ++b) r |= ((v >> b) & 1u) << (3 * b);
    return r;
}
// Morton code of relative cell (cx, cy, cz), x most significant
__device__ __forceinline__ uint32_t cell_morton(uint32_t cx, uint32_t cy, uint32_t cz) {
    return (spread3_10(cx) << 2) | (spread3_10(cy) << 1) | spread3_10(cz);
}
constexpr int GRID_COL_WORDS = 10;                     // words of a block column
constexpr int GRID_BLOCK_WORDS = 64 * GRID_COL_WORDS;  // words of a block
// word of voxel (x, y, z) in its own cell's block
__device__ __forceinline__ int cell_word(int32_t x, int32_t y, int32_t z) {
    return ((x & 7) * 8 + (y & 7)) * GRID_COL_WORDS + (z & 7) + 1;
}
// bits 0, 3, 6, ..., 27 of v gathered into bits 0..9
__device__ __forceinline__ uint32_t compact3_10(uint32_t v) {
    uint32_t r = 0;
#pragma unroll
    for (int b = 0; b < GRID_MAX_BITS; ++b) r |= ((v >> (3 * b)) & 1u) << b;
    return r;
}

// A read-only view of a built grid.
struct GridRef {
    const int32_t* dir;
    const int32_t* blocks;
    int32_t clo[3];
    uint32_t lim;           // cells per axis: 2^bits
    int32_t bits;
};
__device__ __forceinline__ GridRef grid_ref(const int32_t* dir, const GridHdr* h) {
    GridRef g;
    g.dir = dir;
    g.blocks = dir + h->blocks_off;
    g.clo[0] = h->clo[0]; g.clo[1] = h->clo[1]; g.clo[2] = h->clo[2];
    g.bits = h->bits;
    g.lim = 1u << h->bits;
    return g;
}
// Block of the cell with absolute cell coordinates (cx, cy, cz), -1 when none.
__device__ __forceinline__ int32_t grid_block(const GridRef& g, int32_t cx, int32_t cy, int32_t cz) {
    const uint32_t rx = (uint32_t)(cx - g.clo[0]), ry = (uint32_t)(cy - g.clo[1]),
                   rz = (uint32_t)(cz - g.clo[2]);
    if (rx >= g.lim || ry >= g.lim || rz >= g.lim) return -1;
    return g.dir[cell_morton(rx, ry, rz)] - 1;
}

// The 27 neighbours of voxel (x, y, z) (valid coordinates), tap t = 9 (dx + 1) + 3 (dy + 1) +
// (dz + 1): word[t] = row + 1, 0 when absent. The neighbourhood's columns lie in at most 2 x 2
// cells of the voxel's z-layer of cells, so 4 directory reads and 9 three-word reads serve it.
__device__ __forceinline__ void grid_neighbours(const GridRef& g, int32_t x, int32_t y, int32_t z,
                                                int32_t (&word)[kTaps]) {
    const int32_t cx0 = (x - 1) >> 3, cy0 = (y - 1) >> 3, cx1 = (x + 1) >> 3, cy1 = (y + 1) >> 3;
    const int32_t cz = z >> 3;
    const int32_t b00 = grid_block(g, cx0, cy0, cz), b10 = grid_block(g, cx1, cy0, cz);
    const int32_t b01 = grid_block(g, cx0, cy1, cz), b11 = grid_block(g, cx1, cy1, cz);
    // offset d of an axis lies in the upper of its two cells: h[d + 1] (never for d = -1); the
    // block of a column is picked with selects, so that the four stay in registers
    const bool hx[3] = {false, (x >> 3) != cx0, ((x + 1) >> 3) != cx0};
    const bool hy[3] = {false, (y >> 3) != cy0, ((y + 1) >> 3) != cy0};
    const int pz = z & 7;   // the three words start at the word below the voxel's own
#pragma unroll
    for (int dx = 0; dx < 3; ++dx)
#pragma unroll
        for (int dy = 0; dy < 3; ++dy) {
            const int32_t b = hy[dy] ? (hx[dx] ? b11 : b01) : (hx[dx] ? b10 : b00);
            const int32_t nx = x + dx - 1, ny = y + dy - 1;
            const int t = dx * 9 + dy * 3;
            if (b >= 0) {
                const int32_t* w = g.blocks + (int64_t)b * GRID_BLOCK_WORDS + ((nx & 7) * 8 + (ny & 7)) * GRID_COL_WORDS + pz;
                word[t] = w[0]; word[t + 1] = w[1]; word[t + 2] = w[2];
            } else {
                word[t] = word[t + 1] = word[t + 2] = 0;
            }
        }
}

// The brick hash (brick_hash.hpp) that stands in for the grid when it does not fit: cap buckets
// of 16 words -- rows of octants 0..7 (8 words), key (2 words), unused. cap = 0: none.
struct HashView {
    uint32_t* words;
    uint64_t cap;
};

// Builds the grid of coords[0..n) in `region` (region_bytes, 16-byte aligned) with header and
// partials in `tail` (GRID_TAIL bytes), or, when it does not fit and a hash is given (its
// buckets are `region`), the hash. Coordinates outside [0, kCoordMax] are left out and set bit 0
// of *status when status is given. Returns a tsp_status of the launches.
// cell_of (optional, one int per block): each block's directory index (its cell's Morton code).
// block_cap: the most blocks the caller's per-block arrays (cell_of and the like) hold; a grid
// with more blocks is not built (the mode says fallback), as when the region is too small.
int grid_build(const int32_t* coords, int64_t n, void* region, size_t region_bytes, void* tail,
               int32_t* status, HashView hash, int32_t* cell_of, int64_t block_cap, hipStream_t s);

}  // namespace tsp
