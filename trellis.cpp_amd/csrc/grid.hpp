// Cell grid: the map from voxel coordinates to rows used by the neighbour-table and plan builds
// when the voxels' bounding box is compact (surfaces, bands, dense blocks).
//
// Space is cut into cells of 8^3 voxels. A directory, indexed by the Morton code of a cell
// relative to the bounding box's first cell, holds for each occupied cell the index of its block
// (+1, 0 = empty); blocks are numbered in Morton order of their cells. A block is 512 words, one
// per voxel of the cell at (x & 7) << 6 | (y & 7) << 3 | (z & 7), holding row + 1 (0 = absent;
// the largest row for duplicated coordinates, as the reference's map keeps the last insert).
// Position key = block * 512 + local index: the word of the voxel in the block array, unique per
// coordinate, ordered by cell (Morton) and then x, y, z inside the cell.
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
constexpr size_t GRID_TAIL = 32768;            // bytes: header + GRID_PARTS * 6 partials
constexpr int GRID_MODE_CELLS = 0, GRID_MODE_FALLBACK = 1;

struct GridHdr {
    int32_t mode;           // GRID_MODE_CELLS or GRID_MODE_FALLBACK
    int32_t bits;           // Morton bits per axis of the directory
    int32_t clo[3];         // first cell of the bounding box
    int32_t nblocks;        // occupied cells
    int32_t nplaced;        // voxels placed by the plan's cell walk (plan builds only)
    int32_t pad0;
    int64_t dir_n;          // directory words: 8^bits
    int64_t blocks_off;     // words from the directory to the first block
    int64_t region_words;   // words available for directory + blocks
};
static_assert(sizeof(GridHdr) <= 256, "header fits its slot");

// The tail (GRID_TAIL bytes, 16-byte aligned): the header, then int32 partials [6 GRID_PARTS].
struct GridTail {
    GridHdr* hdr;
    int32_t* parts;
};
inline GridTail carve_grid_tail(void* p) {
    char* c = static_cast<char*>(p);
    return GridTail{reinterpret_cast<GridHdr*>(c), reinterpret_cast<int32_t*>(c + 256)};
}
static_assert(256 + 4 * 6 * GRID_PARTS <= GRID_TAIL, "tail layout");

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
__device__ __forceinline__ int cell_local(int32_t x, int32_t y, int32_t z) {
    return ((x & 7) << 6) | ((y & 7) << 3) | (z & 7);
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
// (dz + 1): key[t] = position key (-1 where the cell is absent) and the block word there (row + 1,
// 0 = absent). The neighbourhood spans at most 2 cells per axis, so 8 directory reads serve it.
__device__ __forceinline__ void grid_neighbours(const GridRef& g, int32_t x, int32_t y, int32_t z,
                                                int32_t (&key)[kTaps], int32_t (&word)[kTaps]) {
    const int32_t cx0 = (x - 1) >> 3, cy0 = (y - 1) >> 3, cz0 = (z - 1) >> 3;
    const int32_t cx1 = (x + 1) >> 3, cy1 = (y + 1) >> 3, cz1 = (z + 1) >> 3;
    int32_t blk[8];
#pragma unroll
    for (int c = 0; c < 8; ++c)
        blk[c] = grid_block(g, (c & 1) ? cx1 : cx0, (c & 2) ? cy1 : cy0, (c & 4) ? cz1 : cz0);
#pragma unroll
    for (int t = 0; t < kTaps; ++t) {
        const int32_t nx = x + t / 9 - 1, ny = y + (t / 3) % 3 - 1, nz = z + t % 3 - 1;
        const int c = ((nx >> 3) != cx0 ? 1 : 0) | ((ny >> 3) != cy0 ? 2 : 0) | ((nz >> 3) != cz0 ? 4 : 0);
        key[t] = blk[c] >= 0 ? blk[c] * 512 + cell_local(nx, ny, nz) : -1;
    }
#pragma unroll
    for (int t = 0; t < kTaps; ++t) word[t] = key[t] >= 0 ? g.blocks[key[t]] : 0;
}

// Builds the grid of coords[0..n) in `region` (region_bytes, 16-byte aligned) with header and
// partials in `tail` (GRID_TAIL bytes). Coordinates outside [0, kCoordMax] are left out and set
// bit 0 of *status when status is given. Returns a tsp_status of the launches.
int grid_build(const int32_t* coords, int64_t n, void* region, size_t region_bytes, void* tail,
               int32_t* status, hipStream_t s);

}  // namespace tsp
