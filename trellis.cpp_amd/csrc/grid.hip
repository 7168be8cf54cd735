// Cell grid build (grid.hpp): bounding box, directory, blocks -- seven launches, no host round
// trip. When the grid does not fit and a brick hash is given, the same launches build the hash
// instead (its buckets cleared by the numbering launch, its voxels inserted by the insert launch).
#include <algorithm>

#include "brick_hash.hpp"

namespace tsp {
namespace {

constexpr int GB_NT = 256;        // threads of the grid-build workgroups
constexpr int BBOX_PARTS = GRID_PARTS;   // workgroups of the bounding-box pass

__device__ __forceinline__ int wave_min_i(int v) {
    for (int off = 32; off > 0; off >>= 1) v = min(v, __shfl_xor(v, off, 64));
    return v;
}
__device__ __forceinline__ int wave_max_i(int v) {
    for (int off = 32; off > 0; off >>= 1) v = max(v, __shfl_xor(v, off, 64));
    return v;
}
__device__ __forceinline__ int wave_sum_i(int v) {
    for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
    return v;
}

// Bounding box of the valid coordinates, one partial per workgroup: parts[6 p ..] = lo xyz, hi xyz
// (lo = INT32_MAX, hi = -1 when the workgroup saw none); parts[6 GRID_PARTS + p] = 1 when each
// of the workgroup's rows i > 0 comes strictly after row i - 1 in (x, y, z) order.
__global__ __launch_bounds__(GB_NT) void k_grid_bbox(const int32_t* __restrict__ coords, int64_t n,
                                                     int32_t* __restrict__ parts, int32_t* status) {
    __shared__ int sR[6][GB_NT / 64];
    int lo[3] = {INT32_MAX, INT32_MAX, INT32_MAX}, hi[3] = {-1, -1, -1};
    bool bad = false, desc = false;
    for (int64_t i = blockIdx.x * (int64_t)GB_NT + threadIdx.x; i < n; i += (int64_t)gridDim.x * GB_NT) {
        const int32_t x = coords[3 * i], y = coords[3 * i + 1], z = coords[3 * i + 2];
        if (i > 0) {
            const int32_t px = coords[3 * i - 3], py = coords[3 * i - 2], pz = coords[3 * i - 1];
            desc |= x < px || (x == px && (y < py || (y == py && z <= pz)));
        }
        if (!coords_ok(x, y, z)) {
            bad = true;
            continue;
        }
        lo[0] = min(lo[0], x); lo[1] = min(lo[1], y); lo[2] = min(lo[2], z);
        hi[0] = max(hi[0], x); hi[1] = max(hi[1], y); hi[2] = max(hi[2], z);
    }
    if (status && __ballot(bad) != 0ull && (threadIdx.x & 63) == 0) atomicOr(status, 1);
    const int asc = !__syncthreads_or(desc);
    if (threadIdx.x == 0) parts[6 * GRID_PARTS + blockIdx.x] = asc;
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
#pragma unroll
    for (int a = 0; a < 3; ++a) {
        const int l = wave_min_i(lo[a]), h = wave_max_i(hi[a]);
        if (lane == 0) { sR[a][wave] = l; sR[3 + a][wave] = h; }
    }
    __syncthreads();
    if (threadIdx.x < 6) {
        const int a = threadIdx.x;
        int v = sR[a][0];
        for (int w = 1; w < GB_NT / 64; ++w) v = a < 3 ? min(v, sR[a][w]) : max(v, sR[a][w]);
        parts[6 * blockIdx.x + a] = v;
    }
}

// Every workgroup reduces the bounding-box partials and sizes the directory (the same answer in
// each; workgroup 0 writes the header), then the directory is cleared.
__global__ __launch_bounds__(GB_NT) void k_grid_clear(const int32_t* __restrict__ parts, GridHdr* __restrict__ hdr,
                                                      int32_t* __restrict__ dir, int64_t region_words) {
    static_assert(BBOX_PARTS % GB_NT == 0, "whole partials per thread");
    static_assert(BBOX_PARTS == GRID_PARTS, "the ascending flags fill their partials");
    __shared__ int sR[6][GB_NT / 64];
    __shared__ GridHdr sH;
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
#pragma unroll
    for (int a = 0; a < 6; ++a) {
        int v = parts[6 * tid + a];
        for (int p = tid + GB_NT; p < BBOX_PARTS; p += GB_NT) {
            const int u = parts[6 * p + a];
            v = a < 3 ? min(v, u) : max(v, u);
        }
        const int r = a < 3 ? wave_min_i(v) : wave_max_i(v);
        if (lane == 0) sR[a][wave] = r;
    }
    bool desc = false;
    for (int p = tid; p < BBOX_PARTS; p += GB_NT) desc |= parts[6 * GRID_PARTS + p] == 0;
    const bool ascending = !__syncthreads_or(desc);
    if (tid == 0) {
        int lo[3], hi[3];
#pragma unroll
        for (int a = 0; a < 3; ++a) {
            lo[a] = sR[a][0];
            hi[a] = sR[3 + a][0];
            for (int w = 1; w < GB_NT / 64; ++w) { lo[a] = min(lo[a], sR[a][w]); hi[a] = max(hi[a], sR[3 + a][w]); }
        }
        GridHdr h{};
        h.mode = GRID_MODE_CELLS;
        h.ascending = ascending ? 1 : 0;
        if (hi[0] < 0) {                  // no valid voxel: a one-cell directory that stays empty
            lo[0] = lo[1] = lo[2] = 0;
            hi[0] = hi[1] = hi[2] = 0;
        }
        int ext = 1;
#pragma unroll
        for (int a = 0; a < 3; ++a) {
            h.clo[a] = lo[a] >> 3;
            ext = max(ext, (hi[a] >> 3) - h.clo[a] + 1);
        }
        int bits = 0;
        while ((1 << bits) < ext) ++bits;
        h.bits = bits;
        if (bits > GRID_MAX_BITS) {
            h.mode = GRID_MODE_FALLBACK;
            h.bits = 0;
        }
        h.dir_n = (int64_t)1 << (3 * h.bits);
        h.blocks_off = (h.dir_n + 63) & ~int64_t(63);
        h.region_words = region_words;
        if (h.blocks_off > region_words) h.mode = GRID_MODE_FALLBACK;
        sH = h;
        if (blockIdx.x == 0) *hdr = h;
    }
    __syncthreads();
    if (sH.mode != GRID_MODE_CELLS) return;
    const int64_t nw = sH.dir_n;
    for (int64_t i = blockIdx.x * (int64_t)GB_NT + tid; i < nw; i += (int64_t)gridDim.x * GB_NT) dir[i] = 0;
}

__global__ __launch_bounds__(GB_NT) void k_grid_mark(const int32_t* __restrict__ coords, int64_t n,
                                                     const GridHdr* __restrict__ hdr, int32_t* __restrict__ dir) {
    if (hdr->mode != GRID_MODE_CELLS) return;
    const int64_t i = blockIdx.x * (int64_t)GB_NT + threadIdx.x;
    if (i >= n) return;
    const int32_t x = coords[3 * i], y = coords[3 * i + 1], z = coords[3 * i + 2];
    if (!coords_ok(x, y, z)) return;
    const uint32_t rx = (uint32_t)((x >> 3) - hdr->clo[0]), ry = (uint32_t)((y >> 3) - hdr->clo[1]),
                   rz = (uint32_t)((z >> 3) - hdr->clo[2]);
    dir[cell_morton(rx, ry, rz)] = 1;
    // A voxel at the bottom (top) of its cell is the halo word of the cell below (above), which
    // must then have a block even when it holds no voxel: the neighbours of voxels in that
    // z-layer of cells are read from it.
    const int lz = z & 7;
    if (lz == 0 || lz == 7) {
        const uint32_t hz = lz == 0 ? rz - 1 : rz + 1;
        if (hz < (1u << hdr->bits)) dir[cell_morton(rx, ry, hz)] = 1;
    }
}

// Occupied directory words of each of GRID_PARTS chunks into parts[].
__global__ __launch_bounds__(GB_NT) void k_grid_scan(const GridHdr* __restrict__ hdr, const int32_t* __restrict__ dir,
                                                     int32_t* __restrict__ parts) {
    __shared__ int sW[GB_NT / 64];
    if (hdr->mode != GRID_MODE_CELLS) return;
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int64_t nw = hdr->dir_n, chunk = (nw + GRID_PARTS - 1) / GRID_PARTS;
    const int64_t b = blockIdx.x * chunk, e = min(nw, b + chunk);
    int c = 0;
    for (int64_t i = b + tid; i < e; i += GB_NT) c += dir[i] != 0;
    c = wave_sum_i(c);
    if (lane == 0) sW[wave] = c;
    __syncthreads();
    if (tid == 0) {
        int t = 0;
        for (int w = 0; w < GB_NT / 64; ++w) t += sW[w];
        parts[blockIdx.x] = t;
    }
}

// Every workgroup sums the GRID_PARTS partials for its own prefix and the block count, and
// decides whether the blocks fit the region and the caller's block_cap (the same answer in each;
// workgroup 0 records it). Then: block
// numbers into the directory (Morton order; cell_of, when given, gets each block's directory
// index) and the blocks cleared; or, when the grid does not fit and a hash is given, the hash's
// buckets cleared.
__global__ __launch_bounds__(GB_NT) void k_grid_apply(GridHdr* __restrict__ hdr, int32_t* __restrict__ dir,
                                                      const int32_t* __restrict__ parts, HashView hash,
                                                      int32_t* __restrict__ cell_of, int64_t block_cap) {
    constexpr int PPT = GRID_PARTS / GB_NT;
    __shared__ int sW[2][GB_NT / 64];
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    bool cells = hdr->mode == GRID_MODE_CELLS;
    int64_t nblocks = 0;
    int run = 0;
    if (cells) {
        int v = 0, before = 0;
#pragma unroll
        for (int k = 0; k < PPT; ++k) {
            const int p = tid * PPT + k;
            const int x = parts[p];
            if (p < (int)blockIdx.x) before += x;
            v += x;
        }
        v = wave_sum_i(v);
        before = wave_sum_i(before);
        if (lane == 0) { sW[0][wave] = v; sW[1][wave] = before; }
        __syncthreads();
        int tot = 0;
        for (int w = 0; w < GB_NT / 64; ++w) { tot += sW[0][w]; run += sW[1][w]; }
        __syncthreads();   // sW is reused by the numbering below
        nblocks = tot;
        cells = nblocks <= block_cap && nblocks * GRID_BLOCK_WORDS < ((int64_t)1 << 31) &&
                hdr->blocks_off + nblocks * GRID_BLOCK_WORDS <= hdr->region_words;
        if (blockIdx.x == 0 && tid == 0) {
            hdr->nblocks = (int32_t)nblocks;
            if (!cells) hdr->mode = GRID_MODE_FALLBACK;
        }
    }
    if (!cells) {
        if (hash.cap == 0) return;
        u32x4_t* w = reinterpret_cast<u32x4_t*>(hash.words);
        const int64_t n16 = (int64_t)hash.cap * (kBucketWords / 4);
        for (int64_t s = blockIdx.x * (int64_t)GB_NT + tid; s < n16; s += (int64_t)gridDim.x * GB_NT)
            w[s] = u32x4_t{0u, 0u, 0u, 0u};
        return;
    }
    const int64_t nw = hdr->dir_n, chunk = (nw + GRID_PARTS - 1) / GRID_PARTS;
    const int64_t b = blockIdx.x * chunk, e = min(nw, b + chunk);
    for (int64_t r0 = b; r0 < e; r0 += GB_NT) {
        const int64_t i = r0 + tid;
        const bool occ = i < e && dir[i] != 0;
        const uint64_t bal = __ballot(occ);
        if (lane == 0) sW[0][wave] = __popcll(bal);
        __syncthreads();
        int before = 0, total = 0;
        for (int w = 0; w < GB_NT / 64; ++w) {
            if (w < wave) before += sW[0][w];
            total += sW[0][w];
        }
        if (occ) {
            const int id = run + before + __popcll(bal & ((1ull << lane) - 1ull));
            dir[i] = id + 1;
            if (cell_of) cell_of[id] = (int32_t)i;
        }
        run += total;
        __syncthreads();
    }
    // clear the blocks, 16 bytes per store
    u32x4_t* blk = reinterpret_cast<u32x4_t*>(dir + hdr->blocks_off);
    const int64_t n16 = nblocks * (GRID_BLOCK_WORDS / 4);
    for (int64_t i = blockIdx.x * (int64_t)GB_NT + tid; i < n16; i += (int64_t)gridDim.x * GB_NT)
        blk[i] = u32x4_t{0u, 0u, 0u, 0u};
}

// The words a voxel's row goes to: its own cell's block, and the halo word of the cell below
// (z & 7 == 7) or above (z & 7 == 0) when that cell has a block. Returns how many (1 or 2).
__device__ __forceinline__ int voxel_words(const GridRef& g, int32_t x, int32_t y, int32_t z, int64_t (&w)[2]) {
    const int32_t cx = x >> 3, cy = y >> 3, cz = z >> 3;
    const int col = ((x & 7) * 8 + (y & 7)) * GRID_COL_WORDS;
    w[0] = (int64_t)grid_block(g, cx, cy, cz) * GRID_BLOCK_WORDS + col + (z & 7) + 1;
    if ((z & 7) == 0 || (z & 7) == 7) {
        const bool low = (z & 7) == 0;
        const int32_t b = grid_block(g, cx, cy, low ? cz - 1 : cz + 1);
        if (b >= 0) {
            w[1] = (int64_t)b * GRID_BLOCK_WORDS + col + (low ? GRID_COL_WORDS - 1 : 0);
            return 2;
        }
    }
    return 1;
}

// row + 1 of each voxel into its block words (duplicates: some writer wins, k_grid_fix raises it
// to the largest row); or the voxel into the hash
__global__ __launch_bounds__(GB_NT) void k_grid_insert(const int32_t* __restrict__ coords, int64_t n,
                                                       const GridHdr* __restrict__ hdr, int32_t* __restrict__ dir,
                                                       HashView hash) {
    const bool cells = hdr->mode == GRID_MODE_CELLS;
    if (!cells && hash.cap == 0) return;
    const int64_t i = blockIdx.x * (int64_t)GB_NT + threadIdx.x;
    if (i >= n) return;
    const int32_t x = coords[3 * i], y = coords[3 * i + 1], z = coords[3 * i + 2];
    if (!coords_ok(x, y, z)) return;
    if (!cells) {
        hash_insert(hash, i, x, y, z);
        return;
    }
    const GridRef g = grid_ref(dir, hdr);
    int64_t w[2];
    const int k = voxel_words(g, x, y, z, w);
    int32_t* blocks = dir + hdr->blocks_off;
    blocks[w[0]] = (int32_t)(i + 1);
    if (k == 2) blocks[w[1]] = (int32_t)(i + 1);
}

// Duplicated coordinates: each word raised to the largest row that holds it. Rows strictly
// ascending in (x, y, z) repeat no coordinate, and then the insert's stores are final.
__global__ __launch_bounds__(GB_NT) void k_grid_fix(const int32_t* __restrict__ coords, int64_t n,
                                                    const GridHdr* __restrict__ hdr, int32_t* __restrict__ dir) {
    if (hdr->mode != GRID_MODE_CELLS || hdr->ascending) return;
    const GridRef g = grid_ref(dir, hdr);
    int32_t* blocks = dir + hdr->blocks_off;
    for (int64_t i = blockIdx.x * (int64_t)GB_NT + threadIdx.x; i < n; i += (int64_t)gridDim.x * GB_NT) {
        const int32_t x = coords[3 * i], y = coords[3 * i + 1], z = coords[3 * i + 2];
        if (!coords_ok(x, y, z)) continue;
        int64_t w[2];
        const int k = voxel_words(g, x, y, z, w);
        for (int j = 0; j < k; ++j)
            if (blocks[w[j]] < (int32_t)(i + 1)) atomicMax(&blocks[w[j]], (int32_t)(i + 1));
    }
}

}  // namespace

int grid_build(const int32_t* coords, int64_t n, void* region, size_t region_bytes, void* tail,
               int32_t* status, HashView hash, int32_t* cell_of, int64_t block_cap, hipStream_t s) {
    const GridTail gt = carve_grid_tail(tail);
    int32_t* dir = static_cast<int32_t*>(region);
    const unsigned nvb = (unsigned)std::max<int64_t>(1, ceil_div(n, GB_NT));
    hipLaunchKernelGGL(k_grid_bbox, dim3(BBOX_PARTS), dim3(GB_NT), 0, s, coords, n, gt.parts, status);
    TSP_CHECK_LAUNCH();
    hipLaunchKernelGGL(k_grid_clear, dim3(GRID_PARTS), dim3(GB_NT), 0, s, gt.parts, gt.hdr, dir,
                       (int64_t)(region_bytes / 4));
    TSP_CHECK_LAUNCH();
    hipLaunchKernelGGL(k_grid_mark, dim3(nvb), dim3(GB_NT), 0, s, coords, n, gt.hdr, dir);
    TSP_CHECK_LAUNCH();
    hipLaunchKernelGGL(k_grid_scan, dim3(GRID_PARTS), dim3(GB_NT), 0, s, gt.hdr, dir, gt.parts);
    TSP_CHECK_LAUNCH();
    hipLaunchKernelGGL(k_grid_apply, dim3(GRID_PARTS), dim3(GB_NT), 0, s, gt.hdr, dir, gt.parts, hash, cell_of,
                       block_cap);
    TSP_CHECK_LAUNCH();
    hipLaunchKernelGGL(k_grid_insert, dim3(nvb), dim3(GB_NT), 0, s, coords, n, gt.hdr, dir, hash);
    TSP_CHECK_LAUNCH();
    hipLaunchKernelGGL(k_grid_fix, dim3(std::min(nvb, 4u * GRID_PARTS)), dim3(GB_NT), 0, s, coords, n, gt.hdr, dir);
    TSP_CHECK_LAUNCH();
    return TSP_OK;
}

}  // namespace tsp
