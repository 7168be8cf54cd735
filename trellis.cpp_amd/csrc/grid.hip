// Cell grid build (grid.hpp): bounding box, directory, blocks -- nine launches, no host round
// trip. Every kernel after the set-up returns at once when the header says the grid does not fit.
#include <algorithm>

#include "grid.hpp"

namespace tsp {
namespace {

constexpr int GB_NT = 256;   // threads of the grid-build workgroups

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
// (lo = INT32_MAX, hi = -1 when the workgroup saw none).
__global__ __launch_bounds__(GB_NT) void k_grid_bbox(const int32_t* __restrict__ coords, int64_t n,
                                                     int32_t* __restrict__ parts, int32_t* status) {
    __shared__ int sR[6][GB_NT / 64];
    int lo[3] = {INT32_MAX, INT32_MAX, INT32_MAX}, hi[3] = {-1, -1, -1};
    bool bad = false;
    for (int64_t i = blockIdx.x * (int64_t)GB_NT + threadIdx.x; i < n; i += (int64_t)gridDim.x * GB_NT) {
        const int32_t x = coords[3 * i], y = coords[3 * i + 1], z = coords[3 * i + 2];
        if (!coords_ok(x, y, z)) {
            bad = true;
            continue;
        }
        lo[0] = min(lo[0], x); lo[1] = min(lo[1], y); lo[2] = min(lo[2], z);
        hi[0] = max(hi[0], x); hi[1] = max(hi[1], y); hi[2] = max(hi[2], z);
    }
    if (status && __ballot(bad) != 0ull && (threadIdx.x & 63) == 0) atomicOr(status, 1);
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

// One workgroup: reduce the partials, size the directory, decide the mode.
__global__ __launch_bounds__(1024) void k_grid_setup(const int32_t* __restrict__ parts, int nparts,
                                                     GridHdr* hdr, int64_t region_words) {
    __shared__ int sR[6][16];
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    int v[6];
#pragma unroll
    for (int a = 0; a < 6; ++a) v[a] = tid < nparts ? parts[6 * tid + a] : (a < 3 ? INT32_MAX : -1);
#pragma unroll
    for (int a = 0; a < 6; ++a) {
        const int r = a < 3 ? wave_min_i(v[a]) : wave_max_i(v[a]);
        if (lane == 0) sR[a][wave] = r;
    }
    __syncthreads();
    if (tid != 0) return;
    int lo[3], hi[3];
#pragma unroll
    for (int a = 0; a < 3; ++a) {
        lo[a] = sR[a][0];
        hi[a] = sR[3 + a][0];
        for (int w = 1; w < 16; ++w) { lo[a] = min(lo[a], sR[a][w]); hi[a] = max(hi[a], sR[3 + a][w]); }
    }
    GridHdr h{};
    h.mode = GRID_MODE_CELLS;
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
    *hdr = h;
}

__global__ __launch_bounds__(GB_NT) void k_grid_dir_clear(const GridHdr* __restrict__ hdr, int32_t* __restrict__ dir) {
    if (hdr->mode != GRID_MODE_CELLS) return;
    const int64_t nw = hdr->dir_n;
    for (int64_t i = blockIdx.x * (int64_t)GB_NT + threadIdx.x; i < nw; i += (int64_t)gridDim.x * GB_NT) dir[i] = 0;
}

__global__ __launch_bounds__(GB_NT) void k_grid_mark(const int32_t* __restrict__ coords, int64_t n,
                                                     const GridHdr* __restrict__ hdr, int32_t* __restrict__ dir) {
    if (hdr->mode != GRID_MODE_CELLS) return;
    const int64_t i = blockIdx.x * (int64_t)GB_NT + threadIdx.x;
    if (i >= n) return;
    const int32_t x = coords[3 * i], y = coords[3 * i + 1], z = coords[3 * i + 2];
    if (!coords_ok(x, y, z)) return;
    const uint32_t m = cell_morton((uint32_t)((x >> 3) - hdr->clo[0]), (uint32_t)((y >> 3) - hdr->clo[1]),
                                   (uint32_t)((z >> 3) - hdr->clo[2]));
    dir[m] = 1;
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

// One workgroup of GRID_PARTS threads: the partials into exclusive prefixes, nblocks, and whether
// the blocks fit.
__global__ __launch_bounds__(GRID_PARTS) void k_grid_scan_top(GridHdr* __restrict__ hdr, int32_t* __restrict__ parts) {
    __shared__ int sW[GRID_PARTS / 64];
    if (hdr->mode != GRID_MODE_CELLS) return;
    int total;
    const int v = parts[threadIdx.x];
    parts[threadIdx.x] = block_exclusive_scan<GRID_PARTS>(v, sW, total);
    if (threadIdx.x == 0) {
        hdr->nblocks = total;
        if ((int64_t)total * 512 >= ((int64_t)1 << 31) || hdr->blocks_off + (int64_t)total * 512 > hdr->region_words)
            hdr->mode = GRID_MODE_FALLBACK;
    }
}

// Block numbers into the directory (Morton order), and the blocks cleared.
__global__ __launch_bounds__(GB_NT) void k_grid_apply(const GridHdr* __restrict__ hdr, int32_t* __restrict__ dir,
                                                      const int32_t* __restrict__ parts) {
    __shared__ int sW[GB_NT / 64];
    if (hdr->mode != GRID_MODE_CELLS) return;
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int64_t nw = hdr->dir_n, chunk = (nw + GRID_PARTS - 1) / GRID_PARTS;
    const int64_t b = blockIdx.x * chunk, e = min(nw, b + chunk);
    int run = parts[blockIdx.x];
    for (int64_t r0 = b; r0 < e; r0 += GB_NT) {
        const int64_t i = r0 + tid;
        const bool occ = i < e && dir[i] != 0;
        const uint64_t bal = __ballot(occ);
        if (lane == 0) sW[wave] = __popcll(bal);
        __syncthreads();
        int before = 0, total = 0;
        for (int w = 0; w < GB_NT / 64; ++w) {
            if (w < wave) before += sW[w];
            total += sW[w];
        }
        if (occ) dir[i] = run + before + __popcll(bal & ((1ull << lane) - 1ull)) + 1;
        run += total;
        __syncthreads();
    }
    // clear the blocks: nblocks * 512 words, 16 bytes per store
    u32x4_t* blk = reinterpret_cast<u32x4_t*>(dir + hdr->blocks_off);
    const int64_t n16 = (int64_t)hdr->nblocks * 128;
    for (int64_t i = blockIdx.x * (int64_t)GB_NT + tid; i < n16; i += (int64_t)gridDim.x * GB_NT)
        blk[i] = u32x4_t{0u, 0u, 0u, 0u};
}

// row + 1 of each voxel into its block word; duplicates: some writer wins, k_grid_fix raises it
// to the largest row
__global__ __launch_bounds__(GB_NT) void k_grid_insert(const int32_t* __restrict__ coords, int64_t n,
                                                       const GridHdr* __restrict__ hdr, int32_t* __restrict__ dir) {
    if (hdr->mode != GRID_MODE_CELLS) return;
    const int64_t i = blockIdx.x * (int64_t)GB_NT + threadIdx.x;
    if (i >= n) return;
    const int32_t x = coords[3 * i], y = coords[3 * i + 1], z = coords[3 * i + 2];
    if (!coords_ok(x, y, z)) return;
    const GridRef g = grid_ref(dir, hdr);
    const int32_t blk = grid_block(g, x >> 3, y >> 3, z >> 3);
    dir[hdr->blocks_off + (int64_t)blk * 512 + cell_local(x, y, z)] = (int32_t)(i + 1);
}

__global__ __launch_bounds__(GB_NT) void k_grid_fix(const int32_t* __restrict__ coords, int64_t n,
                                                    const GridHdr* __restrict__ hdr, int32_t* __restrict__ dir) {
    if (hdr->mode != GRID_MODE_CELLS) return;
    const int64_t i = blockIdx.x * (int64_t)GB_NT + threadIdx.x;
    if (i >= n) return;
    const int32_t x = coords[3 * i], y = coords[3 * i + 1], z = coords[3 * i + 2];
    if (!coords_ok(x, y, z)) return;
    const GridRef g = grid_ref(dir, hdr);
    const int32_t blk = grid_block(g, x >> 3, y >> 3, z >> 3);
    int32_t* w = dir + hdr->blocks_off + (int64_t)blk * 512 + cell_local(x, y, z);
    if (*w < (int32_t)(i + 1)) atomicMax(w, (int32_t)(i + 1));
}

}  // namespace

int grid_build(const int32_t* coords, int64_t n, void* region, size_t region_bytes, void* tail,
               int32_t* status, hipStream_t s) {
    const GridTail gt = carve_grid_tail(tail);
    int32_t* dir = static_cast<int32_t*>(region);
    const unsigned nvb = (unsigned)std::max<int64_t>(1, ceil_div(n, GB_NT));
    hipLaunchKernelGGL(k_grid_bbox, dim3(GRID_PARTS), dim3(GB_NT), 0, s, coords, n, gt.parts, status);
    TSP_CHECK_LAUNCH();
    hipLaunchKernelGGL(k_grid_setup, dim3(1), dim3(1024), 0, s, gt.parts, GRID_PARTS, gt.hdr,
                       (int64_t)(region_bytes / 4));
    TSP_CHECK_LAUNCH();
    hipLaunchKernelGGL(k_grid_dir_clear, dim3(GRID_PARTS), dim3(GB_NT), 0, s, gt.hdr, dir);
    TSP_CHECK_LAUNCH();
    hipLaunchKernelGGL(k_grid_mark, dim3(nvb), dim3(GB_NT), 0, s, coords, n, gt.hdr, dir);
    TSP_CHECK_LAUNCH();
    hipLaunchKernelGGL(k_grid_scan, dim3(GRID_PARTS), dim3(GB_NT), 0, s, gt.hdr, dir, gt.parts);
    TSP_CHECK_LAUNCH();
    hipLaunchKernelGGL(k_grid_scan_top, dim3(1), dim3(GRID_PARTS), 0, s, gt.hdr, gt.parts);
    TSP_CHECK_LAUNCH();
    hipLaunchKernelGGL(k_grid_apply, dim3(GRID_PARTS), dim3(GB_NT), 0, s, gt.hdr, dir, gt.parts);
    TSP_CHECK_LAUNCH();
    hipLaunchKernelGGL(k_grid_insert, dim3(nvb), dim3(GB_NT), 0, s, coords, n, gt.hdr, dir);
    TSP_CHECK_LAUNCH();
    hipLaunchKernelGGL(k_grid_fix, dim3(nvb), dim3(GB_NT), 0, s, coords, n, gt.hdr, dir);
    TSP_CHECK_LAUNCH();
    return TSP_OK;
}

}  // namespace tsp
