// Tap-major neighbour table on the GPU.
//
// Replaces trellis::build_neighbor_table (src/sparse.cpp:21-39). The reference inserts every
// voxel into a host std::unordered_map (later rows overwrite earlier ones, :26) and probes the
// 27 offsets of each voxel (:28-37). Here the map is one of two structures in HBM:
//   * the cell grid (grid.hpp) when the voxels' bounding box is compact enough for the
//     workspace: a Morton-ordered directory of 8^3 cells and a block per occupied cell, built
//     without atomics on the hot path (plain stores, then a max-fix pass for duplicated
//     coordinates). A voxel's 27 neighbours are 4 directory reads and 9 three-word block reads,
//     mostly from L2 since neighbouring voxels share cells;
//   * otherwise (scattered or far-flung voxels) the hash of 2x2x2 bricks (brick_hash.hpp).
// Both are built in the same workspace by the same launches; which one is decided on the device.
// One thread per voxel then writes its 27 entries, tap-major, so every store of a wave is one
// coalesced 256-byte row segment.

#include <algorithm>

#include "brick_hash.hpp"
#include "conv_internal.hpp"

namespace tsp {
namespace {

constexpr int kProbeThreads = 256;

// The table: the 27 neighbours of each voxel from the grid or the hash.
__global__ __launch_bounds__(kProbeThreads) void k_table_probe(const int32_t* __restrict__ coords, int64_t n,
                                                               const int32_t* __restrict__ dir,
                                                               const GridHdr* __restrict__ hdr, HashView hash,
                                                               int32_t* __restrict__ nbr) {
    const int64_t i = blockIdx.x * (int64_t)kProbeThreads + threadIdx.x;
    if (i < n) probe_voxel(coords, n, i, dir, hdr, hash, nbr);
}

__global__ void k_count_pairs(const int32_t* __restrict__ nbr, int64_t total, int32_t sentinel,
                              unsigned long long* count) {
    unsigned long long local = 0;
    for (int64_t j = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; j < total;
         j += (int64_t)gridDim.x * blockDim.x)
        local += nbr[j] != sentinel;
    // wave reduction, then one atomic per wave
    for (int off = 32; off > 0; off >>= 1) local += __shfl_down(local, off, 64);
    if ((threadIdx.x & 63) == 0 && local) atomicAdd(count, local);
}

}  // namespace
}  // namespace tsp

using namespace tsp;

// workspace: the hash buckets (also the cell grid's directory and blocks), then the grid's tail
extern "C" size_t tsp_rulebook_workspace_bytes(int64_t n) {
    if (n < 0) return 0;
    return table_capacity(n) * kBucketWords * 4 + GRID_TAIL;
}

static int rulebook_build(const int32_t* d_coords, int64_t n, int32_t* d_nbr, void* d_workspace,
                          size_t workspace_bytes, int32_t* d_status, void* d_plan, hipStream_t s);

extern "C" int tsp_rulebook_build(const int32_t* d_coords, int64_t n, int32_t* d_nbr,
                                  void* d_workspace, size_t workspace_bytes, int32_t* d_status,
                                  void* stream) {
    clear_error();
    return rulebook_build(d_coords, n, d_nbr, d_workspace, workspace_bytes, d_status, nullptr, as_stream(stream));
}

extern "C" int tsp_rulebook_build_planned(const int32_t* d_coords, int64_t n, int32_t* d_nbr, void* d_workspace,
                                          size_t workspace_bytes, int32_t* d_status, void* d_plan,
                                          size_t plan_bytes, void* stream) {
    clear_error();
    TSP_REQUIRE(n >= 0 && n < (int64_t)INT32_MAX, TSP_ERR_INVALID,
                "tsp_rulebook_build_planned: n=%lld out of range", (long long)n);
    if (n == 0) return TSP_OK;
    TSP_REQUIRE(d_plan, TSP_ERR_INVALID, "tsp_rulebook_build_planned: null plan");
    TSP_REQUIRE(plan_bytes >= halo_plan_bytes(n), TSP_ERR_WORKSPACE,
                "tsp_rulebook_build_planned: plan buffer %zu < %zu bytes", plan_bytes, halo_plan_bytes(n));
    TSP_REQUIRE((reinterpret_cast<uintptr_t>(d_plan) & 15) == 0, TSP_ERR_INVALID,
                "tsp_rulebook_build_planned: the plan buffer must be 16-byte aligned");
    return rulebook_build(d_coords, n, d_nbr, d_workspace, workspace_bytes, d_status, d_plan, as_stream(stream));
}

// The table, and with d_plan the ordered plan on the same grid.
static int rulebook_build(const int32_t* d_coords, int64_t n, int32_t* d_nbr, void* d_workspace,
                          size_t workspace_bytes, int32_t* d_status, void* d_plan, hipStream_t s) {
    TSP_REQUIRE(n >= 0 && n < (int64_t)INT32_MAX, TSP_ERR_INVALID,
                "tsp_rulebook_build: n=%lld out of range", (long long)n);
    if (n == 0) return TSP_OK;
    TSP_REQUIRE(d_coords && d_nbr && d_workspace, TSP_ERR_INVALID,
                "tsp_rulebook_build: null pointer");
    TSP_REQUIRE(workspace_bytes >= tsp_rulebook_workspace_bytes(n), TSP_ERR_WORKSPACE,
                "tsp_rulebook_build: workspace %zu < %zu bytes", workspace_bytes,
                tsp_rulebook_workspace_bytes(n));
    HashView h{reinterpret_cast<uint32_t*>(d_workspace), table_capacity(n)};
    TSP_REQUIRE((reinterpret_cast<uintptr_t>(d_workspace) & 63) == 0, TSP_ERR_INVALID,
                "tsp_rulebook_build: workspace must be 64-byte aligned");
    const size_t region = h.cap * kBucketWords * 4;
    void* tail = static_cast<char*>(d_workspace) + region;
    const GridHdr* hdr = carve_grid_tail(tail).hdr;
    const int st = grid_build(d_coords, n, d_workspace, region, tail, d_status, h,
                              d_plan ? plan_cell_of(d_plan, n) : nullptr,
                              d_plan ? plan_block_cap(n) : INT64_MAX, s);
    if (st != TSP_OK) return st;
    if (d_plan) {
        // the probe's workgroups ride on the plan's walk launches (the walk is latency-bound, the
        // probe bound by its stores); the plan reads the table only after those launches
        ProbeJob pj;
        pj.nbr = d_nbr;
        pj.hash = h;
        pj.v1 = n;
        return halo_plan_build_on_grid(d_nbr, d_coords, n, d_plan, d_workspace, tail, s, &pj);
    }
    hipLaunchKernelGGL(k_table_probe, dim3((unsigned)ceil_div(n, kProbeThreads)), dim3(kProbeThreads), 0, s,
                       d_coords, n, static_cast<const int32_t*>(d_workspace), hdr, h, d_nbr);
    TSP_CHECK_LAUNCH();
    return TSP_OK;
}

extern "C" int tsp_rulebook_count_pairs(const int32_t* d_nbr, int64_t n,
                                        unsigned long long* d_count, void* stream) {
    clear_error();
    TSP_REQUIRE(n >= 0, TSP_ERR_INVALID, "tsp_rulebook_count_pairs: negative n");
    if (n == 0) return TSP_OK;
    TSP_REQUIRE(d_nbr && d_count, TSP_ERR_INVALID, "tsp_rulebook_count_pairs: null pointer");
    const int64_t total = 27 * n;
    const int blocks = (int)std::min<int64_t>(ceil_div(total, 256), 2048);
    hipLaunchKernelGGL(k_count_pairs, dim3(blocks), dim3(256), 0, as_stream(stream), d_nbr, total,
                       (int32_t)n, d_count);
    TSP_CHECK_LAUNCH();
    return TSP_OK;
}
