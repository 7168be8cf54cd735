// Coordinate hash and tap-major neighbour table on the GPU.
//
// Replaces trellis::build_neighbor_table (src/sparse.cpp:21-39). The reference inserts every
// voxel into a host std::unordered_map (later rows overwrite earlier ones, :26) and probes the
// 27 offsets of each voxel (:28-37). Here:
//   * the map is an open-addressing table in HBM: 64-bit keys (21 bits per axis, coordinate+1
//     so that the -1 probes have a key of their own) and int32 values, linear probing, load
//     factor <= 1/2;
//   * inserts claim a slot with a 64-bit CAS and keep the largest row with atomicMax -- the
//     reference's "last insert wins" for duplicate coordinates, independent of thread order,
//     so the table is deterministic;
//   * probes run one thread per (voxel, tap) on a tap-major grid, so every store of the table
//     is coalesced and consecutive threads probe neighbouring keys.
#include <algorithm>

#include "common.hpp"

namespace tsp {
namespace {

constexpr uint64_t kEmptyKey = ~0ull;
constexpr int32_t kCoordMax = (1 << 21) - 3;   // voxel coords in [0, kCoordMax]

__device__ __forceinline__ uint64_t pack_key(int32_t x, int32_t y, int32_t z) {
    // x,y,z in [-1, 2^21-2] -> fields of 21 bits; bit 63 is never set, so ~0 is free.
    return (uint64_t)(uint32_t)(x + 1) | ((uint64_t)(uint32_t)(y + 1) << 21) |
           ((uint64_t)(uint32_t)(z + 1) << 42);
}

__device__ __forceinline__ uint64_t slot_hash(uint64_t k) {
    k ^= k >> 31; k *= 0x7fb5d329728ea185ull;
    k ^= k >> 27; k *= 0x81dadef4bc2dd44dull;
    k ^= k >> 33;
    return k;
}

struct HashView {
    uint64_t* keys;
    int32_t* vals;
    uint64_t mask;
};

inline uint64_t table_capacity(int64_t n) {
    uint64_t cap = 1024;
    while (cap < (uint64_t)(2 * n)) cap <<= 1;
    return cap;
}

inline size_t align256(size_t b) { return (b + 255) & ~size_t(255); }

inline HashView carve(void* ws, int64_t n) {
    const uint64_t cap = table_capacity(n);
    HashView h;
    h.keys = reinterpret_cast<uint64_t*>(ws);
    h.vals = reinterpret_cast<int32_t*>(reinterpret_cast<char*>(ws) + align256(cap * 8));
    h.mask = cap - 1;
    return h;
}

__global__ void k_hash_clear(HashView h) {
    const uint64_t cap = h.mask + 1;
    for (uint64_t s = blockIdx.x * (uint64_t)blockDim.x + threadIdx.x; s < cap;
         s += (uint64_t)gridDim.x * blockDim.x) {
        h.keys[s] = kEmptyKey;
        h.vals[s] = -1;
    }
}

__global__ void k_hash_insert(const int32_t* __restrict__ coords, int64_t n, HashView h,
                              int32_t* status) {
    const int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
    if (i >= n) return;
    const int32_t x = coords[3 * i], y = coords[3 * i + 1], z = coords[3 * i + 2];
    if (x < 0 || y < 0 || z < 0 || x > kCoordMax || y > kCoordMax || z > kCoordMax) {
        if (status) atomicOr(status, 1);
        return;
    }
    const uint64_t key = pack_key(x, y, z);
    uint64_t s = slot_hash(key) & h.mask;
    // The table holds at least 2n slots, so an empty or matching slot is always reached.
    for (;;) {
        unsigned long long prev = atomicCAS(reinterpret_cast<unsigned long long*>(h.keys + s),
                                            (unsigned long long)kEmptyKey,
                                            (unsigned long long)key);
        if (prev == kEmptyKey || prev == key) {
            atomicMax(h.vals + s, (int32_t)i);
            return;
        }
        s = (s + 1) & h.mask;
    }
}

__device__ __forceinline__ int32_t hash_find(const HashView& h, uint64_t key, int32_t miss) {
    uint64_t s = slot_hash(key) & h.mask;
    for (;;) {
        const uint64_t k = h.keys[s];
        if (k == key) return h.vals[s];
        if (k == kEmptyKey) return miss;
        s = (s + 1) & h.mask;
    }
}

// Grid: x = runs of kProbeRows consecutive voxels, y = tap.
constexpr int kProbeRows = 256;

__global__ __launch_bounds__(kProbeRows) void k_probe(const int32_t* __restrict__ coords,
                                                      int64_t n, HashView h,
                                                      int32_t* __restrict__ nbr) {
    const int64_t i = blockIdx.x * (int64_t)kProbeRows + threadIdx.x;
    const int t = blockIdx.y;
    if (i >= n) return;
    const int32_t x = coords[3 * i], y = coords[3 * i + 1], z = coords[3 * i + 2];
    const int32_t miss = (int32_t)n;
    int32_t r = miss;
    if (x >= 0 && y >= 0 && z >= 0 && x <= kCoordMax && y <= kCoordMax && z <= kCoordMax) {
        const int dx = t / 9 - 1, dy = (t / 3) % 3 - 1, dz = t % 3 - 1;
        r = hash_find(h, pack_key(x + dx, y + dy, z + dz), miss);
    }
    nbr[(int64_t)t * n + i] = r;
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

extern "C" size_t tsp_rulebook_workspace_bytes(int64_t n) {
    if (n < 0) return 0;
    const uint64_t cap = table_capacity(n);
    return align256(cap * 8) + align256(cap * 4);
}

extern "C" int tsp_rulebook_build(const int32_t* d_coords, int64_t n, int32_t* d_nbr,
                                  void* d_workspace, size_t workspace_bytes, int32_t* d_status,
                                  void* stream) {
    clear_error();
    TSP_REQUIRE(n >= 0 && n < (int64_t)INT32_MAX, TSP_ERR_INVALID,
                "tsp_rulebook_build: n=%lld out of range", (long long)n);
    if (n == 0) return TSP_OK;
    TSP_REQUIRE(d_coords && d_nbr && d_workspace, TSP_ERR_INVALID,
                "tsp_rulebook_build: null pointer");
    TSP_REQUIRE(workspace_bytes >= tsp_rulebook_workspace_bytes(n), TSP_ERR_WORKSPACE,
                "tsp_rulebook_build: workspace %zu < %zu bytes", workspace_bytes,
                tsp_rulebook_workspace_bytes(n));
    hipStream_t s = as_stream(stream);
    HashView h = carve(d_workspace, n);
    const uint64_t cap = h.mask + 1;
    const int clear_blocks = (int)std::min<uint64_t>(ceil_div((int64_t)cap, 256), 4096);
    hipLaunchKernelGGL(k_hash_clear, dim3(clear_blocks), dim3(256), 0, s, h);
    TSP_CHECK_LAUNCH();
    hipLaunchKernelGGL(k_hash_insert, dim3((unsigned)ceil_div(n, 256)), dim3(256), 0, s,
                       d_coords, n, h, d_status);
    TSP_CHECK_LAUNCH();
    hipLaunchKernelGGL(k_probe, dim3((unsigned)ceil_div(n, kProbeRows), kTaps), dim3(kProbeRows),
                       0, s, d_coords, n, h, d_nbr);
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
