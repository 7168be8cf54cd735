// 2x subdivision (channel-to-spatial) index math on the GPU.
//
// Replaces the host loop of sparse_c2s (src/sparse.cpp:205-222): for parent i and octant
// o = 0..7 (ascending), a set mask byte spawns child (2x+(o&1), 2y+((o>>1)&1), 2z+((o>>2)&1))
// with gather index o + 8i; children are numbered parent-major, so mstart -- the first child
// of each parent -- is the exclusive prefix sum of the per-parent popcounts.
//
// Three launches: per-block child counts -> one-workgroup scan of the block counts (which also
// writes M) -> per-block rescan that writes mstart, the child coordinates and gidx.
#include <algorithm>
#include <mutex>

#include "common.hpp"

namespace tsp {
namespace {

constexpr int SD_THREADS = 256;
constexpr int SD_PER_THREAD = 4;
constexpr int SD_ITEMS = SD_THREADS * SD_PER_THREAD;   // parents per block

__device__ __forceinline__ uint32_t octant_bits(const uint8_t* __restrict__ mask, int64_t i) {
    uint32_t m = 0;
#pragma unroll
    for (int o = 0; o < 8; ++o) m |= (mask[8 * i + o] != 0 ? 1u : 0u) << o;
    return m;
}

// Exclusive scan of v over the workgroup; returns the prefix and writes the total.
__device__ __forceinline__ int32_t block_exclusive_scan(int32_t v, int32_t* total) {
    __shared__ int32_t sWave[SD_THREADS / 64];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    int32_t x = v;
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
        const int32_t y = __shfl_up(x, off, 64);
        if (lane >= off) x += y;
    }
    if (lane == 63) sWave[wave] = x;
    __syncthreads();
    int32_t base = 0, tot = 0;
#pragma unroll
    for (int w = 0; w < SD_THREADS / 64; ++w) {
        if (w < wave) base += sWave[w];
        tot += sWave[w];
    }
    __syncthreads();   // sWave may be reused by the caller's next scan
    *total = tot;
    return base + x - v;
}

__global__ __launch_bounds__(SD_THREADS) void k_block_counts(const uint8_t* __restrict__ mask,
                                                            int64_t n, int32_t* block_sums) {
    const int64_t p0 = (int64_t)blockIdx.x * SD_ITEMS + (int64_t)threadIdx.x * SD_PER_THREAD;
    int32_t c = 0;
#pragma unroll
    for (int k = 0; k < SD_PER_THREAD; ++k)
        if (p0 + k < n) c += __popc(octant_bits(mask, p0 + k));
    int32_t tot;
    block_exclusive_scan(c, &tot);
    if (threadIdx.x == 0) block_sums[blockIdx.x] = tot;
}

// One workgroup: exclusive scan of the nb block sums in place; M -> *m_out and mstart[n].
__global__ __launch_bounds__(SD_THREADS) void k_scan_block_sums(int32_t* block_sums, int64_t nb,
                                                               int64_t n, int32_t* mstart,
                                                               int64_t* m_out) {
    int32_t carry = 0;
    for (int64_t b0 = 0; b0 < nb; b0 += SD_THREADS) {
        const int64_t b = b0 + threadIdx.x;
        const int32_t v = b < nb ? block_sums[b] : 0;
        int32_t tot;
        const int32_t ex = block_exclusive_scan(v, &tot);
        if (b < nb) block_sums[b] = carry + ex;
        carry += tot;
    }
    if (threadIdx.x == 0) {
        mstart[n] = carry;
        *m_out = carry;
    }
}

__global__ __launch_bounds__(SD_THREADS) void k_emit_children(
    const uint8_t* __restrict__ mask, const int32_t* __restrict__ coords, int64_t n,
    const int32_t* __restrict__ block_offsets, int32_t* __restrict__ mstart,
    int32_t* __restrict__ child, int32_t* __restrict__ gidx) {
    const int64_t p0 = (int64_t)blockIdx.x * SD_ITEMS + (int64_t)threadIdx.x * SD_PER_THREAD;
    uint32_t bits[SD_PER_THREAD];
    int32_t c = 0;
#pragma unroll
    for (int k = 0; k < SD_PER_THREAD; ++k) {
        bits[k] = (p0 + k < n) ? octant_bits(mask, p0 + k) : 0u;
        c += __popc(bits[k]);
    }
    int32_t tot;
    int32_t m = block_offsets[blockIdx.x] + block_exclusive_scan(c, &tot);
#pragma unroll
    for (int k = 0; k < SD_PER_THREAD; ++k) {
        const int64_t i = p0 + k;
        if (i >= n) break;
        mstart[i] = m;
        const int32_t x = coords[3 * i], y = coords[3 * i + 1], z = coords[3 * i + 2];
        uint32_t b = bits[k];
        while (b) {
            const int o = __builtin_ctz(b);
            b &= b - 1;
            child[3 * (int64_t)m + 0] = 2 * x + (o & 1);
            child[3 * (int64_t)m + 1] = 2 * y + ((o >> 1) & 1);
            child[3 * (int64_t)m + 2] = 2 * z + ((o >> 2) & 1);
            gidx[m] = (int32_t)(o + 8 * i);
            ++m;
        }
    }
}

// The per-block child counts of tsp_subdivide_noalloc: one int32 per SD_ITEMS parents, enough
// for the largest n the subdivision accepts (8n < 2^31 -> at most 2^18 blocks), 1 MiB on each
// device. Host code reaches it only through the address hipGetSymbolAddress gives per device.
constexpr int64_t SD_SCRATCH_WORDS = int64_t(1) << 18;
static __device__ __align__(256) int32_t scratch[SD_SCRATCH_WORDS];

constexpr int SD_MAX_DEVICES = 64;
std::mutex g_scratch_mu;
int32_t* g_scratch_ptr[SD_MAX_DEVICES] = {};

// The three launches over `sums` (nb = ceil(n / SD_ITEMS) int32; every entry is written by
// k_block_counts before it is read, so nothing needs clearing).
int subdivide_launch(const uint8_t* mask, const int32_t* coords, int64_t n, int32_t* mstart,
                     int32_t* child, int32_t* gidx, int64_t* m_out, int32_t* sums, hipStream_t s) {
    const int64_t nb = ceil_div(n, SD_ITEMS);
    if (nb > 0) {
        hipLaunchKernelGGL(k_block_counts, dim3((unsigned)nb), dim3(SD_THREADS), 0, s, mask, n, sums);
        TSP_CHECK_LAUNCH();
    }
    hipLaunchKernelGGL(k_scan_block_sums, dim3(1), dim3(SD_THREADS), 0, s, sums, nb, n, mstart, m_out);
    TSP_CHECK_LAUNCH();
    if (nb > 0) {
        hipLaunchKernelGGL(k_emit_children, dim3((unsigned)nb), dim3(SD_THREADS), 0, s, mask, coords,
                           n, sums, mstart, child, gidx);
        TSP_CHECK_LAUNCH();
    }
    return TSP_OK;
}

int check_subdivide_args(const char* fn, const uint8_t* d_mask, const int32_t* d_coords, int64_t n,
                         const int32_t* d_mstart, const int32_t* d_child, const int32_t* d_gidx,
                         const int64_t* d_m) {
    TSP_REQUIRE(n >= 0 && 8 * n < (int64_t)INT32_MAX, TSP_ERR_INVALID,
                "%s: n=%lld out of range (8n must fit int32)", fn, (long long)n);
    TSP_REQUIRE(d_mstart && d_m, TSP_ERR_INVALID, "%s: null pointer", fn);
    TSP_REQUIRE(n == 0 || (d_mask && d_coords && d_child && d_gidx), TSP_ERR_INVALID,
                "%s: null pointer", fn);
    return TSP_OK;
}

}  // namespace
}  // namespace tsp

using namespace tsp;

extern "C" size_t tsp_subdivide_workspace_bytes(int64_t n) {
    if (n < 0) return 0;
    const int64_t nb = std::max<int64_t>(1, ceil_div(n, SD_ITEMS));
    return (size_t)nb * sizeof(int32_t);
}

extern "C" int tsp_subdivide(const uint8_t* d_mask, const int32_t* d_coords, int64_t n,
                             int32_t* d_mstart, int32_t* d_child_coords, int32_t* d_gidx,
                             int64_t* d_m, void* d_workspace, size_t workspace_bytes,
                             void* stream) {
    clear_error();
    if (int st = check_subdivide_args("tsp_subdivide", d_mask, d_coords, n, d_mstart,
                                      d_child_coords, d_gidx, d_m))
        return st;
    TSP_REQUIRE(d_workspace, TSP_ERR_INVALID, "tsp_subdivide: null pointer");
    TSP_REQUIRE(workspace_bytes >= tsp_subdivide_workspace_bytes(n), TSP_ERR_WORKSPACE,
                "tsp_subdivide: workspace %zu < %zu bytes", workspace_bytes,
                tsp_subdivide_workspace_bytes(n));
    return subdivide_launch(d_mask, d_coords, n, d_mstart, d_child_coords, d_gidx, d_m,
                            reinterpret_cast<int32_t*>(d_workspace), as_stream(stream));
}

extern "C" int tsp_subdivide_noalloc(const uint8_t* d_mask, const int32_t* d_coords, int64_t n,
                                     int32_t* d_mstart, int32_t* d_child_coords, int32_t* d_gidx,
                                     int64_t* d_m, void* stream) {
    clear_error();
    if (int st = check_subdivide_args("tsp_subdivide_noalloc", d_mask, d_coords, n, d_mstart,
                                      d_child_coords, d_gidx, d_m))
        return st;
    const int64_t nb = ceil_div(n, SD_ITEMS);
    TSP_REQUIRE(nb <= SD_SCRATCH_WORDS, TSP_ERR_INVALID,
                "tsp_subdivide_noalloc: n=%lld exceeds the scratch's %lld parents", (long long)n,
                (long long)(SD_SCRATCH_WORDS * SD_ITEMS));
    int dev = 0;
    TSP_CHECK_HIP(hipGetDevice(&dev));
    TSP_REQUIRE(dev >= 0 && dev < SD_MAX_DEVICES, TSP_ERR_INVALID,
                "tsp_subdivide_noalloc: device %d beyond the %d this library tracks", dev,
                SD_MAX_DEVICES);
    int32_t* sums = nullptr;
    {
        // first call on this device (it is current): look up its copy of the scratch array
        std::lock_guard<std::mutex> lock(g_scratch_mu);
        if (!g_scratch_ptr[dev]) {
            void* p = nullptr;
            TSP_CHECK_HIP(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)));
            TSP_REQUIRE(p, TSP_ERR_HIP, "tsp_subdivide_noalloc: no device address for the scratch");
            g_scratch_ptr[dev] = static_cast<int32_t*>(p);
        }
        sums = g_scratch_ptr[dev];
    }
    return subdivide_launch(d_mask, d_coords, n, d_mstart, d_child_coords, d_gidx, d_m, sums,
                            as_stream(stream));
}
