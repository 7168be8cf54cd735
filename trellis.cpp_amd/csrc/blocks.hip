// Per-voxel building blocks of the ConvNeXt and C2S blocks around the conv.
//
//   * row LayerNorm over channels (biased variance), optional affine and SiLU
//     (ggml_norm + mul/add + silu in sparse.cpp:124-127, 259-261, 293);
//   * the channel-to-spatial octant gather: child m takes the Cout-channel block (gidx[m] % 8)
//     of parent gidx[m] / 8 of conv1's [N][8 Cout] output (sparse.cpp:263-291);
//   * the C2S skip: child m adds parent x's K = Cin/8 channel block (gidx[m] % 8), each channel
//     repeated R = Cout/K times (repeat_interleave, sparse.cpp:302-323).
#include <algorithm>

#include "common.hpp"

namespace tsp {
namespace {

template <int DT>
__device__ __forceinline__ float ld(const void* p, int64_t i) {
    return Elem<DT>::load(reinterpret_cast<const typename Elem<DT>::storage*>(p), i);
}
template <int DT>
__device__ __forceinline__ void st(void* p, int64_t i, float v) {
    Elem<DT>::store(reinterpret_cast<typename Elem<DT>::storage*>(p), i, v);
}

__device__ __forceinline__ float wave_sum(float v) {
    for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
    return v;
}

// One wave per row; four rows per workgroup.
template <int XDT, int ODT>
__global__ __launch_bounds__(256) void k_layer_norm(const void* __restrict__ x, int64_t n, int c,
                                                    const float* __restrict__ gamma,
                                                    const float* __restrict__ beta, float eps,
                                                    int silu, void* __restrict__ out) {
    const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    if (row >= n) return;
    const int64_t base = row * c;
    float s = 0.f;
    for (int k = lane; k < c; k += 64) s += ld<XDT>(x, base + k);
    const float mean = wave_sum(s) / (float)c;
    float q = 0.f;
    for (int k = lane; k < c; k += 64) {
        const float d = ld<XDT>(x, base + k) - mean;
        q += d * d;
    }
    const float rstd = 1.0f / sqrtf(wave_sum(q) / (float)c + eps);
    for (int k = lane; k < c; k += 64) {
        float y = (ld<XDT>(x, base + k) - mean) * rstd;
        if (gamma) y *= gamma[k];
        if (beta) y += beta[k];
        if (silu) y = y / (1.0f + expf(-y));
        st<ODT>(out, base + k, y);
    }
}

template <int DT>
__global__ void k_c2s_gather(const void* __restrict__ h, const int32_t* __restrict__ gidx,
                             int64_t m, int cout, void* __restrict__ out) {
    const int64_t total = m * cout;
    for (int64_t e = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; e < total;
         e += (int64_t)gridDim.x * blockDim.x) {
        const int64_t r = e / cout, k = e % cout;
        st<DT>(out, e, ld<DT>(h, (int64_t)gidx[r] * cout + k));
    }
}

template <int XDT, int ADT>
__global__ void k_c2s_skip_add(const void* __restrict__ x, const int32_t* __restrict__ gidx,
                               int64_t m, int kb, int rep, void* __restrict__ acc) {
    const int cout = kb * rep;
    const int64_t total = m * cout;
    for (int64_t e = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; e < total;
         e += (int64_t)gridDim.x * blockDim.x) {
        const int64_t r = e / cout;
        const int ch = (int)(e % cout), k = ch / rep;     // channel k*R + r' -> source k
        const float v = ld<XDT>(x, (int64_t)gidx[r] * kb + k);
        st<ADT>(acc, e, ld<ADT>(acc, e) + v);
    }
}

__global__ void k_mask_positive(const float* __restrict__ logits, int64_t n,
                                uint8_t* __restrict__ mask) {
    for (int64_t e = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; e < n;
         e += (int64_t)gridDim.x * blockDim.x)
        mask[e] = logits[e] > 0.0f ? 1 : 0;
}

inline unsigned grid_for(int64_t total) {
    return (unsigned)std::max<int64_t>(1, std::min<int64_t>(ceil_div(total, 256), 65536));
}

}  // namespace
}  // namespace tsp

using namespace tsp;

#define TSP_DT_SWITCH(dt, NAME, ...)                                   \
    switch (dt) {                                                      \
        case TSP_F32: { constexpr int NAME = TSP_F32; __VA_ARGS__; } break;   \
        case TSP_F16: { constexpr int NAME = TSP_F16; __VA_ARGS__; } break;   \
        case TSP_BF16: { constexpr int NAME = TSP_BF16; __VA_ARGS__; } break; \
    }

extern "C" int tsp_layer_norm(const void* d_x, int x_dtype, int64_t n, int c,
                              const float* d_gamma, const float* d_beta, float eps, int silu,
                              void* d_out, int out_dtype, void* stream) {
    clear_error();
    TSP_REQUIRE(n >= 0 && c > 0, TSP_ERR_INVALID, "tsp_layer_norm: n=%lld c=%d", (long long)n, c);
    TSP_REQUIRE(dtype_valid(x_dtype) && dtype_valid(out_dtype), TSP_ERR_INVALID,
                "tsp_layer_norm: bad dtype");
    if (n == 0) return TSP_OK;
    TSP_REQUIRE(d_x && d_out, TSP_ERR_INVALID, "tsp_layer_norm: null pointer");
    hipStream_t s = as_stream(stream);
    const dim3 grid((unsigned)ceil_div(n, 4)), block(256);
    TSP_DT_SWITCH(x_dtype, XD, TSP_DT_SWITCH(out_dtype, OD,
        hipLaunchKernelGGL((k_layer_norm<XD, OD>), grid, block, 0, s, d_x, n, c, d_gamma,
                           d_beta, eps, silu, d_out)));
    TSP_CHECK_LAUNCH();
    return TSP_OK;
}

extern "C" int tsp_c2s_gather(const void* d_h, int dtype, const int32_t* d_gidx, int64_t m,
                              int cout, void* d_out, void* stream) {
    clear_error();
    TSP_REQUIRE(m >= 0 && cout > 0, TSP_ERR_INVALID, "tsp_c2s_gather: m=%lld cout=%d",
                (long long)m, cout);
    TSP_REQUIRE(dtype_valid(dtype), TSP_ERR_INVALID, "tsp_c2s_gather: bad dtype");
    if (m == 0) return TSP_OK;
    TSP_REQUIRE(d_h && d_gidx && d_out && d_out != d_h, TSP_ERR_INVALID,
                "tsp_c2s_gather: null or aliased pointer");
    hipStream_t s = as_stream(stream);
    TSP_DT_SWITCH(dtype, D, hipLaunchKernelGGL((k_c2s_gather<D>), dim3(grid_for(m * cout)),
                                               dim3(256), 0, s, d_h, d_gidx, m, cout, d_out));
    TSP_CHECK_LAUNCH();
    return TSP_OK;
}

extern "C" int tsp_c2s_skip_add(const void* d_x, int x_dtype, const int32_t* d_gidx, int64_t m,
                                int cin, int cout, void* d_acc, int acc_dtype, void* stream) {
    clear_error();
    TSP_REQUIRE(m >= 0 && cin > 0 && cout > 0 && cin % 8 == 0 && cout % (cin / 8) == 0,
                TSP_ERR_INVALID, "tsp_c2s_skip_add: need cin %% 8 == 0 and cout %% (cin/8) == 0 "
                "(cin=%d cout=%d)", cin, cout);
    TSP_REQUIRE(dtype_valid(x_dtype) && dtype_valid(acc_dtype), TSP_ERR_INVALID,
                "tsp_c2s_skip_add: bad dtype");
    if (m == 0) return TSP_OK;
    TSP_REQUIRE(d_x && d_gidx && d_acc && d_acc != d_x, TSP_ERR_INVALID,
                "tsp_c2s_skip_add: null or aliased pointer");
    hipStream_t s = as_stream(stream);
    const int kb = cin / 8, rep = cout / kb;
    TSP_DT_SWITCH(x_dtype, XD, TSP_DT_SWITCH(acc_dtype, AD,
        hipLaunchKernelGGL((k_c2s_skip_add<XD, AD>), dim3(grid_for(m * cout)), dim3(256), 0, s,
                           d_x, d_gidx, m, kb, rep, d_acc)));
    TSP_CHECK_LAUNCH();
    return TSP_OK;
}

extern "C" int tsp_mask_positive(const float* d_logits, int64_t n, uint8_t* d_mask, void* stream) {
    clear_error();
    TSP_REQUIRE(n >= 0, TSP_ERR_INVALID, "tsp_mask_positive: negative n");
    if (n == 0) return TSP_OK;
    TSP_REQUIRE(d_logits && d_mask, TSP_ERR_INVALID, "tsp_mask_positive: null pointer");
    hipLaunchKernelGGL(k_mask_positive, dim3(grid_for(n)), dim3(256), 0, as_stream(stream),
                       d_logits, n, d_mask);
    TSP_CHECK_LAUNCH();
    return TSP_OK;
}
