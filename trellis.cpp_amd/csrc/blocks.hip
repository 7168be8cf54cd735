// Per-voxel building blocks of the ConvNeXt and C2S blocks around the conv.
//
//   * row LayerNorm over channels (biased variance), optional affine and SiLU
//     (ggml_norm + mul/add + silu in sparse.cpp:124-127, 259-261, 293);
//   * the channel-to-spatial octant gather: child m takes the Cout-channel block (gidx[m] % 8)
//     of parent gidx[m] / 8 of conv1's [N][8 Cout] output (sparse.cpp:263-291);
//   * the C2S skip: child m adds parent x's K = Cin/8 channel block (gidx[m] % 8), each channel
//     repeated R = Cout/K times (repeat_interleave, sparse.cpp:302-323);
//   * the elementwise steps the composite blocks need between library calls: rounding an f32
//     tensor to a product's input type, SiLU into that type, and a residual add.
#include <algorithm>

#include "blocks_internal.hpp"
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

// 4 consecutive elements (16-byte f32 / 8-byte 16-bit accesses; the index is a multiple of 4).
template <int DT>
__device__ __forceinline__ void ld4(const void* p, int64_t i, float (&v)[4]) {
    if constexpr (DT == TSP_F32) {
        const f32x4_t t = *reinterpret_cast<const f32x4_t*>(static_cast<const float*>(p) + i);
#pragma unroll
        for (int e = 0; e < 4; ++e) v[e] = t[e];
    } else {
        const uint2 t = *reinterpret_cast<const uint2*>(static_cast<const uint16_t*>(p) + i);
        const uint16_t h[4] = {(uint16_t)(t.x & 0xffffu), (uint16_t)(t.x >> 16), (uint16_t)(t.y & 0xffffu),
                               (uint16_t)(t.y >> 16)};
#pragma unroll
        for (int e = 0; e < 4; ++e) v[e] = DT == TSP_BF16 ? bf16_bits_to_f32(h[e]) : f16_bits_to_f32(h[e]);
    }
}
template <int DT>
__device__ __forceinline__ void st4(void* p, int64_t i, const float (&v)[4]) {
    if constexpr (DT == TSP_F32) {
        *reinterpret_cast<f32x4_t*>(static_cast<float*>(p) + i) = f32x4_t{v[0], v[1], v[2], v[3]};
    } else {
        uint32_t w[2];
#pragma unroll
        for (int e = 0; e < 2; ++e)
            w[e] = DT == TSP_BF16 ? f32x2_to_bf16x2_bits(v[2 * e], v[2 * e + 1])
                                  : f32_to_f16_bits(v[2 * e]) | ((uint32_t)f32_to_f16_bits(v[2 * e + 1]) << 16);
        *reinterpret_cast<uint2*>(static_cast<uint16_t*>(p) + i) = uint2{w[0], w[1]};
    }
}

// Rows of c = 4 L V channels held in registers: L lanes per row (64 / L rows per wave), each lane
// V groups of 4 channels, interleaved so that a row's lanes read consecutive 16 bytes. One read of
// x, one write of out; every lane takes part in the group reductions, rows past n store nothing.
template <int XDT, int ODT, int L, int V>
__global__ __launch_bounds__(256) void k_layer_norm_vec(const void* __restrict__ x, int64_t n, int c,
                                                        const float* __restrict__ gamma,
                                                        const float* __restrict__ beta, float eps,
                                                        int silu, void* __restrict__ out) {
    constexpr int R = 64 / L;
    const int lane = threadIdx.x & 63, sub = lane % L;
    const int64_t row = ((int64_t)blockIdx.x * 4 + (threadIdx.x >> 6)) * R + lane / L;
    const bool live = row < n;
    const int64_t base = (live ? row : 0) * c;
    float v[V][4];
#pragma unroll
    for (int j = 0; j < V; ++j) ld4<XDT>(x, base + (j * L + sub) * 4, v[j]);
    float s = 0.f;
#pragma unroll
    for (int j = 0; j < V; ++j)
#pragma unroll
        for (int e = 0; e < 4; ++e) s += v[j][e];
    s = group_sum<L>(s);
    const float mean = s / (float)c;
    float q = 0.f;
#pragma unroll
    for (int j = 0; j < V; ++j)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const float d = v[j][e] - mean;
            q += d * d;
        }
    q = group_sum<L>(q);
    const float rstd = 1.0f / sqrtf(q / (float)c + eps);
#pragma unroll
    for (int j = 0; j < V; ++j) {
        const int ch = (j * L + sub) * 4;
        float g[4] = {1.f, 1.f, 1.f, 1.f}, b[4] = {0.f, 0.f, 0.f, 0.f}, y[4];
        if (gamma) ld4<TSP_F32>(gamma, ch, g);
        if (beta) ld4<TSP_F32>(beta, ch, b);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            y[e] = (v[j][e] - mean) * rstd * g[e] + b[e];
            if (silu) y[e] = y[e] / (1.0f + expf(-y[e]));
        }
        if (live) st4<ODT>(out, base + ch, y);
    }
}

// Row copies of 4 elements per thread: out[r][k] = h[gidx[r]][k] (cout % 4 == 0).
template <int DT>
__global__ void k_c2s_gather_vec(const void* __restrict__ h, const int32_t* __restrict__ gidx,
                                 int64_t m, int cout, void* __restrict__ out) {
    const int q = cout / 4;
    const int64_t total = m * q;
    for (int64_t e = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; e < total;
         e += (int64_t)gridDim.x * blockDim.x) {
        const int64_t r = e / q;
        const int k = (int)(e - r * q) * 4;
        float v[4];
        ld4<DT>(h, (int64_t)gidx[r] * cout + k, v);
        st4<DT>(out, r * cout + k, v);
    }
}

// The skip with 4 output channels per thread, all from one source channel (rep % 4 == 0).
template <int XDT, int ADT>
__global__ void k_c2s_skip_add_vec(const void* __restrict__ x, const int32_t* __restrict__ gidx,
                                   int64_t m, int kb, int rep, void* __restrict__ acc) {
    const int q = kb * rep / 4;
    const int64_t total = m * q;
    for (int64_t e = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; e < total;
         e += (int64_t)gridDim.x * blockDim.x) {
        const int64_t r = e / q;
        const int ch = (int)(e - r * q) * 4;
        const float xv = ld<XDT>(x, (int64_t)gidx[r] * kb + ch / rep);
        float a[4];
        ld4<ADT>(acc, r * kb * rep + ch, a);
#pragma unroll
        for (int t = 0; t < 4; ++t) a[t] += xv;
        st4<ADT>(acc, r * kb * rep + ch, a);
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

// y = f(x) stored as DT (round to nearest even for 16-bit types), f = identity or SiLU
template <int DT, bool SILU>
__global__ void k_f32_to(const float* __restrict__ x, int64_t n, void* __restrict__ y) {
    for (int64_t e = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; e < n;
         e += (int64_t)gridDim.x * blockDim.x) {
        float v = x[e];
        if constexpr (SILU) v = v / (1.0f + expf(-v));
        st<DT>(y, e, v);
    }
}

template <int XDT>
__global__ void k_add_to(float* __restrict__ y, const void* __restrict__ x, int64_t n) {
    for (int64_t e = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; e < n;
         e += (int64_t)gridDim.x * blockDim.x)
        y[e] += ld<XDT>(x, e);
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

int f32_to(const float* x, int64_t n, void* y, int ydt, bool silu, hipStream_t s) {
    if (n <= 0) return TSP_OK;
    const dim3 g(grid_for(n)), b(256);
#define TSP_F32_TO(DT)                                                                     \
    if (silu) hipLaunchKernelGGL((k_f32_to<DT, true>), g, b, 0, s, x, n, y);               \
    else hipLaunchKernelGGL((k_f32_to<DT, false>), g, b, 0, s, x, n, y);
    if (ydt == TSP_F32) { TSP_F32_TO(TSP_F32) }
    else if (ydt == TSP_F16) { TSP_F32_TO(TSP_F16) }
    else { TSP_F32_TO(TSP_BF16) }
#undef TSP_F32_TO
    TSP_CHECK_LAUNCH();
    return TSP_OK;
}

int add_to(float* y, const void* x, int xdt, int64_t n, hipStream_t s) {
    if (n <= 0) return TSP_OK;
    const dim3 g(grid_for(n)), b(256);
    if (xdt == TSP_F32) hipLaunchKernelGGL(k_add_to<TSP_F32>, g, b, 0, s, y, x, n);
    else if (xdt == TSP_F16) hipLaunchKernelGGL(k_add_to<TSP_F16>, g, b, 0, s, y, x, n);
    else hipLaunchKernelGGL(k_add_to<TSP_BF16>, g, b, 0, s, y, x, n);
    TSP_CHECK_LAUNCH();
    return TSP_OK;
}

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
    // power-of-two widths 64..2048 with aligned buffers: rows in registers, 16-byte accesses
    const bool aligned = !(reinterpret_cast<uintptr_t>(d_x) % 16 || reinterpret_cast<uintptr_t>(d_out) % 16 ||
                           reinterpret_cast<uintptr_t>(d_gamma) % 16 || reinterpret_cast<uintptr_t>(d_beta) % 16);
    if (aligned && c >= 64 && c <= 2048 && (c & (c - 1)) == 0) {
        auto go = [&](auto lc, auto vc) {
            constexpr int L = decltype(lc)::value, V = decltype(vc)::value, R = 64 / L;
            const dim3 grid((unsigned)ceil_div(n, 4 * R)), block(256);
            TSP_DT_SWITCH(x_dtype, XD, TSP_DT_SWITCH(out_dtype, OD,
                hipLaunchKernelGGL((k_layer_norm_vec<XD, OD, L, V>), grid, block, 0, s, d_x, n, c,
                                   d_gamma, d_beta, eps, silu, d_out)));
        };
        using std::integral_constant;
        switch (c) {
            case 64: go(integral_constant<int, 16>{}, integral_constant<int, 1>{}); break;
            case 128: go(integral_constant<int, 32>{}, integral_constant<int, 1>{}); break;
            case 256: go(integral_constant<int, 64>{}, integral_constant<int, 1>{}); break;
            case 512: go(integral_constant<int, 64>{}, integral_constant<int, 2>{}); break;
            case 1024: go(integral_constant<int, 64>{}, integral_constant<int, 4>{}); break;
            default: go(integral_constant<int, 64>{}, integral_constant<int, 8>{}); break;
        }
    } else {
        const dim3 grid((unsigned)ceil_div(n, 4)), block(256);
        TSP_DT_SWITCH(x_dtype, XD, TSP_DT_SWITCH(out_dtype, OD,
            hipLaunchKernelGGL((k_layer_norm<XD, OD>), grid, block, 0, s, d_x, n, c, d_gamma,
                               d_beta, eps, silu, d_out)));
    }
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
    if (cout % 4 == 0 && !(reinterpret_cast<uintptr_t>(d_h) % 16 || reinterpret_cast<uintptr_t>(d_out) % 16)) {
        TSP_DT_SWITCH(dtype, D, hipLaunchKernelGGL((k_c2s_gather_vec<D>), dim3(grid_for(m * cout / 4)),
                                                   dim3(256), 0, s, d_h, d_gidx, m, cout, d_out));
    } else {
        TSP_DT_SWITCH(dtype, D, hipLaunchKernelGGL((k_c2s_gather<D>), dim3(grid_for(m * cout)),
                                                   dim3(256), 0, s, d_h, d_gidx, m, cout, d_out));
    }
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
    if (rep % 4 == 0 && reinterpret_cast<uintptr_t>(d_acc) % 16 == 0) {
        TSP_DT_SWITCH(x_dtype, XD, TSP_DT_SWITCH(acc_dtype, AD,
            hipLaunchKernelGGL((k_c2s_skip_add_vec<XD, AD>), dim3(grid_for(m * cout / 4)), dim3(256), 0, s,
                               d_x, d_gidx, m, kb, rep, d_acc)));
    } else {
        TSP_DT_SWITCH(x_dtype, XD, TSP_DT_SWITCH(acc_dtype, AD,
            hipLaunchKernelGGL((k_c2s_skip_add<XD, AD>), dim3(grid_for(m * cout)), dim3(256), 0, s,
                               d_x, d_gidx, m, kb, rep, d_acc)));
    }
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
