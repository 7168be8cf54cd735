// Elementwise kernels of the graph runtime: broadcast add / mul, SiLU, dtype conversion and
// row gather. All are grid-stride loops over contiguous tensors; they are memory-bound and
// sized for HBM streaming (256 threads, at most 64K workgroups).
#include <hip/hip_bf16.h>
#include <hip/hip_fp16.h>

#include <algorithm>

#include "runtime.hpp"

namespace tgr {
namespace {

constexpr int kThreads = 256;

inline unsigned grid_for(int64_t total) {
    return (unsigned)std::max<int64_t>(1, std::min<int64_t>((total + kThreads - 1) / kThreads, 65536));
}

template <int DT> struct Io;
// ld / st: element i of a buffer of the type; rnd: v rounded to the type (as a float)
template <> struct Io<TSP_F32> {
    static __device__ float ld(const void* p, int64_t i) { return static_cast<const float*>(p)[i]; }
    static __device__ void st(void* p, int64_t i, float v) { static_cast<float*>(p)[i] = v; }
    static __device__ float rnd(float v) { return v; }
};
template <> struct Io<TSP_F16> {
    static __device__ float ld(const void* p, int64_t i) {
        return __half2float(static_cast<const __half*>(p)[i]);
    }
    static __device__ void st(void* p, int64_t i, float v) {
        static_cast<__half*>(p)[i] = __float2half_rn(v);
    }
    static __device__ float rnd(float v) { return __half2float(__float2half_rn(v)); }
};
template <> struct Io<TSP_BF16> {
    static __device__ float ld(const void* p, int64_t i) {
        const uint32_t b = (uint32_t)static_cast<const uint16_t*>(p)[i] << 16;
        return __uint_as_float(b);
    }
    static __device__ void st(void* p, int64_t i, float v) {
        // round to nearest even; NaN stays a quiet NaN
        const uint32_t u = __float_as_uint(v);
        uint16_t r;
        if ((u & 0x7fffffffu) > 0x7f800000u) r = (uint16_t)((u >> 16) | 0x40u);
        else r = (uint16_t)((u + 0x7fffu + ((u >> 16) & 1u)) >> 16);
        static_cast<uint16_t*>(p)[i] = r;
    }
    static __device__ float rnd(float v) {
        const uint32_t u = __float_as_uint(v);
        if ((u & 0x7fffffffu) > 0x7f800000u) return v;
        return __uint_as_float((u + 0x7fffu + ((u >> 16) & 1u)) & 0xffff0000u);
    }
};

struct Shape4 {
    int64_t ne[4];
};

// out[i] = a[i] (op) b[broadcast(i)]
template <int ADT, int BDT, bool MUL>
__global__ void k_binary(const void* __restrict__ a, const void* __restrict__ b,
                         float* __restrict__ out, Shape4 sa, Shape4 sb, int64_t total) {
    for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < total;
         i += (int64_t)gridDim.x * blockDim.x) {
        int64_t r = i, bi = 0, stride = 1;
#pragma unroll
        for (int d = 0; d < 4; ++d) {
            const int64_t c = r % sa.ne[d];
            r /= sa.ne[d];
            bi += (c % sb.ne[d]) * stride;
            stride *= sb.ne[d];
        }
        const float x = Io<ADT>::ld(a, i), y = Io<BDT>::ld(b, bi);
        out[i] = MUL ? x * y : x + y;
    }
}

// b broadcast along rows only (b has a->ne[0] elements): the common bias / scale case
template <int ADT, int BDT, bool MUL>
__global__ void k_binary_row(const void* __restrict__ a, const void* __restrict__ b,
                             float* __restrict__ out, int64_t ne0, int64_t total) {
    for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < total;
         i += (int64_t)gridDim.x * blockDim.x) {
        const float x = Io<ADT>::ld(a, i), y = Io<BDT>::ld(b, i % ne0);
        out[i] = MUL ? x * y : x + y;
    }
}

__global__ void k_silu(const float* __restrict__ x, float* __restrict__ y, int64_t n) {
    for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < n;
         i += (int64_t)gridDim.x * blockDim.x) {
        const float v = x[i];
        y[i] = v / (1.0f + expf(-v));
    }
}

template <int YDT>
__global__ void k_silu_to(const float* __restrict__ x, void* __restrict__ y, int64_t n) {
    for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < n;
         i += (int64_t)gridDim.x * blockDim.x) {
        const float v = x[i];
        Io<YDT>::st(y, i, v / (1.0f + expf(-v)));
    }
}

template <int XDT>
__global__ void k_add_inplace(float* __restrict__ y, const void* __restrict__ x, int64_t n) {
    for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < n;
         i += (int64_t)gridDim.x * blockDim.x)
        y[i] += Io<XDT>::ld(x, i);
}

template <int XDT, int YDT>
__global__ void k_convert(const void* __restrict__ x, void* __restrict__ y, int64_t n) {
    for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < n;
         i += (int64_t)gridDim.x * blockDim.x)
        Io<YDT>::st(y, i, Io<XDT>::ld(x, i));
}

// f32 -> f16 / bf16, four elements per thread (16-byte loads, 8-byte stores). bf16 through the
// packed hardware conversion, which rounds to nearest even exactly as Io<TSP_BF16>::st does.
template <int YDT>
__global__ void k_convert_f32_x4(const float4* __restrict__ x, uint2* __restrict__ y, int64_t n4) {
    typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
    typedef float f32x2 __attribute__((ext_vector_type(2)));
    for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < n4;
         i += (int64_t)gridDim.x * blockDim.x) {
        const float4 v = x[i];
        uint32_t lo, hi;
        if constexpr (YDT == TSP_BF16) {
            lo = __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2{v.x, v.y}, bf16x2));
            hi = __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2{v.z, v.w}, bf16x2));
        } else {
            lo = (uint32_t)__half_as_ushort(__float2half_rn(v.x)) | ((uint32_t)__half_as_ushort(__float2half_rn(v.y)) << 16);
            hi = (uint32_t)__half_as_ushort(__float2half_rn(v.z)) | ((uint32_t)__half_as_ushort(__float2half_rn(v.w)) << 16);
        }
        y[i] = uint2{lo, hi};
    }
}

template <int DT>
__global__ void k_get_rows(const void* __restrict__ a, int64_t rows, const int32_t* __restrict__ idx,
                           int64_t n_idx, int64_t k, float* __restrict__ out) {
    const int64_t total = n_idx * k;
    for (int64_t e = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; e < total;
         e += (int64_t)gridDim.x * blockDim.x) {
        const int64_t r = e / k, c = e % k;
        const int64_t src = idx[r];
        out[e] = (src >= 0 && src < rows) ? Io<DT>::ld(a, src * k + c) : 0.0f;
    }
}

__global__ void k_get_rows_i32(const int32_t* __restrict__ a, int64_t rows,
                               const int32_t* __restrict__ idx, int64_t n_idx, int64_t k,
                               int32_t* __restrict__ out) {
    const int64_t total = n_idx * k;
    for (int64_t e = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; e < total;
         e += (int64_t)gridDim.x * blockDim.x) {
        const int64_t r = e / k, c = e % k;
        const int64_t src = idx[r];
        out[e] = (src >= 0 && src < rows) ? a[src * k + c] : 0;
    }
}

template <bool MUL>
hipError_t binary_typed(const ggml_tensor* a, const ggml_tensor* b, float* out, hipStream_t s) {
    const int64_t total = ggml_nelements(a);
    const bool row = ggml_nelements(b) == b->ne[0] && b->ne[0] == a->ne[0];
    const int ad = tsp_dtype_of(a->type), bd = tsp_dtype_of(b->type);
    Shape4 sa{{a->ne[0], a->ne[1], a->ne[2], a->ne[3]}}, sb{{b->ne[0], b->ne[1], b->ne[2], b->ne[3]}};
    const dim3 g(grid_for(total)), blk(kThreads);
#define TGR_BIN(AD, BD)                                                                        \
    if (ad == AD && bd == BD) {                                                                \
        if (row)                                                                               \
            hipLaunchKernelGGL((k_binary_row<AD, BD, MUL>), g, blk, 0, s, a->data, b->data, out, \
                               a->ne[0], total);                                               \
        else                                                                                   \
            hipLaunchKernelGGL((k_binary<AD, BD, MUL>), g, blk, 0, s, a->data, b->data, out, sa, \
                               sb, total);                                                     \
        return hipGetLastError();                                                              \
    }
    TGR_BIN(TSP_F32, TSP_F32)
    TGR_BIN(TSP_F32, TSP_F16)
    TGR_BIN(TSP_F16, TSP_F32)
    TGR_BIN(TSP_F16, TSP_F16)
#undef TGR_BIN
    return hipErrorInvalidValue;
}

// The decoders' head (shape_decoder.cpp:63-77, 116): out[r][o] = bias[o] + sum_i LN(x[r])[i] W[o][i]
// with LN the row LayerNorm of eps without affine, for co <= 8 outputs. L lanes hold a row, each V
// groups of 4 channels (ci = 4 L V); the row is normalised in registers and every output is a
// reduction over the row's lanes, so x is read once and nothing else is written. Waves walk the
// rows with a grid stride, keeping their weights in registers.
constexpr int kHeadMaxCo = 8;

// DPP lane moves within a row of 16 lanes: lane ^ 1, lane ^ 2, 7 - lane within each 8, 15 - lane.
constexpr int kDppXor1 = 0xB1, kDppXor2 = 0x4E, kDppHalfMirror = 0x141, kDppMirror = 0x140;
template <int CTRL>
__device__ __forceinline__ float dpp(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xF, 0xF, false));
}
// Sum over the 16 lanes of a DPP row; every lane ends with the same value.
__device__ __forceinline__ float row16_sum(float v) {
    v += dpp<kDppXor1>(v);
    v += dpp<kDppXor2>(v);
    v += dpp<kDppHalfMirror>(v);
    v += dpp<kDppMirror>(v);
    return v;
}
template <int WDT, int L, int V>
__global__ __launch_bounds__(256) void k_norm_linear(const float* __restrict__ x, int64_t n, float eps,
                                                     const void* __restrict__ w, const float* __restrict__ bias,
                                                     int co, float* __restrict__ out) {
    constexpr int R = 64 / L, C = 4 * L * V;
    const int lane = threadIdx.x & 63, sub = lane % L;
    float wv[kHeadMaxCo][V][4];
#pragma unroll
    for (int o = 0; o < kHeadMaxCo; ++o)
#pragma unroll
        for (int j = 0; j < V; ++j)
#pragma unroll
            for (int e = 0; e < 4; ++e)
                wv[o][j][e] = o < co ? Io<WDT>::ld(w, (int64_t)o * C + (j * L + sub) * 4 + e) : 0.f;
    constexpr int NO = (kHeadMaxCo + L - 1) / L;   // outputs per lane: o = k L + sub
    float bo[NO];
#pragma unroll
    for (int k = 0; k < NO; ++k) bo[k] = k * L + sub < co ? bias[k * L + sub] : 0.f;
    const int o16 = (sub & 8 ? 4 : 0) + (sub & 4 ? 2 : 0) + (sub & 2 ? 1 : 0);   // L == 16 path
    const float bo16 = o16 < co ? bias[o16] : 0.f;
    const int64_t waves = (int64_t)gridDim.x * 4;
    // The next row group's x is loaded before this group's reductions, so a load is always in
    // flight while the lanes shuffle.
    auto load = [&](int64_t g, float4 (&t)[V]) {
        const int64_t row = g * R + lane / L;
        const float* xr = x + (row < n ? row : 0) * C;
#pragma unroll
        for (int j = 0; j < V; ++j) t[j] = *reinterpret_cast<const float4*>(xr + (j * L + sub) * 4);
    };
    int64_t g = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    float4 nxt[V];
    load(g, nxt);
    for (; g * R < n; g += waves) {
        const int64_t row = g * R + lane / L;
        const bool live = row < n;
        float v[V][4];
#pragma unroll
        for (int j = 0; j < V; ++j) {
            v[j][0] = nxt[j].x; v[j][1] = nxt[j].y; v[j][2] = nxt[j].z; v[j][3] = nxt[j].w;
        }
        load(g + waves, nxt);
        float sum = 0.f;
#pragma unroll
        for (int j = 0; j < V; ++j)
#pragma unroll
            for (int e = 0; e < 4; ++e) sum += v[j][e];
        if constexpr (L == 16) {
            sum = row16_sum(sum);
        } else {
#pragma unroll
            for (int off = L / 2; off > 0; off >>= 1) sum += __shfl_xor(sum, off, 64);
        }
        const float mean = sum / (float)C;
        float q = 0.f;
#pragma unroll
        for (int j = 0; j < V; ++j)
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                v[j][e] -= mean;
                q += v[j][e] * v[j][e];
            }
        if constexpr (L == 16) {
            q = row16_sum(q);
        } else {
#pragma unroll
            for (int off = L / 2; off > 0; off >>= 1) q += __shfl_xor(q, off, 64);
        }
        const float rstd = 1.0f / sqrtf(q / (float)C + eps);
        // the normalised row rounded to the weights' type, as ggml's mul_mat rounds its input
#pragma unroll
        for (int j = 0; j < V; ++j)
#pragma unroll
            for (int e = 0; e < 4; ++e) v[j][e] = Io<WDT>::rnd(v[j][e] * rstd);
        float acc[kHeadMaxCo];
#pragma unroll
        for (int o = 0; o < kHeadMaxCo; ++o) {
            acc[o] = 0.f;
#pragma unroll
            for (int j = 0; j < V; ++j)
#pragma unroll
                for (int e = 0; e < 4; ++e) acc[o] += v[j][e] * wv[o][j][e];
        }
        if constexpr (L == 16) {
            // Reduce-scatter of the 8 sums over the row's 16 lanes in 8 DPP moves: each step
            // pairs lanes that differ in one of bits 3, 2, 1 of sub, and the lane keeps the half
            // of its sums that bit selects. Lanes sub and sub ^ 1 end with the total of output
            // o = 4 b3 + 2 b2 + b1; the even one stores it.
            const bool h3 = sub & 8, h2 = sub & 4, h1 = sub & 2;
            float a4[4], a2[2];
#pragma unroll
            for (int k = 0; k < 4; ++k)
                a4[k] = (h3 ? acc[4 + k] : acc[k]) + dpp<kDppMirror>(h3 ? acc[k] : acc[4 + k]);
#pragma unroll
            for (int k = 0; k < 2; ++k)
                a2[k] = (h2 ? a4[2 + k] : a4[k]) + dpp<kDppHalfMirror>(h2 ? a4[k] : a4[2 + k]);
            float r = (h1 ? a2[1] : a2[0]) + dpp<kDppXor2>(h1 ? a2[0] : a2[1]);
            r += dpp<kDppXor1>(r);
            const int o = (h3 ? 4 : 0) + (h2 ? 2 : 0) + (h1 ? 1 : 0);
            if (live && !(sub & 1) && o < co) out[row * co + o] = r + bo16;
            continue;
        }
#pragma unroll
        for (int o = 0; o < kHeadMaxCo; ++o) {
#pragma unroll
            for (int off = L / 2; off > 0; off >>= 1) acc[o] += __shfl_xor(acc[o], off, 64);
        }
        // every lane of the row holds every sum: lane sub of the row writes outputs k L + sub
#pragma unroll
        for (int k = 0; k < NO; ++k) {
            const int o = k * L + sub;
            float r = 0.f;
#pragma unroll
            for (int i = 0; i < kHeadMaxCo; ++i)
                if (o == i) r = acc[i];
            if (live && o < co) out[row * co + o] = r + bo[k];
        }
    }
}

}  // namespace

hipError_t launch_norm_linear(const float* x, int64_t n, int ci, float eps, const void* w, int w_dtype,
                              const float* bias, int co, float* out, hipStream_t s) {
    if (co < 1 || co > kHeadMaxCo) return hipErrorInvalidValue;
    if (reinterpret_cast<uintptr_t>(x) % 16) return hipErrorInvalidValue;
    if (n == 0) return hipSuccess;
#define TGR_HEAD(WD, L, V)                                                                        \
    if (w_dtype == WD && ci == 4 * L * V) {                                                         \
        const int64_t rows_per_block = 4 * (64 / L);                                                \
        const dim3 g((unsigned)std::min<int64_t>((n + rows_per_block - 1) / rows_per_block, 4096)),   \
            blk(256);                                                                                \
        hipLaunchKernelGGL((k_norm_linear<WD, L, V>), g, blk, 0, s, x, n, eps, w, bias, co, out);   \
        return hipGetLastError();                                                                    \
    }
#define TGR_HEAD_W(L, V) TGR_HEAD(TSP_F32, L, V) TGR_HEAD(TSP_F16, L, V) TGR_HEAD(TSP_BF16, L, V)
    TGR_HEAD_W(4, 1)
    TGR_HEAD_W(8, 1)
    TGR_HEAD_W(16, 1)
    TGR_HEAD_W(32, 1)
    TGR_HEAD_W(64, 1)
    TGR_HEAD_W(64, 2)
    TGR_HEAD_W(64, 4)
#undef TGR_HEAD_W
#undef TGR_HEAD
    return hipErrorInvalidValue;
}

hipError_t launch_binary(int op_mul, const ggml_tensor* a, const ggml_tensor* b, float* out,
                         hipStream_t s) {
    if (ggml_nelements(a) == 0) return hipSuccess;
    return op_mul ? binary_typed<true>(a, b, out, s) : binary_typed<false>(a, b, out, s);
}

hipError_t launch_silu(const float* x, float* y, int64_t n, hipStream_t s) {
    if (n == 0) return hipSuccess;
    hipLaunchKernelGGL(k_silu, dim3(grid_for(n)), dim3(kThreads), 0, s, x, y, n);
    return hipGetLastError();
}

hipError_t launch_silu_to(const float* x, void* y, int yd, int64_t n, hipStream_t s) {
    if (n == 0) return hipSuccess;
    const dim3 g(grid_for(n)), blk(kThreads);
    switch (yd) {
        case TSP_F16: hipLaunchKernelGGL((k_silu_to<TSP_F16>), g, blk, 0, s, x, y, n); break;
        case TSP_BF16: hipLaunchKernelGGL((k_silu_to<TSP_BF16>), g, blk, 0, s, x, y, n); break;
        case TSP_F32: hipLaunchKernelGGL(k_silu, g, blk, 0, s, x, static_cast<float*>(y), n); break;
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

hipError_t launch_add_inplace(float* y, const void* x, int xd, int64_t n, hipStream_t s) {
    if (n == 0) return hipSuccess;
    const dim3 g(grid_for(n)), blk(kThreads);
    switch (xd) {
        case TSP_F32: hipLaunchKernelGGL((k_add_inplace<TSP_F32>), g, blk, 0, s, y, x, n); break;
        case TSP_F16: hipLaunchKernelGGL((k_add_inplace<TSP_F16>), g, blk, 0, s, y, x, n); break;
        case TSP_BF16: hipLaunchKernelGGL((k_add_inplace<TSP_BF16>), g, blk, 0, s, y, x, n); break;
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

hipError_t launch_convert(const void* x, int xd, void* y, int yd, int64_t n, hipStream_t s) {
    if (n == 0) return hipSuccess;
    const dim3 g(grid_for(n)), blk(kThreads);
    if (xd == TSP_F32 && (yd == TSP_BF16 || yd == TSP_F16) && n % 4 == 0 &&
        reinterpret_cast<uintptr_t>(x) % 16 == 0 && reinterpret_cast<uintptr_t>(y) % 8 == 0) {
        const dim3 g4(grid_for(n / 4));
        if (yd == TSP_BF16)
            hipLaunchKernelGGL(k_convert_f32_x4<TSP_BF16>, g4, blk, 0, s, static_cast<const float4*>(x),
                               static_cast<uint2*>(y), n / 4);
        else
            hipLaunchKernelGGL(k_convert_f32_x4<TSP_F16>, g4, blk, 0, s, static_cast<const float4*>(x),
                               static_cast<uint2*>(y), n / 4);
        return hipGetLastError();
    }
#define TGR_CVT(XD, YD)                                                                   \
    if (xd == XD && yd == YD) {                                                           \
        hipLaunchKernelGGL((k_convert<XD, YD>), g, blk, 0, s, x, y, n);                   \
        return hipGetLastError();                                                         \
    }
    TGR_CVT(TSP_F32, TSP_F16)
    TGR_CVT(TSP_F32, TSP_BF16)
    TGR_CVT(TSP_F16, TSP_F32)
    TGR_CVT(TSP_BF16, TSP_F32)
#undef TGR_CVT
    return hipErrorInvalidValue;
}

hipError_t launch_get_rows(const ggml_tensor* a, const int32_t* idx, int64_t n_idx, void* out,
                           hipStream_t s) {
    const int64_t k = a->ne[0], rows = a->ne[1];
    if (n_idx * k == 0) return hipSuccess;
    const dim3 g(grid_for(n_idx * k)), blk(kThreads);
    switch (a->type) {
        case GGML_TYPE_F32:
            hipLaunchKernelGGL((k_get_rows<TSP_F32>), g, blk, 0, s, a->data, rows, idx, n_idx, k,
                               static_cast<float*>(out));
            break;
        case GGML_TYPE_F16:
            hipLaunchKernelGGL((k_get_rows<TSP_F16>), g, blk, 0, s, a->data, rows, idx, n_idx, k,
                               static_cast<float*>(out));
            break;
        case GGML_TYPE_BF16:
            hipLaunchKernelGGL((k_get_rows<TSP_BF16>), g, blk, 0, s, a->data, rows, idx, n_idx, k,
                               static_cast<float*>(out));
            break;
        case GGML_TYPE_I32:
            hipLaunchKernelGGL(k_get_rows_i32, g, blk, 0, s, static_cast<const int32_t*>(a->data),
                               rows, idx, n_idx, k, static_cast<int32_t*>(out));
            break;
    }
    return hipGetLastError();
}

}  // namespace tgr
