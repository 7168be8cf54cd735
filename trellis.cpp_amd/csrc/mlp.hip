// The ConvNeXt block's MLP in one kernel (tsp_convnext_mlp): y = x + b2 + W2 . silu(W0 . xn + b0),
// C = 128 (4C = 512 hidden units).
//
// Replaces the two mul_mats of sparse_convnext (sparse.cpp:126-134: mlp.0, SiLU, mlp.2, + x), whose
// [N, 4C] hidden layer would otherwise go to HBM and back. Weight-stationary: one workgroup per CU,
// 8 waves (two per SIMD); wave w keeps hidden units 64 w .. 64 w + 63 of both weight matrices in
// its registers for the whole launch (W0's 64 x 128 and W2's 128 x 64 slices: 128 registers a
// lane), and the workgroup walks 32-row blocks of the input:
//  * the block's normalised rows are staged in LDS (loaded one block ahead), and each wave reads
//    them as the B operand of its 2 x 8 MFMAs H^T = W0_w . xn^T + b0 (32 hidden units x 32 rows a
//    tile, the bias as the accumulators' initial value);
//  * SiLU and rounding to the input's 16-bit type (as the two-GEMM path stores its hidden layer)
//    happen in the accumulator registers, which then ARE the A operand of the second product (a
//    lane holds 8 hidden units of one row: the second product's k steps take the hidden units in
//    that order, and W2 is packed to match), so the hidden layer never leaves the wave;
//  * each wave's Y_w = H_w . W2_w^T (32 rows x 128 columns, f32) goes to LDS, and after a barrier
//    each wave sums a 16-row x 32-column part over the 8 waves and stores y = sum + b2 + x.
// HBM sees xn (16-bit), x and y (f32) once; the weights are read once per workgroup. The SiLU's
// exponential and reciprocal over 4C values a row cost about as much issue time as the MFMAs:
// the two waves of a SIMD overlap one's VALU work with the other's products.
#include "conv_internal.hpp"

namespace tsp {
namespace {

constexpr int MLP_C = 128, MLP_H = 4 * MLP_C;
constexpr int MLP_W = 8, MLP_NT = 64 * MLP_W;   // 8 waves, two a SIMD
constexpr int MLP_XS = MLP_C + 8;   // LDS row stride of a staged row (16-bit values)

// [R][K] 16-bit, row-major -> [R/32][K/16][64 lanes][8]: lane l of block (r, k) holds row
// 32 r + l % 32, columns 16 k + 8 (l / 32) .. + 7 (the A operand of v_mfma_f32_32x32x16 for W0)
__global__ void k_mat_pack(const uint16_t* __restrict__ w, int R, int K, uint16_t* __restrict__ packed) {
    const int64_t blk = blockIdx.x;
    const int kb = (int)(blk % (K / 16)), rb = (int)(blk / (K / 16));
    const int lane = threadIdx.x;
    reinterpret_cast<u32x4_t*>(packed)[blk * 64 + lane] =
        *reinterpret_cast<const u32x4_t*>(w + (int64_t)(rb * 32 + (lane & 31)) * K + kb * 16 + (lane >> 5) * 8);
}

// The same blocks for W2 (the B operand of the second product) with each k step's 16 columns
// (hidden units) taken in the order the first product's accumulator holds them: lane l holds
// row 32 r + l % 32, columns 16 k + 4 (l / 32) + (0..3), then 16 k + 8 + 4 (l / 32) + (0..3).
__global__ void k_mat_pack_hidden(const uint16_t* __restrict__ w, int R, int K, uint16_t* __restrict__ packed) {
    const int64_t blk = blockIdx.x;
    const int kb = (int)(blk % (K / 16)), rb = (int)(blk / (K / 16));
    const int lane = threadIdx.x;
    const uint16_t* src = w + (int64_t)(rb * 32 + (lane & 31)) * K + kb * 16 + (lane >> 5) * 4;
    const uint2 lo = *reinterpret_cast<const uint2*>(src), hi = *reinterpret_cast<const uint2*>(src + 8);
    reinterpret_cast<u32x4_t*>(packed)[blk * 64 + lane] = u32x4_t{lo.x, lo.y, hi.x, hi.y};
}

// two values rounded to the 16-bit type, the first in the low half
template <bool BF16>
__device__ __forceinline__ uint32_t pack16x2(float lo, float hi) {
    if constexpr (BF16) return f32x2_to_bf16x2_bits(lo, hi);
    else return (uint32_t)f32_to_f16_bits(lo) | ((uint32_t)f32_to_f16_bits(hi) << 16);
}
// A buffer resource over `bytes` bytes from `base`: loads past the end return 0 and stores past
// it are dropped, which is how the last, partial row block is handled.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t span_rsrc(const void* base, int bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, bytes, 0x00020000);
}

// SiLU with a hardware reciprocal (the value is rounded to 16 bits next)
__device__ __forceinline__ float silu(float v) { return v * __builtin_amdgcn_rcpf(1.f + __expf(-v)); }

template <bool BF16>
__global__ __launch_bounds__(MLP_NT) __attribute__((amdgpu_waves_per_eu(2, 2)))
void k_mlp_ws(const uint16_t* __restrict__ xn, int64_t n, const uint16_t* __restrict__ pw0,
              const float* __restrict__ b0, const uint16_t* __restrict__ pw2, const float* __restrict__ b2,
              const float* x, float* y, uint16_t* y16, bool y16_bf16) {   // (y may be x: not restrict)
    __shared__ __attribute__((aligned(16))) uint16_t sX[2][32 * MLP_XS];   // staged rows, two blocks
    __shared__ f32x4_t sY[MLP_W * 4 * 4 * 64];                              // [wave][col block][j][lane]
    __shared__ __attribute__((aligned(16))) float sB0[MLP_H];
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int r32 = lane & 31, g = lane >> 5;
    const int64_t nrb = (n + 31) / 32;

    // this wave's weights: W0 hidden blocks 2 w + hb (A operands, 8 k steps over the channels);
    // W2 column blocks cb over hidden k steps 4 w .. 4 w + 3 (B operands)
    u32x4_t w0f[2][8], w2f[4][4];
#pragma unroll
    for (int hb = 0; hb < 2; ++hb)
#pragma unroll
        for (int ks = 0; ks < 8; ++ks)
            w0f[hb][ks] = *reinterpret_cast<const u32x4_t*>(pw0 + ((int64_t)((2 * wave + hb) * 8 + ks) * 64 + lane) * 8);
#pragma unroll
    for (int cb = 0; cb < 4; ++cb)
#pragma unroll
        for (int k = 0; k < 4; ++k)
            w2f[cb][k] = *reinterpret_cast<const u32x4_t*>(pw2 + ((int64_t)(cb * (MLP_H / 16) + 4 * wave + k) * 64 + lane) * 8);
    for (int i = tid; i < MLP_H; i += MLP_NT) sB0[i] = b0 ? b0[i] : 0.f;
    // the outputs this lane sums and stores: column block w / 2, rows 8 j + 4 g + t for
    // j = 2 (w % 2) + (0, 1)
    const int col = 32 * (wave >> 1) + r32, j0 = 2 * (wave & 1);
    const float bb2 = b2 ? b2[col] : 0.f;

    // Global accesses go through buffer resources spanning one row block (rows past n, and blocks
    // past the last, read as zeros and are not stored: an output row depends on its own input row
    // only). The staged rows: 32 rows x 128 channels = 512 pieces of 16 bytes, one a thread.
    const int xr_r = tid >> 4, xr_c = (tid & 15) * 8;
    auto block_rows = [&](int64_t rb) { return (int)max<int64_t>(0, min<int64_t>(32, n - rb * 32)); };
    auto load_x = [&](int64_t rb) {
        const __amdgpu_buffer_rsrc_t r = span_rsrc(xn + rb * 32 * MLP_C, block_rows(rb) * MLP_C * 2);
        return __builtin_bit_cast(u32x4_t, __builtin_amdgcn_raw_buffer_load_b128(r, (xr_r * MLP_C + xr_c) * 2, 0, 0));
    };
    // byte offset in a block of this lane's output e: row 8 j + 4 g + t (j = j0 + e / 4, t = e % 4)
    auto out_off = [&](int e) { return ((8 * (j0 + (e >> 2)) + 4 * g + (e & 3)) * MLP_C + col) * 4; };
    int64_t rb = blockIdx.x;
    if (rb < nrb) *reinterpret_cast<u32x4_t*>(&sX[0][xr_r * MLP_XS + xr_c]) = load_x(rb);
    __syncthreads();

    for (int it = 0; rb < nrb; ++it, rb += gridDim.x) {
        const int buf = it & 1;
        const int64_t nxt = rb + gridDim.x;
        const int span = block_rows(rb) * MLP_C * 4;   // bytes of x and y in this block
        const u32x4_t xr = load_x(nxt);                  // the next block's rows
        // this block's inputs to add (needed last)
        const __amdgpu_buffer_rsrc_t xres = span_rsrc(x + rb * 32 * MLP_C, span);
        float xv[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) xv[e] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(xres, out_off(e), 0, 0));
        __builtin_amdgcn_sched_barrier(0);               // (issued here, a whole block ahead of their use)
        // xn^T as B operands: lane l holds row r32, channels 16 ks + 8 g .. + 7
        u32x4_t xf[8];
#pragma unroll
        for (int ks = 0; ks < 8; ++ks) xf[ks] = *reinterpret_cast<const u32x4_t*>(&sX[buf][r32 * MLP_XS + ks * 16 + g * 8]);
        // H^T = W0 . xn^T + b0, the bias as the accumulators' initial value: element 4 i + t is
        // hidden unit 64 w + 32 hb + 8 i + 4 g + t of row r32
        f32x16_t a1[2];
#pragma unroll
        for (int hb = 0; hb < 2; ++hb)
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const f32x4_t bb = *reinterpret_cast<const f32x4_t*>(&sB0[64 * wave + 32 * hb + 8 * i + 4 * g]);
#pragma unroll
                for (int t = 0; t < 4; ++t) a1[hb][4 * i + t] = bb[t];
            }
#pragma unroll
        for (int ks = 0; ks < 8; ++ks)
#pragma unroll
            for (int hb = 0; hb < 2; ++hb) a1[hb] = mfma32x32x16<BF16>(w0f[hb][ks], xf[ks], a1[hb]);
        // SiLU, rounded: the A operands of the second product, hidden units in the accumulator's
        // order (elements 8 kk .. 8 kk + 7 for k step kk)
        u32x4_t hf[2][2];
#pragma unroll
        for (int hb = 0; hb < 2; ++hb)
#pragma unroll
            for (int h = 0; h < 8; ++h)
                hf[hb][h >> 2][h & 3] = pack16x2<BF16>(silu(a1[hb][2 * h]), silu(a1[hb][2 * h + 1]));
        // Y_w = H_w . W2_w^T, two column blocks at a time
        f32x16_t acc[2];
        __syncthreads();   // every wave has summed the previous block's partial products
#pragma unroll
        for (int cp = 0; cp < 2; ++cp) {
#pragma unroll
            for (int q = 0; q < 2; ++q)
#pragma unroll
                for (int e = 0; e < 16; ++e) acc[q][e] = 0.f;
#pragma unroll
            for (int k = 0; k < 4; ++k)
#pragma unroll
                for (int q = 0; q < 2; ++q) acc[q] = mfma32x32x16<BF16>(hf[k >> 1][k & 1], w2f[2 * cp + q][k], acc[q]);
#pragma unroll
            for (int q = 0; q < 2; ++q)
#pragma unroll
                for (int j = 0; j < 4; ++j)
                    sY[((wave * 4 + 2 * cp + q) * 4 + j) * 64 + lane] =
                        f32x4_t{acc[q][4 * j], acc[q][4 * j + 1], acc[q][4 * j + 2], acc[q][4 * j + 3]};
        }
        *reinterpret_cast<u32x4_t*>(&sX[buf ^ 1][xr_r * MLP_XS + xr_c]) = xr;
        __syncthreads();
        // this lane's outputs summed over the 8 waves
        float yv[8];
#pragma unroll
        for (int jj = 0; jj < 2; ++jj) {
            const int j = j0 + jj;
            f32x4_t s = sY[((0 * 4 + (wave >> 1)) * 4 + j) * 64 + lane];
#pragma unroll
            for (int w = 1; w < MLP_W; ++w) {
                const f32x4_t p = sY[((w * 4 + (wave >> 1)) * 4 + j) * 64 + lane];
                s[0] += p[0];
                s[1] += p[1];
                s[2] += p[2];
                s[3] += p[3];
            }
#pragma unroll
            for (int t = 0; t < 4; ++t) yv[4 * jj + t] = s[t] + bb2 + xv[4 * jj + t];
        }
        const __amdgpu_buffer_rsrc_t yres = span_rsrc(y + rb * 32 * MLP_C, span);
#pragma unroll
        for (int e = 0; e < 8; ++e) __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(uint32_t, yv[e]), yres, out_off(e), 0, 0);
        if (y16) {
            // the next conv's 16-bit input: y rounded as a rounding pass over it would
            const __amdgpu_buffer_rsrc_t hres = span_rsrc(y16 + rb * 32 * MLP_C, span / 2);
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                const uint16_t h = y16_bf16 ? f32_to_bf16_bits(yv[e]) : f32_to_f16_bits(yv[e]);
                __builtin_amdgcn_raw_buffer_store_b16(h, hres, out_off(e) / 2, 0, 0);
            }
        }
    }
}

}  // namespace

size_t mlp_packed_bytes(int c) { return (size_t)2 * 4 * c * c * 2; }

int mlp_pack(const void* w0, const void* w2, int c, void* packed, hipStream_t s) {
    auto* p = static_cast<uint16_t*>(packed);
    hipLaunchKernelGGL(k_mat_pack, dim3((unsigned)((4 * c / 32) * (c / 16))), dim3(64), 0, s,
                       static_cast<const uint16_t*>(w0), 4 * c, c, p);
    TSP_CHECK_LAUNCH();
    hipLaunchKernelGGL(k_mat_pack_hidden, dim3((unsigned)((c / 32) * (4 * c / 16))), dim3(64), 0, s,
                       static_cast<const uint16_t*>(w2), c, 4 * c, p + (size_t)4 * c * c);
    TSP_CHECK_LAUNCH();
    return TSP_OK;
}

bool mlp_fused_eligible(int dt, int c, const void* xn, const void* packed, const float* x, const float* y) {
    auto al = [](const void* p, uintptr_t a) { return (reinterpret_cast<uintptr_t>(p) & (a - 1)) == 0; };
    return (dt == TSP_BF16 || dt == TSP_F16) && c == MLP_C && al(xn, 16) && al(packed, 16) && al(x, 4) &&
           al(y, 4);
}

int mlp_fused(const void* xn, int dt, int64_t n, int c, const void* packed, const float* b0, const float* b2,
              const float* x, float* y, hipStream_t s, void* y16, int y16_dtype) {
    if (n == 0) return TSP_OK;
    if (c != MLP_C) return TSP_ERR_UNSUPPORTED;
    // one workgroup per CU (the staged rows and partial products fill its LDS), each walking row
    // blocks with a stride of the grid
    static int cus[64] = {0};
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) dev = 0;
    if (!cus[dev] && (hipDeviceGetAttribute(&cus[dev], hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
                      cus[dev] <= 0))
        cus[dev] = 256;
    const unsigned grid = (unsigned)std::min<int64_t>((n + 31) / 32, cus[dev]);
    const auto* a = static_cast<const uint16_t*>(xn);
    const auto* p0 = static_cast<const uint16_t*>(packed);
    const auto* p2 = p0 + (size_t)4 * c * c;
    if (dt == TSP_BF16)
        hipLaunchKernelGGL(k_mlp_ws<true>, dim3(grid), dim3(MLP_NT), 0, s, a, n, p0, b0, p2, b2, x, y,
                           static_cast<uint16_t*>(y16), y16_dtype == TSP_BF16);
    else
        hipLaunchKernelGGL(k_mlp_ws<false>, dim3(grid), dim3(MLP_NT), 0, s, a, n, p0, b0, p2, b2, x, y,
                           static_cast<uint16_t*>(y16), y16_dtype == TSP_BF16);
    TSP_CHECK_LAUNCH();
    return TSP_OK;
}

}  // namespace tsp

using namespace tsp;

extern "C" size_t tsp_convnext_mlp_packed_bytes(int c) { return c > 0 ? mlp_packed_bytes(c) : 0; }

extern "C" int tsp_convnext_mlp_pack(const void* d_w0, const void* d_w2, int dtype, int c, void* d_packed,
                                     void* stream) {
    clear_error();
    TSP_REQUIRE(dtype == TSP_BF16 || dtype == TSP_F16, TSP_ERR_UNSUPPORTED,
                "tsp_convnext_mlp_pack: needs bf16 or f16 weights, got dtype %d", dtype);
    TSP_REQUIRE(c == MLP_C, TSP_ERR_UNSUPPORTED, "tsp_convnext_mlp_pack: C=%d (the fused MLP is for C = 128)", c);
    TSP_REQUIRE(d_w0 && d_w2 && d_packed, TSP_ERR_INVALID, "tsp_convnext_mlp_pack: null pointer");
    auto al = [](const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; };
    TSP_REQUIRE(al(d_w0) && al(d_w2) && al(d_packed), TSP_ERR_INVALID,
                "tsp_convnext_mlp_pack: buffers must be 16-byte aligned");
    return mlp_pack(d_w0, d_w2, c, d_packed, as_stream(stream));
}

extern "C" int tsp_convnext_mlp(const void* d_xn, int dtype, int64_t n, int c, const void* d_packed,
                                const float* d_b0, const float* d_b2, const float* d_x, float* d_out,
                                void* stream) {
    clear_error();
    TSP_REQUIRE(n >= 0 && n < (int64_t)INT32_MAX, TSP_ERR_INVALID, "tsp_convnext_mlp: n=%lld out of range",
                (long long)n);
    TSP_REQUIRE(dtype == TSP_BF16 || dtype == TSP_F16, TSP_ERR_UNSUPPORTED,
                "tsp_convnext_mlp: needs bf16 or f16 input and weights, got dtype %d", dtype);
    TSP_REQUIRE(c == MLP_C, TSP_ERR_UNSUPPORTED, "tsp_convnext_mlp: C=%d (the fused MLP is for C = 128)", c);
    if (n == 0) return TSP_OK;
    TSP_REQUIRE(d_xn && d_packed && d_x && d_out, TSP_ERR_INVALID, "tsp_convnext_mlp: null pointer");
    TSP_REQUIRE(static_cast<const void*>(d_out) != d_xn, TSP_ERR_INVALID, "tsp_convnext_mlp: out aliases xn");
    TSP_REQUIRE(mlp_fused_eligible(dtype, c, d_xn, d_packed, d_x, d_out), TSP_ERR_INVALID,
                "tsp_convnext_mlp: xn and the packed weights must be 16-byte aligned, x and out 4-byte");
    return mlp_fused(d_xn, dtype, n, c, d_packed, d_b0, d_b2, d_x, d_out, as_stream(stream));
}
