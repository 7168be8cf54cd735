// Shared helpers for the sparse-voxel HIP library (gfx950 / CDNA4 only).
#pragma once
#include <hip/hip_runtime.h>
#include <hip/hip_bf16.h>
#include <hip/hip_fp16.h>

#include <cstdint>
#include <cstdio>
#include <string>

#include "trellis_sparse.h"

namespace tsp {

// ---- status ------------------------------------------------------------------------------
// The C ABI never throws: every entry point returns a tsp_status and leaves a message in a
// thread-local buffer readable through tsp_last_error().
void set_error(const char* fmt, ...);
void clear_error();

#define TSP_CHECK_HIP(expr)                                                                 \
    do {                                                                                    \
        hipError_t e_ = (expr);                                                             \
        if (e_ != hipSuccess) {                                                             \
            ::tsp::set_error("%s failed: %s (%s:%d)", #expr, hipGetErrorString(e_),        \
                             __FILE__, __LINE__);                                           \
            return TSP_ERR_HIP;                                                             \
        }                                                                                   \
    } while (0)

#define TSP_REQUIRE(cond, code, ...)                                                        \
    do {                                                                                    \
        if (!(cond)) {                                                                      \
            ::tsp::set_error(__VA_ARGS__);                                                  \
            return (code);                                                                  \
        }                                                                                   \
    } while (0)

// Checks the launch that was just issued.
#define TSP_CHECK_LAUNCH() TSP_CHECK_HIP(hipGetLastError())

inline size_t dtype_size(int dt) { return dt == TSP_F32 ? 4 : 2; }
inline bool dtype_valid(int dt) { return dt == TSP_F32 || dt == TSP_F16 || dt == TSP_BF16; }
inline hipStream_t as_stream(void* s) { return reinterpret_cast<hipStream_t>(s); }

// ---- element conversions -------------------------------------------------------------------
// bf16 and fp16 values are handled as raw 16-bit patterns in memory.
__device__ __forceinline__ float bf16_bits_to_f32(uint16_t b) {
    return __uint_as_float(static_cast<uint32_t>(b) << 16);
}
// Round to nearest even; NaN stays NaN with its sign and upper payload bits and the quiet bit
// forced. On gfx950 the conversion is v_cvt_pk_bf16_f32, two values per instruction; it gives
// exactly these bits for every one of the 2^32 float patterns (checked against the integer form
// u += 0x7fff + ((u >> 16) & 1), NaN -> (u >> 16) | 0x40).
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef float f32x2_t __attribute__((ext_vector_type(2)));
__device__ __forceinline__ uint32_t f32x2_to_bf16x2_bits(float lo, float hi) {
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2_t{lo, hi}, bf16x2_t));
}
__device__ __forceinline__ uint16_t f32_to_bf16_bits(float f) {
    return static_cast<uint16_t>(f32x2_to_bf16x2_bits(f, 0.f));
}
__device__ __forceinline__ float f16_bits_to_f32(uint16_t b) {
    return __half2float(__ushort_as_half(b));
}
__device__ __forceinline__ uint16_t f32_to_f16_bits(float f) {
    return __half_as_ushort(__float2half_rn(f));
}

template <int DT> struct Elem;
template <> struct Elem<TSP_F32> {
    using storage = float;
    __device__ __forceinline__ static float load(const storage* p, int64_t i) { return p[i]; }
    __device__ __forceinline__ static void store(storage* p, int64_t i, float v) { p[i] = v; }
};
template <> struct Elem<TSP_BF16> {
    using storage = uint16_t;
    __device__ __forceinline__ static float load(const storage* p, int64_t i) { return bf16_bits_to_f32(p[i]); }
    __device__ __forceinline__ static void store(storage* p, int64_t i, float v) { p[i] = f32_to_bf16_bits(v); }
};
template <> struct Elem<TSP_F16> {
    using storage = uint16_t;
    __device__ __forceinline__ static float load(const storage* p, int64_t i) { return f16_bits_to_f32(p[i]); }
    __device__ __forceinline__ static void store(storage* p, int64_t i, float v) { p[i] = f32_to_f16_bits(v); }
};

// ---- MFMA operand types (gfx950) ----------------------------------------------------------------
typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));

// The padding row that absent taps read, 0 * x (submconv_pad, sparse.cpp:81-85: row N of the
// padded input is feats[0] scaled by 0), for eight 16-bit values of x: a zero with x's sign, or
// a quiet NaN where x is an Inf or a NaN.
template <bool BF16>
__device__ __forceinline__ u32x4_t zero_times16(u32x4_t x) {
    constexpr uint32_t kExp = BF16 ? 0x7F80u : 0x7C00u, kNan = BF16 ? 0x7FC0u : 0x7E00u;
    u32x4_t r;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        const uint32_t lo = x[e] & 0xffffu, hi = x[e] >> 16;
        const uint32_t zlo = (lo & kExp) == kExp ? kNan : (lo & 0x8000u);
        const uint32_t zhi = (hi & kExp) == kExp ? kNan : (hi & 0x8000u);
        r[e] = zlo | (zhi << 16);
    }
    return r;
}

constexpr int kWave = 64;
constexpr int kTaps = 27;

inline int64_t ceil_div(int64_t a, int64_t b) { return (a + b - 1) / b; }

// Sum over aligned groups of L lanes (16 <= L <= 64); every lane of a group ends with the same
// value. Within a 16-lane DPP row the moves are lane ^ 1, lane ^ 2, 7 - lane within each 8 and
// 15 - lane, each pairing lanes whose partial sums cover disjoint lanes; across rows, shuffles.
template <int CTRL>
__device__ __forceinline__ float dpp_move(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xF, 0xF, false));
}
template <int L>
__device__ __forceinline__ float group_sum(float v) {
    static_assert(L == 8 || L == 16 || L == 32 || L == 64, "group of 8, 16, 32 or 64 lanes");
    v += dpp_move<0xB1>(v);    // quad_perm [1, 0, 3, 2]
    v += dpp_move<0x4E>(v);    // quad_perm [2, 3, 0, 1]
    v += dpp_move<0x141>(v);   // row_half_mirror
    if constexpr (L >= 16) v += dpp_move<0x140>(v);   // row_mirror
    if constexpr (L >= 32) v += __shfl_xor(v, 16, 64);
    if constexpr (L >= 64) v += __shfl_xor(v, 32, 64);
    return v;
}

}  // namespace tsp
