// Dense linear layers (the ConvNeXt MLPs, to_subdiv) as library GEMMs on hipBLASLt.
//
// out[i] = act(x[i] . W^T + bias) + residual[i] for x [n][ci] and W [co][ci] row-major, i.e. the
// column-major product D (co x n) = op(W') (co x ci) . x' (ci x n) with W' = W viewed column-major
// (ci x co, transposed by the op) and x' = x viewed column-major. Bias and SiLU run in the GEMM's
// epilogue (fp32, before the output's rounding); the residual enters as C with beta = 1.
// Algorithms come from hipBLASLt's heuristic with no workspace, cached per shape and device.
#include <hipblaslt/hipblaslt.h>

#include <map>
#include <algorithm>
#include <mutex>
#include <tuple>

#include "conv_internal.hpp"

namespace tsp {
namespace {

constexpr int kMaxDevices = 64;

struct AlgoKey {
    int dev;
    int64_t n;
    int ci, co, xdt, odt, epilogue;
    bool residual;
    bool operator<(const AlgoKey& o) const {
        return std::tie(dev, n, ci, co, xdt, odt, epilogue, residual) <
               std::tie(o.dev, o.n, o.ci, o.co, o.xdt, o.odt, o.epilogue, o.residual);
    }
};
struct AlgoEntry {
    bool ok = false;
    hipblasLtMatmulAlgo_t algo{};
};

std::mutex g_mu;
hipblasLtHandle_t g_handle[kMaxDevices] = {};
std::map<AlgoKey, AlgoEntry> g_algos;

hipDataType hip_type(int dt) {
    return dt == TSP_F32 ? HIP_R_32F : dt == TSP_BF16 ? HIP_R_16BF : HIP_R_16F;
}

// Matmul description and layouts of one call; destroyed when it goes out of scope.
struct Gemm {
    hipblasLtMatmulDesc_t desc = nullptr;
    hipblasLtMatrixLayout_t a = nullptr, b = nullptr, c = nullptr, d = nullptr;
    ~Gemm() {
        if (desc) hipblasLtMatmulDescDestroy(desc);
        if (a) hipblasLtMatrixLayoutDestroy(a);
        if (b) hipblasLtMatrixLayoutDestroy(b);
        if (c) hipblasLtMatrixLayoutDestroy(c);
        if (d) hipblasLtMatrixLayoutDestroy(d);
    }
};

}  // namespace

bool blaslt_eligible(int x_dtype, int weight_dtype, int out_dtype, int ci, int co, const void* x,
                     const void* w, const void* out) {
    if (x_dtype == TSP_F32 || x_dtype != weight_dtype) return false;
    if (out_dtype != TSP_F32 && out_dtype != x_dtype) return false;
    if (ci % 8 || co % 8) return false;
    return !(reinterpret_cast<uintptr_t>(x) % 16 || reinterpret_cast<uintptr_t>(w) % 16 ||
             reinterpret_cast<uintptr_t>(out) % 16);
}

static int blaslt_linear_rows(const void* x, int xdt, int64_t n, int ci, const void* w, const float* bias,
                              int co, int act, const float* residual, void* out, int odt, hipStream_t s);

// Rows of one library call: no operand (x, out, residual) of a call spans 2^31 bytes or more (a
// multiple of 256 rows where one fits; 0 when not even one row does).
int64_t blaslt_rows_per_call(int ci, int co, int xdt, int odt, bool residual) {
    if (ci <= 0 || co <= 0 || !dtype_valid(xdt) || !dtype_valid(odt)) return 0;
    const int64_t row_bytes = std::max<int64_t>({(int64_t)ci * (int64_t)dtype_size(xdt), (int64_t)co * (int64_t)dtype_size(odt),
                                                 residual ? (int64_t)co * 4 : 0});
    const int64_t rows = ((((int64_t)1) << 31) - 1) / row_bytes;
    return rows >= 256 ? rows / 256 * 256 : rows;
}

// Row chunks of blaslt_rows_per_call rows: one library call never addresses 2^31 bytes or more
// in an operand (the composite blocks already bound their hidden layers to 1 GiB).
int blaslt_linear(const void* x, int xdt, int64_t n, int ci, const void* w, const float* bias,
                  int co, int act, const float* residual, void* out, int odt, hipStream_t s) {
    const int64_t rows = blaslt_rows_per_call(ci, co, xdt, odt, residual != nullptr);
    TSP_REQUIRE(rows > 0, TSP_ERR_UNSUPPORTED, "linear: a row of ci=%d co=%d spans 2 GiB", ci, co);
    for (int64_t r0 = 0; r0 < n; r0 += rows) {
        const int64_t nr = std::min(rows, n - r0);
        const int st = blaslt_linear_rows(static_cast<const char*>(x) + r0 * ci * (int64_t)dtype_size(xdt), xdt, nr,
                                          ci, w, bias, co, act, residual ? residual + r0 * co : nullptr,
                                          static_cast<char*>(out) + r0 * co * (int64_t)dtype_size(odt), odt, s);
        if (st != TSP_OK) return st;
    }
    return TSP_OK;
}

static int blaslt_linear_rows(const void* x, int xdt, int64_t n, int ci, const void* w, const float* bias,
                              int co, int act, const float* residual, void* out, int odt, hipStream_t s) {
    int dev = 0;
    TSP_CHECK_HIP(hipGetDevice(&dev));
    TSP_REQUIRE(dev >= 0 && dev < kMaxDevices, TSP_ERR_INVALID, "linear: device %d out of range", dev);
    const int epi = act ? (bias ? HIPBLASLT_EPILOGUE_SWISH_BIAS_EXT : HIPBLASLT_EPILOGUE_SWISH_EXT)
                        : (bias ? HIPBLASLT_EPILOGUE_BIAS : HIPBLASLT_EPILOGUE_DEFAULT);
    std::lock_guard<std::mutex> lock(g_mu);
    if (!g_handle[dev] && hipblasLtCreate(&g_handle[dev]) != HIPBLAS_STATUS_SUCCESS) {
        g_handle[dev] = nullptr;
        set_error("linear: hipblasLtCreate failed on device %d", dev);
        return TSP_ERR_UNSUPPORTED;
    }
    hipblasLtHandle_t h = g_handle[dev];
    Gemm g;
    const hipblasOperation_t opa = HIPBLAS_OP_T, opb = HIPBLAS_OP_N;
    const hipDataType bias_type = HIP_R_32F;
    const uint32_t epi32 = (uint32_t)epi;
    bool ok = hipblasLtMatmulDescCreate(&g.desc, HIPBLAS_COMPUTE_32F, HIP_R_32F) == HIPBLAS_STATUS_SUCCESS &&
              hipblasLtMatmulDescSetAttribute(g.desc, HIPBLASLT_MATMUL_DESC_TRANSA, &opa, sizeof(opa)) == HIPBLAS_STATUS_SUCCESS &&
              hipblasLtMatmulDescSetAttribute(g.desc, HIPBLASLT_MATMUL_DESC_TRANSB, &opb, sizeof(opb)) == HIPBLAS_STATUS_SUCCESS &&
              hipblasLtMatmulDescSetAttribute(g.desc, HIPBLASLT_MATMUL_DESC_EPILOGUE, &epi32, sizeof(epi32)) == HIPBLAS_STATUS_SUCCESS;
    if (ok && bias)
        ok = hipblasLtMatmulDescSetAttribute(g.desc, HIPBLASLT_MATMUL_DESC_BIAS_POINTER, &bias, sizeof(bias)) == HIPBLAS_STATUS_SUCCESS &&
             hipblasLtMatmulDescSetAttribute(g.desc, HIPBLASLT_MATMUL_DESC_BIAS_DATA_TYPE, &bias_type, sizeof(bias_type)) == HIPBLAS_STATUS_SUCCESS;
    const hipDataType cd = hip_type(odt);
    ok = ok && hipblasLtMatrixLayoutCreate(&g.a, hip_type(xdt), ci, co, ci) == HIPBLAS_STATUS_SUCCESS &&
         hipblasLtMatrixLayoutCreate(&g.b, hip_type(xdt), ci, n, ci) == HIPBLAS_STATUS_SUCCESS &&
         hipblasLtMatrixLayoutCreate(&g.c, cd, co, n, co) == HIPBLAS_STATUS_SUCCESS &&
         hipblasLtMatrixLayoutCreate(&g.d, cd, co, n, co) == HIPBLAS_STATUS_SUCCESS;
    if (!ok) {
        set_error("linear: hipBLASLt descriptor setup failed (n=%lld ci=%d co=%d)", (long long)n, ci, co);
        return TSP_ERR_UNSUPPORTED;
    }
    const AlgoKey key{dev, n, ci, co, xdt, odt, epi, residual != nullptr};
    auto it = g_algos.find(key);
    if (it == g_algos.end()) {
        AlgoEntry e;
        hipblasLtMatmulPreference_t pref = nullptr;
        uint64_t ws = 0;
        hipblasLtMatmulHeuristicResult_t res{};
        int count = 0;
        if (hipblasLtMatmulPreferenceCreate(&pref) == HIPBLAS_STATUS_SUCCESS &&
            hipblasLtMatmulPreferenceSetAttribute(pref, HIPBLASLT_MATMUL_PREF_MAX_WORKSPACE_BYTES, &ws, sizeof(ws)) == HIPBLAS_STATUS_SUCCESS &&
            hipblasLtMatmulAlgoGetHeuristic(h, g.desc, g.a, g.b, g.c, g.d, pref, 1, &res, &count) == HIPBLAS_STATUS_SUCCESS &&
            count > 0) {
            e.ok = true;
            e.algo = res.algo;
        }
        if (pref) hipblasLtMatmulPreferenceDestroy(pref);
        it = g_algos.emplace(key, e).first;
    }
    if (!it->second.ok) {
        set_error("linear: hipBLASLt has no algorithm for n=%lld ci=%d co=%d", (long long)n, ci, co);
        return TSP_ERR_UNSUPPORTED;
    }
    const float alpha = 1.f, beta = residual ? 1.f : 0.f;
    const hipblasStatus_t st = hipblasLtMatmul(h, g.desc, &alpha, w, g.a, x, g.b, &beta,
                                               residual ? static_cast<const void*>(residual) : out, g.c,
                                               out, g.d, &it->second.algo, nullptr, 0, s);
    if (st != HIPBLAS_STATUS_SUCCESS) {
        set_error("linear: hipblasLtMatmul failed (%d)", (int)st);
        return TSP_ERR_HIP;
    }
    return TSP_OK;
}

}  // namespace tsp

using namespace tsp;

extern "C" int64_t tsp_linear_rows_per_call(int ci, int co, int x_dtype, int out_dtype, int has_residual) {
    return blaslt_rows_per_call(ci, co, x_dtype, out_dtype, has_residual != 0);
}

extern "C" int tsp_linear_ex(const void* d_x, int x_dtype, int64_t n, int ci, const void* d_weight,
                             int weight_dtype, const float* d_bias, int co, int act,
                             const float* d_residual, void* d_out, int out_dtype, void* stream) {
    clear_error();
    TSP_REQUIRE(n >= 0 && ci > 0 && co > 0, TSP_ERR_INVALID, "tsp_linear_ex: n=%lld ci=%d co=%d",
                (long long)n, ci, co);
    TSP_REQUIRE(dtype_valid(x_dtype) && dtype_valid(weight_dtype) && dtype_valid(out_dtype),
                TSP_ERR_INVALID, "tsp_linear_ex: bad dtype");
    TSP_REQUIRE(act == TSP_ACT_NONE || act == TSP_ACT_SILU, TSP_ERR_INVALID, "tsp_linear_ex: bad act %d", act);
    if (n == 0) return TSP_OK;
    TSP_REQUIRE(d_x && d_weight && d_out, TSP_ERR_INVALID, "tsp_linear_ex: null pointer");
    TSP_REQUIRE(d_out != d_x, TSP_ERR_INVALID, "tsp_linear_ex: out aliases x");
    TSP_REQUIRE(n < (int64_t)INT32_MAX, TSP_ERR_INVALID, "tsp_linear_ex: n=%lld out of range", (long long)n);
    TSP_REQUIRE(!d_residual || out_dtype == TSP_F32, TSP_ERR_UNSUPPORTED,
                "tsp_linear_ex: a residual needs f32 output");
    TSP_REQUIRE(!d_residual || reinterpret_cast<uintptr_t>(d_residual) % 16 == 0, TSP_ERR_INVALID,
                "tsp_linear_ex: residual must be 16-byte aligned");
    TSP_REQUIRE(blaslt_eligible(x_dtype, weight_dtype, out_dtype, ci, co, d_x, d_weight, d_out),
                TSP_ERR_UNSUPPORTED,
                "tsp_linear_ex: needs 16-bit x and weights of one dtype, ci %% 8 == 0, co %% 8 == 0, "
                "16-byte aligned buffers");
    return blaslt_linear(d_x, x_dtype, n, ci, d_weight, d_bias, co, act, d_residual, d_out, out_dtype,
                         as_stream(stream));
}
