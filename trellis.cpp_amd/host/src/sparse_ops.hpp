// Device-level pieces of the sparse path, shared by the ggml graph nodes of sparse.cpp, the
// device-resident C2S block and the decoder: everything takes device pointers and a stream, and
// allocates its own temporaries unless a scratch Carve is passed in.
#pragma once

#include <functional>
#include <string>
#include <vector>

#include "ggml.h"
#include "runtime.hpp"
#include "trellis_model.h"

namespace trellis {
namespace ops {

void lib(int st, const std::string& what);   // throws std::runtime_error with tsp_last_error()

// Scratch carving: the same walk sizes a buffer (a default-constructed Carve: nothing runs) and,
// over the real buffer, hands out its pieces while the work runs.
struct Carve {
    char* base = nullptr;
    size_t off = 0;
    bool sizing = true;
    Carve() = default;
    explicit Carve(void* b) : base(static_cast<char*>(b)), sizing(false) {}
    bool running() const { return !sizing; }
    void* take(size_t bytes) {
        void* p = sizing ? nullptr : base + off;
        off += tgr::align_up(bytes);
        return p;
    }
};

const ggml_tensor* vec_param(const Model& m, const std::string& name, int64_t n);
const ggml_tensor* mat_param(const Model& m, const std::string& name, int64_t k, int64_t rows);
// f32 view of a 1-D parameter (converted into scratch when stored in 16 bits)
const float* f32_param(const ggml_tensor* t, Carve& sc, hipStream_t s);

// The dtype ggml's mul_mat rounds an F32 activation to before its product with weights of
// dtype wdt (the CPU backend's vec_dot type): F16 and BF16 weights round it to their own type,
// F32 weights take it as it is. Conv weights under g_sparse_cast_f32 are F32 casts of F16 ones
// (w32, sparse.cpp:16-19; BF16 conv weights are not cast); linear weights are never cast.
int act_dtype(int wdt, bool conv_weight);

// A submanifold conv's weights (`prefix.weight` ggml [Ci, 27, Co], `prefix.bias` [Co]).
struct Conv {
    const ggml_tensor* w = nullptr;
    const ggml_tensor* b = nullptr;
    int ci = 0, co = 0, wdt = 0;
    int xdt = 0;         // the dtype the input is rounded to (act_dtype)
    bool mfma = false;   // matrix-core kernel (16-bit xdt, Ci % 16 == 0, Co % 64 == 0)
};
Conv conv_of(const Model& m, const std::string& prefix);
// c's weights packed for the matrix-core kernel, packed on first use and cached when they are a
// loaded model's (register_model_weights, by Model::load; forget_model_weights, by Model::free,
// frees the copies); null when !c.mfma or the weights are not a model's. With running false
// (a sizing pass) a non-null stand-in where a copy would be returned.
const void* packed_weights(const Conv& c, bool running, hipStream_t s);
void register_model_weights(const std::vector<const void*>& data);
void forget_model_weights(const std::vector<const void*>& data);
// out [n][co] f32 = conv(x [n][ci] of dtype xdt); plan may be null unless c.mfma.
void run_conv(const Conv& c, const void* x, int xdt, int64_t n, const int32_t* nbr, const void* plan,
              float* out, Carve& sc, hipStream_t s);
size_t conv_scratch(const Conv& c, int64_t n, int xdt);

// SparseConvNeXtBlock3d weights and the launch shape of one block over n voxels.
struct ConvNext {
    Conv conv;
    const ggml_tensor *nw = nullptr, *nb = nullptr, *w0 = nullptr, *b0 = nullptr, *w2 = nullptr,
                      *b2 = nullptr;
    int64_t n = 0;
    int c = 0;
};
ConvNext convnext_of(const Model& m, const std::string& prefix, int64_t n);
// out [n][c] f32 = block(x [n][c]) by tsp_convnext_ex (plan needed where conv.mfma); out must not
// alias x. x16 (optional, with f32 x): x rounded to a.conv.xdt; out16 (optional): receives out
// rounded to out16_dtype, for the next block's x16.
void run_convnext(const ConvNext& a, const void* x, int xdt, const int32_t* nbr, const void* plan,
                  float* out, Carve& sc, hipStream_t s, const void* x16 = nullptr, void* out16 = nullptr,
                  int out16_dtype = TSP_BF16);
size_t convnext_scratch(const ConvNext& a, int xdt);

// A voxel set on the device with its neighbour table and (optionally) conv plan.
struct Table {
    int64_t n = 0;
    tgr::DeviceBuffer nbr;    // int32 [27 n]
    tgr::DeviceBuffer plan;   // built with the table (Morton tiles) or by ensure_plan (row tiles)
    // The coordinates the table was built from when its plan has Morton-ordered tiles (6-8 % off
    // each conv against tiles of consecutive rows); null: row tiles.
    const int32_t* coords = nullptr;
    void ensure_plan(hipStream_t s);
};
// Builds the table of d_coords [n][3] (its buffers stream-ordered on s). Without d_status it
// waits for the build and throws for coordinates outside [0, 2^21-3]; with d_status (a device
// int32 the caller zeroed) it ORs the range check into it and returns without waiting. With
// morton_plan the table's Morton-ordered plan is built in the same call, on the same cell grid
// (tsp_rulebook_build_planned).
void build_table(const int32_t* d_coords, int64_t n, Table& t, hipStream_t s, int32_t* d_status = nullptr,
                 bool morton_plan = false);

// Nonzero bytes of p[0, n) (the children a subdivision mask asks for).
int64_t count_nonzero(const uint8_t* p, size_t n);

// The C2S up-block on device data: x f32 [n][cin] on coords (table `parent`); ext_mask (host,
// 8n entries) or, when null, the block's to_subdiv prediction. Returns the children's features
// f32 [m][cout], coords [m][3], their table (with plan if conv2 uses the matrix cores) and, with
// want_mask, the [8n] mask used (on the host). ext_count, when >= 0, is count_nonzero of ext_mask,
// counted by the caller beforehand.
struct C2SOut {
    int64_t m = 0;
    tgr::DeviceBuffer feats, coords;
    tgr::DeviceBuffer feats16;   // feats rounded to out16_dtype (run_c2s's, when >= 0)
    Table table;
    std::vector<uint8_t> mask;
    // With defer_conv2: conv2 (and the skip) over the child rows [r0, r1) on s, rows of feats being
    // final only once a call covered them (the block's input x and `table` must still be alive).
    std::function<void(int64_t r0, int64_t r1)> conv2_rows;
};
// defer_conv2: the block's conv2 waits for conv2_rows (the child plan then holds tiles of
// consecutive rows, so that ranges of rows are ranges of tiles).
C2SOut run_c2s(const Model& m, const std::string& prefix, const float* d_x, const int32_t* d_coords,
               Table& parent, int cin, int cout, const std::vector<uint8_t>* ext_mask, hipStream_t s,
               int32_t* d_status = nullptr, bool want_mask = true, int64_t ext_count = -1,
               int out16_dtype = -1, bool defer_conv2 = false);

// out [n][co] f32 = (optionally LN(eps, no affine) of) x [n][ci] . W^T + b for `prefix.weight`
// ggml [ci, co]; the input (the LN's output) is rounded to act_dtype of the weight.
void run_linear(const Model& m, const std::string& prefix, const float* d_x, int64_t n, int ci, int co,
                bool pre_norm, float eps, float* d_out, hipStream_t s);

}  // namespace ops
}  // namespace trellis
