// sparse.h -- trellis.cpp's sparse-voxel API (include/sparse.h:1-35), same declarations, running on
// the MI355X kernels of libtrellis_sparse through this build's HIP graph runtime.
#pragma once
#include <array>
#include <cstdint>
#include <string>
#include <vector>

struct ggml_context;
struct ggml_tensor;

namespace trellis {
struct Model;

// Tap-major neighbour table int32 [27*N]: nbr[t*N + i] = row of the voxel at
// coords[i] + (kd-1, kh-1, kw-1) with t = kd*9 + kh*3 + kw, or N when absent; for duplicate
// coordinates the largest row. Built on the current HIP device. Coordinates must lie in
// [0, 2^21-3]; throws std::runtime_error otherwise.
std::vector<int32_t> build_neighbor_table(const std::vector<std::array<int, 3>>& coords);

// Graph ops. feats: F32 ggml [C, N] (row-major N x C); nbr: I32 ggml [N, 27] holding the
// tap-major table. Submanifold conv with `prefix.weight` ggml [Ci, 27, Co] and `prefix.bias`
// [Co] -> F32 [Co, N].
ggml_tensor* sparse_submconv(ggml_context* c, const Model& m, const std::string& prefix,
                             ggml_tensor* feats, ggml_tensor* nbr, int N);
// SparseConvNeXtBlock3d: conv -> LayerNorm(affine, 1e-6) -> Linear(C, 4C) -> SiLU ->
// Linear(4C, C) -> + feats.
ggml_tensor* sparse_convnext(ggml_context* c, const Model& m, const std::string& prefix,
                             ggml_tensor* feats, ggml_tensor* nbr, int N);

// SparseResBlockC2S3d (channel -> spatial x2). feats_in: host [Cin*N] channel-major (= row-major
// N x Cin). ext_subdiv: an [8*N] mask to use instead of the block's own to_subdiv prediction.
// Returns the children's features [Cout*M], their coords, Cout and the [8*N] mask used.
struct C2SResult {
    std::vector<float> feats;
    std::vector<std::array<int, 3>> coords;
    int C = 0;
    std::vector<uint8_t> subdiv;
};
C2SResult sparse_c2s(const Model& m, const std::string& prefix, const std::vector<float>& feats_in,
                     int Cin, const std::vector<std::array<int, 3>>& coords, int Cout,
                     const std::vector<uint8_t>* ext_subdiv = nullptr);

// When true, convs run in fp32 on the F16 weights' exact values (the reference's precision-check
// switch); when false, F32 activations are rounded to the weights' 16-bit type and the conv runs
// on the matrix cores with fp32 accumulation.
extern bool g_sparse_cast_f32;

}  // namespace trellis
