// Checks trellis::sparse_submconv and trellis::sparse_convnext (include/sparse.h) as a caller
// of the reference's API would use them: a neighbour table from build_neighbor_table, then each
// op as its own single-output ggml graph on this build's HIP runtime, compared with expected
// arrays written by the CPU oracle.
//
//   sparse_conv_check <model.gguf> <case_dir> [gpu] [--f32] [--prefix blocks.3.0]
//
// case_dir: coords.npy int32 [N,3], feats_in.npy f32 [N,C], nbr.npy int32 [27*N] (the expected
// table), conv_out.npy and block_out.npy f32 [N,C]. Output, one line each: "nbr_exact 0|1",
// "conv_out rel=<x>", "block_out rel=<x>" with rel = max|mine - expected| / max|expected|
// (the error measure of the reference's sparse-conv test). Exit status 0 when every step ran,
// 2 on a usage error, 3 when a step threw.
#include <array>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <functional>
#include <stdexcept>
#include <string>
#include <vector>

#include "ggml-alloc.h"
#include "ggml-backend.h"
#include "ggml.h"
#include "npy_io.hpp"
#include "sparse.h"
#include "trellis_model.h"

namespace {

struct Options {
    std::string model, dir, prefix = "blocks.3.0";
    int gpu = 0;
};

bool parse(int argc, char** argv, Options& o) {
    if (argc < 3) return false;
    o.model = argv[1];
    o.dir = argv[2];
    for (int k = 3; k < argc; ++k) {
        const std::string a = argv[k];
        if (a == "--f32") {
            trellis::g_sparse_cast_f32 = true;
        } else if (a == "--prefix") {
            if (++k == argc) return false;
            o.prefix = argv[k];
        } else {
            char* end = nullptr;
            o.gpu = (int)strtol(a.c_str(), &end, 10);
            if (!end || *end) return false;
        }
    }
    return true;
}

// max |a - b| / max |b| over two equally long arrays (max |a - b| when b is all zero)
double max_rel(const std::vector<float>& got, const float* want, size_t count) {
    if (got.size() != count) throw std::runtime_error("output has the wrong number of values");
    double worst = 0, scale = 0;
    for (size_t k = 0; k < count; ++k) {
        worst = std::fmax(worst, std::fabs((double)got[k] - (double)want[k]));
        scale = std::fmax(scale, std::fabs((double)want[k]));
    }
    return scale == 0 ? worst : worst / scale;
}

// Builds a graph with the features [C, N] and the table [N, 27] as inputs and the node that
// `make` returns as its only output, runs it on the model's backend and returns the output.
std::vector<float> run_single(const trellis::Model& m, int n, int c, const float* feats,
                              const std::vector<int32_t>& table,
                              const std::function<ggml_tensor*(ggml_context*, ggml_tensor*, ggml_tensor*)>& make) {
    ggml_init_params ip{};
    ip.mem_size = 64 * ggml_tensor_overhead() + ggml_graph_overhead_custom(64, false);
    ip.mem_buffer = nullptr;
    ip.no_alloc = true;
    ggml_context* ctx = ggml_init(ip);
    if (!ctx) throw std::runtime_error("ggml_init failed");
    ggml_gallocr_t galloc = nullptr;
    try {
        ggml_tensor* x = ggml_new_tensor_2d(ctx, GGML_TYPE_F32, c, n);
        ggml_tensor* nb = ggml_new_tensor_2d(ctx, GGML_TYPE_I32, n, 27);
        ggml_set_input(x);
        ggml_set_input(nb);
        ggml_tensor* y = make(ctx, x, nb);
        ggml_set_output(y);
        ggml_cgraph* graph = ggml_new_graph_custom(ctx, 64, false);
        ggml_build_forward_expand(graph, y);
        galloc = ggml_gallocr_new(ggml_backend_get_default_buffer_type(m.backend));
        if (!ggml_gallocr_alloc_graph(galloc, graph)) throw std::runtime_error("graph allocation failed");
        ggml_backend_tensor_set(x, feats, 0, sizeof(float) * (size_t)n * c);
        ggml_backend_tensor_set(nb, table.data(), 0, sizeof(int32_t) * table.size());
        if (ggml_backend_graph_compute(m.backend, graph) != GGML_STATUS_SUCCESS)
            throw std::runtime_error("graph compute failed");
        std::vector<float> out = trellis::tensor_to_f32(y);
        ggml_gallocr_free(galloc);
        ggml_free(ctx);
        return out;
    } catch (...) {
        if (galloc) ggml_gallocr_free(galloc);
        ggml_free(ctx);
        throw;
    }
}

}  // namespace

int main(int argc, char** argv) {
    Options opt;
    if (!parse(argc, argv, opt)) {
        fprintf(stderr, "usage: %s <model.gguf> <case_dir> [gpu] [--f32] [--prefix P]\n", argv[0]);
        return 2;
    }
    try {
        trellis::Model model = trellis::Model::load(opt.model, opt.gpu);
        const npyio::Array coords_in = npyio::load(opt.dir + "/coords.npy");
        const npyio::Array feats = npyio::load(opt.dir + "/feats_in.npy");
        const npyio::Array want_table = npyio::load(opt.dir + "/nbr.npy");
        const npyio::Array want_conv = npyio::load(opt.dir + "/conv_out.npy");
        const npyio::Array want_block = npyio::load(opt.dir + "/block_out.npy");
        const int n = (int)coords_in.shape.at(0), c = (int)feats.shape.at(1);

        std::vector<std::array<int, 3>> voxels((size_t)n);
        const int32_t* xyz = coords_in.as<int32_t>();
        for (int i = 0; i < n; ++i) voxels[i] = {xyz[3 * i], xyz[3 * i + 1], xyz[3 * i + 2]};
        const std::vector<int32_t> table = trellis::build_neighbor_table(voxels);
        bool same = table.size() == want_table.size();
        for (size_t k = 0; same && k < table.size(); ++k) same = table[k] == want_table.as<int32_t>()[k];
        printf("voxels %d channels %d weights %zu bytes\n", n, c, model.total_bytes());
        printf("nbr_exact %d\n", same ? 1 : 0);

        const std::string conv_name = opt.prefix + ".conv";
        const std::vector<float> conv = run_single(
            model, n, c, feats.as<float>(), table, [&](ggml_context* ctx, ggml_tensor* x, ggml_tensor* nb) {
                return trellis::sparse_submconv(ctx, model, conv_name, x, nb, n);
            });
        printf("conv_out rel=%.4e\n", max_rel(conv, want_conv.as<float>(), want_conv.size()));
        const std::vector<float> block = run_single(
            model, n, c, feats.as<float>(), table, [&](ggml_context* ctx, ggml_tensor* x, ggml_tensor* nb) {
                return trellis::sparse_convnext(ctx, model, opt.prefix, x, nb, n);
            });
        printf("block_out rel=%.4e\n", max_rel(block, want_block.as<float>(), want_block.size()));
        model.free();
    } catch (const std::exception& e) {
        fprintf(stderr, "sparse_conv_check: %s\n", e.what());
        return 3;
    }
    return 0;
}
