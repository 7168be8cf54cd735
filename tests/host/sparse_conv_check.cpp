// The conv / ConvNeXt check of the reference's test_sparse_conv.cpp (same inputs, graph and
// metric), run through this build's sparse.h adapter and HIP graph runtime:
//   sparse_conv_check <model.gguf> <ref_dir> [gpu] [--f32] [--prefix blocks.3.0]
// ref_dir holds coords.npy [N,3] int32, feats_in.npy [N,C], nbr.npy [27*N] int32 (expected
// table), conv_out.npy and block_out.npy [N,C] (expected outputs). Prints the table check and
// max|d|/max|ref| of both outputs; exit status 0 when it ran.
#include <array>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <string>
#include <vector>

#include "ggml-alloc.h"
#include "ggml-backend.h"
#include "ggml.h"
#include "npy_io.hpp"
#include "sparse.h"
#include "trellis_model.h"

static double rel(const std::vector<float>& mine, const npyio::Array& ref) {
    const float* r = ref.as<float>();
    double maxd = 0, gmax = 0;
    for (size_t i = 0; i < mine.size(); ++i) {
        maxd = std::max(maxd, std::fabs((double)mine[i] - r[i]));
        gmax = std::max(gmax, std::fabs((double)r[i]));
    }
    return gmax > 0 ? maxd / gmax : maxd;
}

int main(int argc, char** argv) {
    if (argc < 3) {
        fprintf(stderr, "usage: %s <model.gguf> <ref_dir> [gpu] [--f32] [--prefix P]\n", argv[0]);
        return 1;
    }
    const std::string dir = argv[2];
    int gpu = 0;
    std::string prefix = "blocks.3.0";
    for (int i = 3; i < argc; ++i) {
        if (!strcmp(argv[i], "--f32")) trellis::g_sparse_cast_f32 = true;
        else if (!strcmp(argv[i], "--prefix") && i + 1 < argc) prefix = argv[++i];
        else gpu = atoi(argv[i]);
    }
    try {
        trellis::Model m = trellis::Model::load(argv[1], gpu);
        npyio::Array co = npyio::load(dir + "/coords.npy");
        npyio::Array fi = npyio::load(dir + "/feats_in.npy");
        npyio::Array nb = npyio::load(dir + "/nbr.npy");
        npyio::Array cref = npyio::load(dir + "/conv_out.npy");
        npyio::Array bref = npyio::load(dir + "/block_out.npy");
        const int N = (int)co.shape[0], C = (int)fi.shape[1];
        printf("N=%d C=%d arch=%s weights=%zu bytes\n", N, C, m.arch.c_str(), m.total_bytes());

        std::vector<std::array<int, 3>> coords(N);
        memcpy(coords.data(), co.as<int32_t>(), (size_t)N * 12);
        std::vector<int32_t> nbr = trellis::build_neighbor_table(coords);
        const bool exact = nbr.size() == (size_t)nb.size() &&
                           memcmp(nbr.data(), nb.as<int32_t>(), nbr.size() * 4) == 0;
        printf("nbr_exact %d\n", exact ? 1 : 0);

        // feats [N, C] row-major == ggml [C, N]
        const size_t meta = ggml_tensor_overhead() * 4096 + ggml_graph_overhead_custom(8192, false) + (1 << 20);
        ggml_context* c = ggml_init({meta, nullptr, true});
        ggml_tensor* gf = ggml_new_tensor_2d(c, GGML_TYPE_F32, C, N);
        ggml_set_input(gf);
        ggml_tensor* gn = ggml_new_tensor_2d(c, GGML_TYPE_I32, N, 27);
        ggml_set_input(gn);
        ggml_tensor* convo = trellis::sparse_submconv(c, m, prefix + ".conv", gf, gn, N);
        ggml_tensor* blko = trellis::sparse_convnext(c, m, prefix, gf, gn, N);
        ggml_set_output(convo);
        ggml_set_output(blko);
        ggml_cgraph* g = ggml_new_graph_custom(c, 8192, false);
        ggml_build_forward_expand(g, convo);
        ggml_build_forward_expand(g, blko);
        ggml_gallocr_t alloc = ggml_gallocr_new(ggml_backend_get_default_buffer_type(m.backend));
        if (!ggml_gallocr_alloc_graph(alloc, g)) {
            fprintf(stderr, "alloc failed\n");
            return 1;
        }
        printf("graph nodes=%d buffer=%zu bytes\n", ggml_graph_n_nodes(g), ggml_gallocr_get_buffer_size(alloc, 0));
        ggml_backend_tensor_set(gf, fi.as<float>(), 0, (size_t)N * C * 4);
        ggml_backend_tensor_set(gn, nbr.data(), 0, nbr.size() * 4);
        if (ggml_backend_graph_compute(m.backend, g) != GGML_STATUS_SUCCESS) {
            fprintf(stderr, "compute failed\n");
            return 1;
        }
        printf("conv_out rel=%.4e\n", rel(trellis::tensor_to_f32(convo), cref));
        printf("block_out rel=%.4e\n", rel(trellis::tensor_to_f32(blko), bref));
        ggml_gallocr_free(alloc);
        ggml_free(c);
        m.free();
    } catch (const std::exception& e) {
        fprintf(stderr, "error: %s\n", e.what());
        return 3;
    }
    return 0;
}
