// The C2S up-block check of the reference's test_c2s.cpp, run through this build's sparse.h
// adapter:
//   c2s_check <model.gguf> <ref_dir> [gpu] [--ext] [--f32] [--prefix blocks.3.4]
// ref_dir holds coords.npy [N,3], feats_in.npy [N,Cin], new_coords.npy [M,3], out.npy [M,Cout],
// subdiv.npy [8N] u8 (expected mask) and, for --ext, ext_mask.npy [8N] u8 to drive the block.
// Prints whether the children (in order) and the mask match exactly and max|d|/max|ref|.
#include <array>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <string>
#include <vector>

#include "npy_io.hpp"
#include "sparse.h"
#include "trellis_model.h"

int main(int argc, char** argv) {
    if (argc < 3) {
        fprintf(stderr, "usage: %s <model.gguf> <ref_dir> [gpu] [--ext] [--f32] [--prefix P]\n", argv[0]);
        return 1;
    }
    const std::string dir = argv[2];
    int gpu = 0;
    bool ext = false;
    std::string prefix = "blocks.3.4";
    for (int i = 3; i < argc; ++i) {
        if (!strcmp(argv[i], "--ext")) ext = true;
        else if (!strcmp(argv[i], "--f32")) trellis::g_sparse_cast_f32 = true;
        else if (!strcmp(argv[i], "--prefix") && i + 1 < argc) prefix = argv[++i];
        else gpu = atoi(argv[i]);
    }
    try {
        trellis::Model m = trellis::Model::load(argv[1], gpu);
        npyio::Array co = npyio::load(dir + "/coords.npy");
        npyio::Array fi = npyio::load(dir + "/feats_in.npy");
        npyio::Array nco = npyio::load(dir + "/new_coords.npy");
        npyio::Array out = npyio::load(dir + "/out.npy");
        npyio::Array sub = npyio::load(dir + "/subdiv.npy");
        const int N = (int)co.shape[0], Cin = (int)fi.shape[1], M = (int)nco.shape[0];
        const int Cout = (int)out.shape[1];
        printf("N=%d Cin=%d ref M=%d Cout=%d\n", N, Cin, M, Cout);
        std::vector<std::array<int, 3>> coords(N);
        memcpy(coords.data(), co.as<int32_t>(), (size_t)N * 12);
        std::vector<float> feats(fi.as<float>(), fi.as<float>() + (size_t)N * Cin);
        std::vector<uint8_t> ext_mask;
        if (ext) {
            npyio::Array em = npyio::load(dir + "/ext_mask.npy");
            ext_mask.assign(em.bytes.begin(), em.bytes.end());
        }
        trellis::C2SResult r = trellis::sparse_c2s(m, prefix, feats, Cin, coords, Cout, ext ? &ext_mask : nullptr);
        printf("mine M=%d C=%d\n", (int)r.coords.size(), r.C);
        const bool coords_ok = (int)r.coords.size() == M &&
                               memcmp(r.coords.data(), nco.as<int32_t>(), (size_t)M * 12) == 0;
        const bool mask_ok = r.subdiv.size() == sub.bytes.size() &&
                             memcmp(r.subdiv.data(), sub.bytes.data(), r.subdiv.size()) == 0;
        printf("coords_exact %d\nmask_exact %d\n", coords_ok ? 1 : 0, mask_ok ? 1 : 0);
        if (coords_ok) {
            const float* ref = out.as<float>();
            double maxd = 0, gmax = 0;
            for (size_t i = 0; i < r.feats.size(); ++i) {
                maxd = std::max(maxd, std::fabs((double)r.feats[i] - ref[i]));
                gmax = std::max(gmax, std::fabs((double)ref[i]));
            }
            printf("feats rel=%.4e\n", gmax > 0 ? maxd / gmax : maxd);
        }
        m.free();
    } catch (const std::exception& e) {
        fprintf(stderr, "error: %s\n", e.what());
        return 3;
    }
    return 0;
}
