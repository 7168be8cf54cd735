// Runs the device-resident decoders of this build on a GGUF model and writes their results:
//   decoder_check <model.gguf> <dir> [gpu] [--f32] [--tex | --upsample] [--repeat K]
// dir holds latent.npy [N, Cl] f32 and coords.npy [N, 3] int32; with --tex also subs_<s>.npy
// (u8 [8 N_s]) per stage, which drive tex_decode. shape_decode writes out.npy [M, 7] f32,
// coords_out.npy [M, 3] and subs_out_<s>.npy; tex_decode writes out.npy [M, 6]; shape_upsample
// writes coords_out.npy. Prints "M=<m> ...". With --repeat K, tex_decode runs K times (the later
// runs reuse the device blocks the earlier ones released) and every run must give the same bits.
#include <array>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <string>
#include <vector>

#include "npy_io.hpp"
#include "shape_decoder.h"
#include "sparse.h"
#include "trellis_model.h"

int main(int argc, char** argv) {
    if (argc < 3) {
        fprintf(stderr, "usage: %s <model.gguf> <dir> [gpu] [--f32] [--tex]\n", argv[0]);
        return 1;
    }
    const std::string dir = argv[2];
    int gpu = 0;
    bool tex = false, upsample = false;
    int repeat = 1;
    for (int i = 3; i < argc; ++i) {
        if (!strcmp(argv[i], "--f32")) trellis::g_sparse_cast_f32 = true;
        else if (!strcmp(argv[i], "--repeat") && i + 1 < argc) repeat = atoi(argv[++i]);
        else if (!strcmp(argv[i], "--tex")) tex = true;
        else if (!strcmp(argv[i], "--upsample")) upsample = true;
        else gpu = atoi(argv[i]);
    }
    try {
        trellis::Model m = trellis::Model::load(argv[1], gpu);
        npyio::Array la = npyio::load(dir + "/latent.npy");
        npyio::Array co = npyio::load(dir + "/coords.npy");
        const int n = (int)co.shape[0];
        std::vector<std::array<int, 3>> coords(n);
        memcpy(coords.data(), co.as<int32_t>(), (size_t)n * 12);
        std::vector<float> latent(la.as<float>(), la.as<float>() + la.size());
        std::vector<float> out;
        std::vector<std::array<int, 3>> oc;
        std::vector<std::vector<uint8_t>> subs;
        int out_ch;
        if (tex) {
            for (int s = 0;; ++s) {
                const std::string f = dir + "/subs_" + std::to_string(s) + ".npy";
                FILE* probe = fopen(f.c_str(), "rb");
                if (!probe) break;
                fclose(probe);
                npyio::Array a = npyio::load(f);
                subs.emplace_back(a.bytes.begin(), a.bytes.end());
            }
            out = trellis::tex_decode(m, latent, coords, subs);
            for (int r = 1; r < repeat; ++r) {
                const std::vector<float> again = trellis::tex_decode(m, latent, coords, subs);
                if (again.size() != out.size() || memcmp(again.data(), out.data(), out.size() * 4)) {
                    fprintf(stderr, "error: tex_decode run %d differs from run 0\n", r);
                    return 4;
                }
            }
            out_ch = 6;
        } else if (upsample) {
            oc = trellis::shape_upsample(m, latent, coords);
            npyio::save(dir + "/coords_out.npy", "<i4", {(int64_t)oc.size(), 3}, oc.data(), oc.size() * 12);
            printf("M=%zu\n", oc.size());
            m.free();
            return 0;
        } else {
            trellis::ShapeOut so = trellis::shape_decode(m, latent, coords);
            out = std::move(so.feats7);
            oc = std::move(so.coords);
            subs = std::move(so.subs);
            out_ch = 7;
        }
        const int64_t mm = (int64_t)out.size() / out_ch;
        npyio::save(dir + "/out.npy", "<f4", {mm, out_ch}, out.data(), out.size() * 4);
        if (!tex) {
            npyio::save(dir + "/coords_out.npy", "<i4", {(int64_t)oc.size(), 3}, oc.data(), oc.size() * 12);
            for (size_t s = 0; s < subs.size(); ++s)
                npyio::save(dir + "/subs_out_" + std::to_string(s) + ".npy", "|u1", {(int64_t)subs[s].size()},
                            subs[s].data(), subs[s].size());
        }
        printf("M=%lld stages=%zu\n", (long long)mm, subs.size());
        m.free();
    } catch (const std::exception& e) {
        fprintf(stderr, "error: %s\n", e.what());
        return 3;
    }
    return 0;
}
