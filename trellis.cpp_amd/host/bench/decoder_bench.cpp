// Times the device-resident texture decoder (trellis::tex_decode: the sparse U-Net decoder driven
// by given subdivision masks) on a GGUF model:
//   decoder_bench <model.gguf> <dir> <gpu> <warmup> <steps>
// dir holds latent.npy [N, Cl] f32, coords.npy [N, 3] int32 and subs_<s>.npy (u8 [8 N_s]) per
// stage. Each decode is one call: host inputs in, host output [6 M] back (the reference's API),
// so the time includes those transfers. Prints one JSON line, with the device memory in use
// after the decodes (the model and the host library's cached blocks).
#include <algorithm>
#include <array>
#include <chrono>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <string>
#include <vector>

#include <hip/hip_runtime.h>

#include "npy_io.hpp"
#include "shape_decoder.h"
#include "trellis_model.h"

int main(int argc, char** argv) {
    if (argc < 6) {
        fprintf(stderr, "usage: %s <model.gguf> <dir> <gpu> <warmup> <steps>\n", argv[0]);
        return 1;
    }
    const std::string dir = argv[2];
    const int gpu = atoi(argv[3]), warmup = atoi(argv[4]), steps = atoi(argv[5]);
    try {
        const auto t0 = std::chrono::steady_clock::now();
        trellis::Model m = trellis::Model::load(argv[1], gpu);
        const double load_ms =
            std::chrono::duration<double, std::milli>(std::chrono::steady_clock::now() - t0).count();
        npyio::Array la = npyio::load(dir + "/latent.npy");
        npyio::Array co = npyio::load(dir + "/coords.npy");
        const int n = (int)co.shape[0];
        std::vector<std::array<int, 3>> coords(n);
        memcpy(coords.data(), co.as<int32_t>(), (size_t)n * 12);
        std::vector<float> latent(la.as<float>(), la.as<float>() + la.size());
        std::vector<std::vector<uint8_t>> subs;
        for (int s = 0;; ++s) {
            const std::string f = dir + "/subs_" + std::to_string(s) + ".npy";
            FILE* probe = fopen(f.c_str(), "rb");
            if (!probe) break;
            fclose(probe);
            npyio::Array a = npyio::load(f);
            subs.emplace_back(a.bytes.begin(), a.bytes.end());
        }
        std::vector<float> out;
        std::vector<double> ms;
        for (int i = 0; i < warmup + steps; ++i) {
            const auto a = std::chrono::steady_clock::now();
            out = trellis::tex_decode(m, latent, coords, subs);
            const double d = std::chrono::duration<double, std::milli>(std::chrono::steady_clock::now() - a).count();
            if (i >= warmup) ms.push_back(d);
            fprintf(stderr, "decode %d: %.2f ms\n", i, d);
        }
        double sum = 0, mn = 1e30;
        for (double d : ms) { sum += d; mn = std::min(mn, d); }
        double checksum = 0;
        for (size_t i = 0; i < out.size(); i += 97) checksum += out[i];
        size_t free_b = 0, total_b = 0;
        if (hipMemGetInfo(&free_b, &total_b) != hipSuccess) free_b = total_b = 0;
        printf("{\"decode_ms\": %.4f, \"min_ms\": %.4f, \"steps\": %d, \"load_ms\": %.1f, \"voxels_in\": %d, "
               "\"voxels_out\": %zu, \"stages\": %zu, \"model_bytes\": %zu, \"device_bytes_in_use\": %zu, "
               "\"checksum\": %.6e}\n",
               sum / std::max<size_t>(1, ms.size()), mn, steps, load_ms, n, out.size() / 6, subs.size(),
               m.total_bytes(), total_b - free_b, checksum);
        m.free();
    } catch (const std::exception& e) {
        fprintf(stderr, "error: %s\n", e.what());
        return 3;
    }
    return 0;
}
