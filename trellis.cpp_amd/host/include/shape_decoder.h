// shape_decoder.h -- trellis.cpp's sparse U-Net VAE decoders (include/shape_decoder.h), same
// declarations, running every stage on the device of the model.
#pragma once
#include <array>
#include <cstdint>
#include <vector>

namespace trellis {
struct Model;

struct ShapeOut {
    std::vector<float> feats7;                 // [7*M] channel-major (= row-major M x 7)
    std::vector<std::array<int, 3>> coords;    // [M] voxel coords at the final resolution
    int res = 512;
    std::vector<std::vector<uint8_t>> subs;    // the [8*N] subdivision mask of each C2S block
};

// latent: shape latent [32*N0] channel-major on coords0. Runs from_latent -> 4 x (ConvNeXt
// stage + C2S) -> LayerNorm -> output_layer; resolution is recorded in the result.
ShapeOut shape_decode(const Model& m, const std::vector<float>& latent,
                      const std::vector<std::array<int, 3>>& coords0, int resolution = 512);

// The grown coordinates only (input res * 16), skipping the output head.
std::vector<std::array<int, 3>> shape_upsample(const Model& m, const std::vector<float>& latent,
                                               const std::vector<std::array<int, 3>>& coords0);

// Texture decoder: the same network driven by the shape decoder's masks, so it grows the same
// voxel tree; returns [6*M] channel-major at shape_decode's coords and order.
std::vector<float> tex_decode(const Model& m, const std::vector<float>& tex_latent,
                              const std::vector<std::array<int, 3>>& coords0,
                              const std::vector<std::vector<uint8_t>>& subs);

}  // namespace trellis
