// trellis_model.h -- the GGUF model container that trellis.cpp's sparse-path callers use
// (include/trellis_model.h): the declarations are the reference's, so callers compile unchanged;
// the weights live on a HIP device of this build's runtime.
#pragma once

#include <cstdint>
#include <map>
#include <string>
#include <vector>

struct ggml_tensor;
struct ggml_context;
struct gguf_context;
struct ggml_backend;
struct ggml_backend_buffer;

namespace trellis {

// One loaded checkpoint: GGUF metadata, tensor structs, the device buffer holding every weight
// and a name -> tensor map (trellis_model.h:18-37).
struct Model {
    gguf_context* gguf = nullptr;
    ggml_context* meta = nullptr;
    ggml_backend* backend = nullptr;
    ggml_backend_buffer* buffer = nullptr;
    std::map<std::string, ggml_tensor*> tensors;
    std::string arch;          // general.architecture
    std::string config_json;   // trellis.config_json
    bool on_gpu = false;

    // gpu = HIP device index. This build has no CPU backend: gpu < 0 throws.
    static Model load(const std::string& path, int gpu = 0);

    ggml_tensor* get(const std::string& name) const;       // throws std::runtime_error if missing
    ggml_tensor* try_get(const std::string& name) const;   // nullptr if missing
    bool has(const std::string& name) const;

    size_t total_bytes() const;
    void free();
};

// A tensor's contents on the host as float32 (F32, F16 and BF16; throws for other types).
std::vector<float> tensor_to_f32(ggml_tensor* t);

}  // namespace trellis
