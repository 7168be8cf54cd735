// Model: GGUF checkpoint -> one device buffer of weights on a HIP device
// (trellis_model.cpp:96-186 of the reference: same steps, names and error messages).
#include "trellis_model.h"

#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdio>
#include <cstring>
#include <stdexcept>

#include "ggml-backend.h"
#include "ggml.h"
#include "gguf.h"

namespace trellis {

Model Model::load(const std::string& path, int gpu) {
    if (gpu < 0)
        throw std::runtime_error("Model::load: this build runs on HIP devices only (gpu < 0 asks "
                                 "for a CPU backend, which it does not have)");
    Model m;
    ggml_context* meta = nullptr;
    gguf_init_params gp{};
    gp.no_alloc = true;
    gp.ctx = &meta;
    m.gguf = gguf_init_from_file(path.c_str(), gp);
    if (!m.gguf) throw std::runtime_error("failed to open gguf: " + path);
    m.meta = meta;

    if (int64_t k = gguf_find_key(m.gguf, "general.architecture"); k >= 0)
        m.arch = gguf_get_val_str(m.gguf, k);
    if (int64_t k = gguf_find_key(m.gguf, "trellis.config_json"); k >= 0)
        m.config_json = gguf_get_val_str(m.gguf, k);

    m.backend = ggml_backend_hip_init(gpu);
    if (!m.backend) {
        m.free();
        throw std::runtime_error("Model::load: no HIP device " + std::to_string(gpu));
    }
    m.on_gpu = true;
    m.buffer = ggml_backend_alloc_ctx_tensors(meta, m.backend);
    if (!m.buffer) {
        m.free();
        throw std::runtime_error("failed to allocate tensor buffer for " + path);
    }

    // stream the weights through one pinned staging buffer
    FILE* f = fopen(path.c_str(), "rb");
    if (!f) {
        m.free();
        throw std::runtime_error("cannot reopen gguf: " + path);
    }
    const size_t data_off = gguf_get_data_offset(m.gguf);
    const int64_t n = gguf_get_n_tensors(m.gguf);
    size_t max_bytes = 0;
    for (int64_t i = 0; i < n; ++i)
        max_bytes = std::max(max_bytes, ggml_nbytes(ggml_get_tensor(meta, gguf_get_tensor_name(m.gguf, i))));
    void* staging = nullptr;
    if (max_bytes && hipHostMalloc(&staging, max_bytes, hipHostMallocDefault) != hipSuccess) {
        fclose(f);
        m.free();
        throw std::runtime_error("Model::load: cannot allocate pinned staging memory");
    }
    try {
        for (int64_t i = 0; i < n; ++i) {
            const char* name = gguf_get_tensor_name(m.gguf, i);
            ggml_tensor* t = ggml_get_tensor(meta, name);
            const size_t nbytes = ggml_nbytes(t);
            const size_t off = data_off + gguf_get_tensor_offset(m.gguf, i);
            if (fseeko(f, (off_t)off, SEEK_SET) != 0 || fread(staging, 1, nbytes, f) != nbytes)
                throw std::runtime_error(std::string("short read for tensor ") + name);
            ggml_backend_tensor_set(t, staging, 0, nbytes);
            m.tensors[name] = t;
        }
    } catch (...) {
        fclose(f);
        if (staging) (void)hipHostFree(staging);
        m.free();
        throw;
    }
    fclose(f);
    if (staging) (void)hipHostFree(staging);
    return m;
}

ggml_tensor* Model::try_get(const std::string& name) const {
    auto it = tensors.find(name);
    return it == tensors.end() ? nullptr : it->second;
}

ggml_tensor* Model::get(const std::string& name) const {
    ggml_tensor* t = try_get(name);
    if (!t) throw std::runtime_error("missing tensor: " + name);
    return t;
}

bool Model::has(const std::string& name) const { return tensors.count(name) > 0; }

size_t Model::total_bytes() const {
    size_t s = 0;
    for (auto& kv : tensors) s += ggml_nbytes(kv.second);
    return s;
}

void Model::free() {
    if (buffer) ggml_backend_buffer_free(buffer);
    if (backend) ggml_backend_free(backend);
    if (gguf) gguf_free(gguf);
    if (meta) ggml_free(meta);
    buffer = nullptr;
    backend = nullptr;
    gguf = nullptr;
    meta = nullptr;
    tensors.clear();
}

std::vector<float> tensor_to_f32(ggml_tensor* t) {
    const int64_t ne = ggml_nelements(t);
    std::vector<float> out((size_t)ne);
    if (t->type == GGML_TYPE_F32) {
        ggml_backend_tensor_get(t, out.data(), 0, (size_t)ne * sizeof(float));
    } else if (t->type == GGML_TYPE_F16) {
        std::vector<ggml_fp16_t> raw((size_t)ne);
        ggml_backend_tensor_get(t, raw.data(), 0, (size_t)ne * sizeof(ggml_fp16_t));
        ggml_fp16_to_fp32_row(raw.data(), out.data(), ne);
    } else {
        throw std::runtime_error("tensor_to_f32: unsupported type");
    }
    return out;
}

}  // namespace trellis
