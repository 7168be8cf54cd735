// trellis::Model on a HIP device: a GGUF checkpoint's tensors in one device buffer plus a
// name -> tensor map (the container of include/trellis_model.h; the reference loads through
// ggml's gguf reader into a ggml backend buffer, src/trellis_model.cpp:96-186).
//
// Loading here is a streaming upload: the tensor table from gguf.cpp is sorted by file offset
// and the data section is read front to back in 16 MiB pieces into two pinned host buffers
// that alternate, each piece's host-to-device copy running on a stream of its own while the
// next piece is read from disk. Tensors larger than a piece are split; several small tensors
// share a piece. Every failure throws std::runtime_error naming the file and what went wrong,
// and leaves nothing allocated.
#include "trellis_model.h"

#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdio>
#include <cstring>
#include <memory>
#include <numeric>
#include <stdexcept>
#include <utility>

#include "ggml-backend.h"
#include "ggml.h"
#include "gguf.h"
#include "sparse_ops.hpp"

namespace trellis {
namespace {

constexpr size_t kPiece = size_t(16) << 20;   // bytes per pinned staging buffer

[[noreturn]] void load_error(const std::string& path, const std::string& what) {
    throw std::runtime_error("trellis::Model::load(" + path + "): " + what);
}

// One tensor's bytes in the file and their destination.
struct Extent {
    uint64_t file_off;
    size_t bytes;
    ggml_tensor* dst;
};

// Two pinned buffers, two events and a copy stream; everything released on scope exit.
class Uploader {
public:
    explicit Uploader(const std::string& path) : path_(path) {
        if (hipStreamCreate(&stream_) != hipSuccess) load_error(path_, "hipStreamCreate failed");
        for (int b = 0; b < 2; ++b) {
            if (hipHostMalloc(&host_[b], kPiece, hipHostMallocDefault) != hipSuccess)
                load_error(path_, "no pinned host memory for the staging buffers");
            if (hipEventCreateWithFlags(&done_[b], hipEventDisableTiming) != hipSuccess)
                load_error(path_, "hipEventCreate failed");
        }
    }
    ~Uploader() {
        if (stream_) (void)hipStreamSynchronize(stream_);
        for (int b = 0; b < 2; ++b) {
            if (done_[b]) (void)hipEventDestroy(done_[b]);
            if (host_[b]) (void)hipHostFree(host_[b]);
        }
        if (stream_) (void)hipStreamDestroy(stream_);
    }
    Uploader(const Uploader&) = delete;
    Uploader& operator=(const Uploader&) = delete;

    // The next free staging buffer (waits for the copy that last used it).
    char* acquire() {
        cur_ ^= 1;
        if (used_[cur_] && hipEventSynchronize(done_[cur_]) != hipSuccess)
            load_error(path_, "host-to-device copy failed");
        return static_cast<char*>(host_[cur_]);
    }
    // Queues `bytes` of the current buffer, from offset `src_off`, to device address `dst`.
    void send(void* dst, size_t src_off, size_t bytes) {
        if (hipMemcpyAsync(dst, static_cast<char*>(host_[cur_]) + src_off, bytes,
                           hipMemcpyHostToDevice, stream_) != hipSuccess)
            load_error(path_, "hipMemcpyAsync failed");
    }
    // Marks the end of the current buffer's copies.
    void release() {
        if (hipEventRecord(done_[cur_], stream_) != hipSuccess) load_error(path_, "hipEventRecord failed");
        used_[cur_] = true;
    }
    void finish() {
        if (hipStreamSynchronize(stream_) != hipSuccess) load_error(path_, "host-to-device copy failed");
    }

private:
    std::string path_;
    hipStream_t stream_ = nullptr;
    void* host_[2] = {nullptr, nullptr};
    hipEvent_t done_[2] = {nullptr, nullptr};
    bool used_[2] = {false, false};
    int cur_ = 1;
};

struct FileCloser {
    void operator()(FILE* f) const { fclose(f); }
};

// Reads [off, off + len) of the file into dst.
void read_at(FILE* f, uint64_t off, char* dst, size_t len, const std::string& path,
             const char* tensor) {
    if (fseeko(f, (off_t)off, SEEK_SET) != 0 || fread(dst, 1, len, f) != len)
        load_error(path, std::string("the file ends inside the data of tensor '") + tensor + "'");
}

// Streams every extent (sorted by file offset) through the uploader. A piece collects whole
// small tensors until the next one does not fit; a tensor larger than a piece goes alone, in
// piece-sized parts.
void upload(FILE* f, const std::vector<Extent>& ext, Uploader& up, const std::string& path) {
    size_t k = 0;
    while (k < ext.size()) {
        if (ext[k].bytes > kPiece) {
            for (size_t done = 0; done < ext[k].bytes; done += kPiece) {
                const size_t len = std::min(kPiece, ext[k].bytes - done);
                char* buf = up.acquire();
                read_at(f, ext[k].file_off + done, buf, len, path, ext[k].dst->name);
                up.send(static_cast<char*>(ext[k].dst->data) + done, 0, len);
                up.release();
            }
            ++k;
            continue;
        }
        char* buf = up.acquire();
        size_t fill = 0;
        while (k < ext.size() && ext[k].bytes <= kPiece - fill) {
            read_at(f, ext[k].file_off, buf + fill, ext[k].bytes, path, ext[k].dst->name);
            if (ext[k].bytes) up.send(ext[k].dst->data, fill, ext[k].bytes);
            fill += ext[k].bytes;
            ++k;
        }
        up.release();
    }
    up.finish();
}

// bf16 / f16 bit patterns -> float
float half_bits_to_float(uint16_t h) {
    const uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    const uint32_t exp = (h >> 10) & 0x1fu, man = h & 0x3ffu;
    uint32_t bits;
    if (exp == 0x1f) {
        bits = sign | 0x7f800000u | (man << 13);                  // Inf / NaN
    } else if (exp != 0) {
        bits = sign | ((exp + 112) << 23) | (man << 13);          // normal: rebias 15 -> 127
    } else if (man == 0) {
        bits = sign;                                              // signed zero
    } else {                                                      // subnormal: normalise
        int e = 113;
        uint32_t m = man;
        while (!(m & 0x400u)) { m <<= 1; --e; }
        bits = sign | ((uint32_t)e << 23) | ((m & 0x3ffu) << 13);
    }
    float v;
    std::memcpy(&v, &bits, 4);
    return v;
}

}  // namespace

Model Model::load(const std::string& path, int gpu) {
    if (gpu < 0)
        load_error(path, "gpu < 0 selects a CPU backend; this build runs its weights on a HIP device");
    Model m;
    try {
        gguf_init_params params{};
        params.no_alloc = true;
        params.ctx = &m.meta;
        m.gguf = gguf_init_from_file(path.c_str(), params);
        if (!m.gguf) load_error(path, "not a readable GGUF v2/v3 file");
        const auto str_key = [&](const char* key) -> std::string {
            const int64_t id = gguf_find_key(m.gguf, key);
            return id < 0 ? std::string() : std::string(gguf_get_val_str(m.gguf, id));
        };
        m.arch = str_key("general.architecture");
        m.config_json = str_key("trellis.config_json");

        m.backend = ggml_backend_hip_init(gpu);
        if (!m.backend) load_error(path, "HIP device " + std::to_string(gpu) + " is not available");
        m.on_gpu = true;
        m.buffer = ggml_backend_alloc_ctx_tensors(m.meta, m.backend);
        if (!m.buffer) load_error(path, "hipMalloc of the weight buffer failed");

        const int64_t count = gguf_get_n_tensors(m.gguf);
        const uint64_t base = gguf_get_data_offset(m.gguf);
        std::vector<Extent> ext;
        ext.reserve((size_t)count);
        for (int64_t i = 0; i < count; ++i) {
            const char* name = gguf_get_tensor_name(m.gguf, i);
            ggml_tensor* t = ggml_get_tensor(m.meta, name);
            if (!t || !t->data) load_error(path, std::string("tensor '") + name + "' has no device memory");
            ext.push_back({base + gguf_get_tensor_offset(m.gguf, i), ggml_nbytes(t), t});
            m.tensors.emplace(name, t);
        }
        std::sort(ext.begin(), ext.end(),
                  [](const Extent& a, const Extent& b) { return a.file_off < b.file_off; });

        std::unique_ptr<FILE, FileCloser> file(fopen(path.c_str(), "rb"));
        if (!file) load_error(path, "cannot open the file to read tensor data");
        (void)hipSetDevice(gpu);
        Uploader up(path);
        upload(file.get(), ext, up, path);
    } catch (...) {
        m.free();
        throw;
    }
    std::vector<const void*> data;
    for (const auto& e : m.tensors) data.push_back(e.second->data);
    ops::register_model_weights(data);
    return m;
}

ggml_tensor* Model::try_get(const std::string& name) const {
    const auto hit = tensors.find(name);
    if (hit != tensors.end()) return hit->second;
    return nullptr;
}

ggml_tensor* Model::get(const std::string& name) const {
    if (ggml_tensor* t = try_get(name)) return t;
    throw std::runtime_error("trellis::Model::get: the model has no tensor '" + name + "'");
}

bool Model::has(const std::string& name) const { return try_get(name) != nullptr; }

size_t Model::total_bytes() const {
    return std::accumulate(tensors.begin(), tensors.end(), size_t(0),
                           [](size_t acc, const auto& entry) { return acc + ggml_nbytes(entry.second); });
}

void Model::free() {
    std::vector<const void*> data;   // the packed copies of these weights go too
    for (const auto& e : tensors) data.push_back(e.second->data);
    ops::forget_model_weights(data);
    tensors.clear();
    if (auto* b = std::exchange(buffer, nullptr)) ggml_backend_buffer_free(b);
    if (auto* be = std::exchange(backend, nullptr)) ggml_backend_free(be);
    if (auto* g = std::exchange(gguf, nullptr)) gguf_free(g);
    if (auto* c = std::exchange(meta, nullptr)) ggml_free(c);
    on_gpu = false;
}

std::vector<float> tensor_to_f32(ggml_tensor* t) {
    const size_t count = (size_t)ggml_nelements(t);
    std::vector<float> values(count);
    switch (t->type) {
        case GGML_TYPE_F32:
            ggml_backend_tensor_get(t, values.data(), 0, count * sizeof(float));
            break;
        case GGML_TYPE_F16:
        case GGML_TYPE_BF16: {
            std::vector<uint16_t> bits(count);
            ggml_backend_tensor_get(t, bits.data(), 0, count * sizeof(uint16_t));
            const bool brain = t->type == GGML_TYPE_BF16;
            std::transform(bits.begin(), bits.end(), values.begin(), [brain](uint16_t b) {
                if (!brain) return half_bits_to_float(b);
                const uint32_t w = (uint32_t)b << 16;
                float v;
                std::memcpy(&v, &w, 4);
                return v;
            });
            break;
        }
        default:
            throw std::runtime_error("trellis::tensor_to_f32: tensor '" + std::string(t->name) +
                                     "' is neither F32, F16 nor BF16");
    }
    return values;
}

}  // namespace trellis
