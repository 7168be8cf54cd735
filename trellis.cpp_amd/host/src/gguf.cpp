// Read-only GGUF reader (format versions 2 and 3): the key/value table, the tensor table and
// the data offset, which is what Model::load needs (trellis_model.cpp:96-142). Tensor data is not
// read here; the loader streams it to the device itself.
//
// Layout (little endian): "GGUF", u32 version, u64 n_tensors, u64 n_kv; n_kv x (string key,
// u32 type, value); n_tensors x (string name, u32 n_dims, u64 ne[n_dims], u32 ggml type,
// u64 offset); padding to general.alignment (default 32); tensor data. A string is a u64 length
// and bytes; an array is u32 element type, u64 count, elements.
#include <cstdio>
#include <cstring>
#include <string>
#include <vector>

#include "gguf.h"

namespace {

enum : uint32_t {
    T_U8 = 0, T_I8 = 1, T_U16 = 2, T_I16 = 3, T_U32 = 4, T_I32 = 5, T_F32 = 6, T_BOOL = 7,
    T_STRING = 8, T_ARRAY = 9, T_U64 = 10, T_I64 = 11, T_F64 = 12,
};

struct Kv {
    std::string key;
    uint32_t type = 0;
    std::string str;      // T_STRING
    uint64_t u = 0;       // integer types
};

struct TensorInfo {
    std::string name;
    uint64_t offset = 0;
};

// Every length read from the file is checked against the bytes the file has left before it is
// used, so a corrupt count is rejected instead of allocated or skipped past the end.
class Reader {
public:
    explicit Reader(FILE* f) : f_(f) {
        if (fseeko(f_, 0, SEEK_END) == 0) size_ = (uint64_t)ftello(f_);
        fseeko(f_, 0, SEEK_SET);
    }
    bool bytes(void* p, size_t n) { return fread(p, 1, n, f_) == n; }
    template <class T> bool pod(T& v) { return bytes(&v, sizeof(T)); }
    bool str(std::string& s) {
        uint64_t n;
        if (!pod(n) || n > left()) return false;
        s.resize(n);
        return n == 0 || bytes(&s[0], n);
    }
    bool skip(uint64_t n) { return n <= left() && fseeko(f_, (off_t)n, SEEK_CUR) == 0; }
    uint64_t tell() { return (uint64_t)ftello(f_); }
    uint64_t left() {
        const uint64_t t = tell();
        return t <= size_ ? size_ - t : 0;
    }

private:
    FILE* f_;
    uint64_t size_ = 0;
};

size_t scalar_size(uint32_t t) {
    switch (t) {
        case T_U8: case T_I8: case T_BOOL: return 1;
        case T_U16: case T_I16: return 2;
        case T_U32: case T_I32: case T_F32: return 4;
        case T_U64: case T_I64: case T_F64: return 8;
        default: return 0;
    }
}

}  // namespace

struct gguf_context {
    uint32_t version = 0;
    std::vector<Kv> kv;
    std::vector<TensorInfo> tensors;
    size_t data_offset = 0;
};

extern "C" {

struct gguf_context* gguf_init_from_file(const char* fname, struct gguf_init_params params) {
    FILE* f = fopen(fname, "rb");
    if (!f) {
        fprintf(stderr, "gguf_init_from_file: cannot open %s\n", fname);
        return nullptr;
    }
    Reader r(f);
    auto* g = new gguf_context;
    ggml_context* meta = nullptr;
    auto bad = [&](const char* why) -> gguf_context* {
        fprintf(stderr, "gguf_init_from_file: %s: %s\n", fname, why);
        fclose(f);
        if (meta) ggml_free(meta);
        delete g;
        return nullptr;
    };
    char magic[4];
    uint64_t n_tensors = 0, n_kv = 0;
    if (!r.bytes(magic, 4) || memcmp(magic, "GGUF", 4) != 0) return bad("not a GGUF file");
    if (!r.pod(g->version) || (g->version != 2 && g->version != 3))
        return bad("unsupported GGUF version");
    if (!r.pod(n_tensors) || !r.pod(n_kv) || n_tensors > (1u << 24) || n_kv > (1u << 24))
        return bad("bad header");

    uint64_t alignment = 32;
    for (uint64_t i = 0; i < n_kv; ++i) {
        Kv kv;
        if (!r.str(kv.key) || !r.pod(kv.type)) return bad("truncated key/value table");
        if (kv.type == T_STRING) {
            if (!r.str(kv.str)) return bad("truncated string value");
        } else if (kv.type == T_ARRAY) {
            uint32_t et;
            uint64_t n;
            if (!r.pod(et) || !r.pod(n)) return bad("truncated array");
            if (et == T_STRING) {
                std::string s;
                if (n > r.left() / 8) return bad("truncated string array");   // 8 length bytes each
                for (uint64_t j = 0; j < n; ++j)
                    if (!r.str(s)) return bad("truncated string array");
            } else {
                const size_t es = scalar_size(et);
                if (!es) return bad("bad array element type");
                if (n > r.left() / es || !r.skip(es * n)) return bad("truncated array");
            }
        } else {
            const size_t es = scalar_size(kv.type);
            if (!es || !r.bytes(&kv.u, es)) return bad("bad value type");
        }
        if (kv.key == "general.alignment" && (kv.type == T_U32 || kv.type == T_U64)) {
            alignment = kv.u;
            if (alignment == 0 || (alignment & (alignment - 1))) return bad("bad alignment");
        }
        g->kv.push_back(std::move(kv));
    }

    if (params.ctx) {
        ggml_init_params ip{ggml_tensor_overhead() * (size_t)(n_tensors + 1) + 4096, nullptr, true};
        meta = ggml_init(ip);
    }
    for (uint64_t i = 0; i < n_tensors; ++i) {
        TensorInfo ti;
        uint32_t n_dims, type;
        int64_t ne[GGML_MAX_DIMS] = {1, 1, 1, 1};
        if (!r.str(ti.name) || !r.pod(n_dims) || n_dims < 1 || n_dims > GGML_MAX_DIMS)
            return bad("bad tensor info");
        for (uint32_t d = 0; d < n_dims; ++d) {
            uint64_t v;
            if (!r.pod(v) || v > (1ull << 40)) return bad("bad tensor shape");
            ne[d] = (int64_t)v;
        }
        if (!r.pod(type) || !r.pod(ti.offset)) return bad("bad tensor info");
        if (type != GGML_TYPE_F32 && type != GGML_TYPE_F16 && type != GGML_TYPE_BF16 &&
            type != GGML_TYPE_I32)
            return bad("tensor type not supported by this build (F32, F16, BF16, I32)");
        if (ti.name.size() >= GGML_MAX_NAME) return bad("tensor name too long");
        if (meta) {
            ggml_tensor* t = ggml_new_tensor(meta, (enum ggml_type)type, (int)n_dims, ne);
            ggml_set_name(t, ti.name.c_str());
        }
        g->tensors.push_back(std::move(ti));
    }
    const uint64_t pos = r.tell();
    g->data_offset = (size_t)((pos + alignment - 1) / alignment * alignment);
    fclose(f);
    if (params.ctx) *params.ctx = meta;
    (void)params.no_alloc;
    return g;
}

void gguf_free(struct gguf_context* ctx) { delete ctx; }

int64_t gguf_find_key(const struct gguf_context* ctx, const char* key) {
    for (size_t i = 0; i < ctx->kv.size(); ++i)
        if (ctx->kv[i].key == key) return (int64_t)i;
    return -1;
}

const char* gguf_get_val_str(const struct gguf_context* ctx, int64_t key_id) {
    if (key_id < 0 || key_id >= (int64_t)ctx->kv.size() || ctx->kv[key_id].type != T_STRING)
        ggml_abort(__FILE__, __LINE__, "gguf_get_val_str: not a string key");
    return ctx->kv[key_id].str.c_str();
}

int64_t gguf_get_n_tensors(const struct gguf_context* ctx) { return (int64_t)ctx->tensors.size(); }

const char* gguf_get_tensor_name(const struct gguf_context* ctx, int64_t id) {
    return ctx->tensors.at((size_t)id).name.c_str();
}

size_t gguf_get_tensor_offset(const struct gguf_context* ctx, int64_t id) {
    return (size_t)ctx->tensors.at((size_t)id).offset;
}

size_t gguf_get_data_offset(const struct gguf_context* ctx) { return ctx->data_offset; }

}  // extern "C"
