// Runs the host side's file parsers over the files named on the command line, for a build with
// AddressSanitizer and UndefinedBehaviorSanitizer: every file must either load or be rejected
// with an error, and nothing may read or write out of bounds or leak on either path.
//   san_parsers gguf <file>...   gguf_init_from_file and the tables it read
//   san_parsers npy <file>...    npyio::load
// Prints "ok <file>" or "reject <file>: <why>" per file; exit 0 unless the usage is wrong.
#include <cstdio>
#include <cstring>
#include <exception>

#include "ggml.h"
#include "gguf.h"
#include "npy_io.hpp"

static void gguf_one(const char* path) {
    ggml_context* ctx = nullptr;
    gguf_init_params p{};
    p.no_alloc = true;
    p.ctx = &ctx;
    gguf_context* g = gguf_init_from_file(path, p);
    if (!g) {
        printf("reject %s\n", path);
        return;
    }
    size_t total = 0;
    for (int64_t i = 0; i < gguf_get_n_tensors(g); ++i) {
        const ggml_tensor* t = ggml_get_tensor(ctx, gguf_get_tensor_name(g, i));
        if (t) total += ggml_nbytes(t);
    }
    if (int64_t k = gguf_find_key(g, "general.architecture"); k >= 0) {
        const char* v = gguf_get_val_str(g, k);
        if (v) total += strlen(v);
    }
    total += gguf_get_data_offset(g);
    printf("ok %s (%zu bytes)\n", path, total);
    gguf_free(g);
    if (ctx) ggml_free(ctx);
}

static void npy_one(const char* path) {
    try {
        npyio::Array a = npyio::load(path);
        printf("ok %s (%s, %lld elements, %zu bytes)\n", path, a.descr.c_str(), (long long)a.size(),
               a.bytes.size());
    } catch (const std::exception& e) {
        printf("reject %s: %s\n", path, e.what());
    }
}

int main(int argc, char** argv) {
    if (argc < 2 || (strcmp(argv[1], "gguf") != 0 && strcmp(argv[1], "npy") != 0)) {
        fprintf(stderr, "usage: %s gguf|npy <file>...\n", argv[0]);
        return 1;
    }
    const bool gguf = strcmp(argv[1], "gguf") == 0;
    for (int i = 2; i < argc; ++i) gguf ? gguf_one(argv[i]) : npy_one(argv[i]);
    return 0;
}
