// Lists a GGUF file's architecture, config and tensor table as the shim's reader sees it:
//   gguf_dump <file.gguf>   ->  "arch <a>", "config <json>", "data_offset <n>", then one line
//   "<name> <type> <ne0>,<ne1>,... <offset>" per tensor. Runs on the CPU.
#include <cstdio>

#include "ggml.h"
#include "gguf.h"

int main(int argc, char** argv) {
    if (argc < 2) {
        fprintf(stderr, "usage: %s <file.gguf>\n", argv[0]);
        return 1;
    }
    ggml_context* meta = nullptr;
    gguf_init_params p{};
    p.no_alloc = true;
    p.ctx = &meta;
    gguf_context* g = gguf_init_from_file(argv[1], p);
    if (!g) return 2;
    if (int64_t k = gguf_find_key(g, "general.architecture"); k >= 0) printf("arch %s\n", gguf_get_val_str(g, k));
    if (int64_t k = gguf_find_key(g, "trellis.config_json"); k >= 0) printf("config %s\n", gguf_get_val_str(g, k));
    printf("data_offset %zu\n", gguf_get_data_offset(g));
    for (int64_t i = 0; i < gguf_get_n_tensors(g); ++i) {
        const char* name = gguf_get_tensor_name(g, i);
        ggml_tensor* t = ggml_get_tensor(meta, name);
        printf("%s %d %lld,%lld,%lld,%lld %zu %zu\n", name, (int)t->type, (long long)t->ne[0],
               (long long)t->ne[1], (long long)t->ne[2], (long long)t->ne[3],
               gguf_get_tensor_offset(g, i), ggml_nbytes(t));
    }
    gguf_free(g);
    ggml_free(meta);
    return 0;
}
