/* gguf.h -- read-only GGUF (v2/v3) subset of the ggml shim. */
#ifndef TRELLIS_GGUF_SHIM_H
#define TRELLIS_GGUF_SHIM_H

#include "ggml.h"

#ifdef __cplusplus
extern "C" {
#endif

struct gguf_context;

struct gguf_init_params {
    bool no_alloc;               /* must be true: tensor data stays in the file */
    struct ggml_context** ctx;   /* if not NULL: receives a context holding the tensor infos */
};

struct gguf_context* gguf_init_from_file(const char* fname, struct gguf_init_params params);
void gguf_free(struct gguf_context* ctx);
int64_t gguf_find_key(const struct gguf_context* ctx, const char* key);   /* -1 if absent */
const char* gguf_get_val_str(const struct gguf_context* ctx, int64_t key_id);
int64_t gguf_get_n_tensors(const struct gguf_context* ctx);
const char* gguf_get_tensor_name(const struct gguf_context* ctx, int64_t tensor_id);
size_t gguf_get_tensor_offset(const struct gguf_context* ctx, int64_t tensor_id);
size_t gguf_get_data_offset(const struct gguf_context* ctx);

#ifdef __cplusplus
}
#endif
#endif
