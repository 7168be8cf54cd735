/* ggml-backend.h -- backend subset of the ggml shim: one HIP device per backend. */
#ifndef TRELLIS_GGML_BACKEND_SHIM_H
#define TRELLIS_GGML_BACKEND_SHIM_H

#include "ggml.h"

#ifdef __cplusplus
extern "C" {
#endif

typedef struct ggml_backend* ggml_backend_t;
typedef struct ggml_backend_buffer* ggml_backend_buffer_t;
typedef struct ggml_backend_buffer_type* ggml_backend_buffer_type_t;

/* The GPU backend of this build: HIP device `device` (NULL when it does not exist). */
ggml_backend_t ggml_backend_hip_init(int device);
void ggml_backend_free(ggml_backend_t backend);
const char* ggml_backend_name(ggml_backend_t backend);
void ggml_backend_synchronize(ggml_backend_t backend);
ggml_backend_buffer_type_t ggml_backend_get_default_buffer_type(ggml_backend_t backend);
/* The backend's HIP stream (a hipStream_t). */
void* ggml_backend_hip_stream(ggml_backend_t backend);

/* Allocates device memory for every tensor of ctx that has none; NULL on failure. */
ggml_backend_buffer_t ggml_backend_alloc_ctx_tensors(struct ggml_context* ctx,
                                                     ggml_backend_t backend);
void ggml_backend_buffer_free(ggml_backend_buffer_t buffer);
size_t ggml_backend_buffer_get_size(ggml_backend_buffer_t buffer);

void ggml_backend_tensor_set(struct ggml_tensor* tensor, const void* data, size_t offset,
                             size_t size);
void ggml_backend_tensor_get(const struct ggml_tensor* tensor, void* data, size_t offset,
                             size_t size);

enum ggml_status ggml_backend_graph_compute(ggml_backend_t backend, struct ggml_cgraph* graph);

#ifdef __cplusplus
}
#endif
#endif
