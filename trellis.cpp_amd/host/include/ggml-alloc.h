/* ggml-alloc.h -- graph allocator subset of the ggml shim. */
#ifndef TRELLIS_GGML_ALLOC_SHIM_H
#define TRELLIS_GGML_ALLOC_SHIM_H

#include "ggml-backend.h"

#ifdef __cplusplus
extern "C" {
#endif

typedef struct ggml_gallocr* ggml_gallocr_t;

ggml_gallocr_t ggml_gallocr_new(ggml_backend_buffer_type_t buft);
void ggml_gallocr_free(ggml_gallocr_t galloc);
/* Gives every tensor of the graph without data (inputs and intermediate results) device
 * memory, plus each custom node's scratch; returns false when the allocation fails. */
bool ggml_gallocr_alloc_graph(ggml_gallocr_t galloc, struct ggml_cgraph* graph);
size_t ggml_gallocr_get_buffer_size(ggml_gallocr_t galloc, int buffer_id);

#ifdef __cplusplus
}
#endif
#endif
