/*
 * ggml.h -- the subset of the ggml tensor/graph API that trellis.cpp's sparse-path callers use
 * (shape_decoder.cpp, test_sparse_conv.cpp, test_c2s.cpp, trellis_model.h), implemented by this
 * library's own HIP runtime (host/ggml_runtime.cpp). Graphs are deferred as in ggml: ops build
 * nodes, data flows at ggml_backend_graph_compute. Tensors are laid out as in ggml: ne[0] is the
 * fastest dimension and nb[] are byte strides. Type ids are ggml's, which GGUF files store.
 */
#ifndef TRELLIS_GGML_SHIM_H
#define TRELLIS_GGML_SHIM_H

#include <stdbool.h>
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define GGML_MAX_DIMS 4
#define GGML_MAX_SRC 10
#define GGML_MAX_NAME 64
#define GGML_MAX_OP_PARAMS 64

#define GGML_ASSERT(x)                                                                   \
    do {                                                                                 \
        if (!(x)) ggml_abort(__FILE__, __LINE__, "GGML_ASSERT(" #x ") failed");           \
    } while (0)

enum ggml_type {
    GGML_TYPE_F32 = 0,
    GGML_TYPE_F16 = 1,
    GGML_TYPE_I32 = 26,
    GGML_TYPE_BF16 = 30,
};

enum ggml_status {
    GGML_STATUS_ALLOC_FAILED = -2,
    GGML_STATUS_FAILED = -1,
    GGML_STATUS_SUCCESS = 0,
    GGML_STATUS_ABORTED = 1,
};

enum ggml_op {
    GGML_OP_NONE = 0,
    GGML_OP_ADD,
    GGML_OP_MUL,
    GGML_OP_NORM,
    GGML_OP_MUL_MAT,
    GGML_OP_SILU,
    GGML_OP_GET_ROWS,
    GGML_OP_CONCAT,
    GGML_OP_CUSTOM,
};

enum ggml_tensor_flag {
    GGML_TENSOR_FLAG_INPUT = 1,
    GGML_TENSOR_FLAG_OUTPUT = 2,
};

typedef uint16_t ggml_fp16_t;

struct ggml_init_params {
    size_t mem_size;     /* metadata budget in bytes (tensor and graph structs) */
    void* mem_buffer;    /* must be NULL: metadata lives in the context's own storage */
    bool no_alloc;       /* must be true: data comes from a gallocr or a backend buffer */
};

struct ggml_context;
struct ggml_cgraph;
struct ggml_backend_buffer;

/* A custom node computes `dst` from dst->src[] on the backend's HIP stream; `scratch` is device
 * memory of the size the node declared when it was created. Returns 0 on success. */
typedef int (*ggml_custom_fn)(struct ggml_tensor* dst, void* stream, void* scratch,
                              void* userdata);

struct ggml_tensor {
    enum ggml_type type;
    struct ggml_backend_buffer* buffer;
    int64_t ne[GGML_MAX_DIMS];
    size_t nb[GGML_MAX_DIMS];
    enum ggml_op op;
    int32_t op_params[GGML_MAX_OP_PARAMS / sizeof(int32_t)];
    int32_t flags;
    struct ggml_tensor* src[GGML_MAX_SRC];
    void* data;
    char name[GGML_MAX_NAME];
    /* custom nodes: the function, its argument, the scratch bytes it asked for and, once a
     * gallocr has placed the graph, the scratch's device address */
    ggml_custom_fn custom_fn;
    void* custom_userdata;
    size_t custom_scratch;
    void* extra;
};

void ggml_abort(const char* file, int line, const char* msg);

struct ggml_context* ggml_init(struct ggml_init_params params);
void ggml_free(struct ggml_context* ctx);
size_t ggml_tensor_overhead(void);
size_t ggml_graph_overhead_custom(size_t size, bool grads);

size_t ggml_type_size(enum ggml_type type);
size_t ggml_element_size(const struct ggml_tensor* t);
int64_t ggml_nelements(const struct ggml_tensor* t);
size_t ggml_nbytes(const struct ggml_tensor* t);

struct ggml_tensor* ggml_new_tensor(struct ggml_context* ctx, enum ggml_type type, int n_dims,
                                    const int64_t* ne);
struct ggml_tensor* ggml_new_tensor_1d(struct ggml_context* ctx, enum ggml_type type, int64_t ne0);
struct ggml_tensor* ggml_new_tensor_2d(struct ggml_context* ctx, enum ggml_type type, int64_t ne0,
                                       int64_t ne1);
struct ggml_tensor* ggml_new_tensor_3d(struct ggml_context* ctx, enum ggml_type type, int64_t ne0,
                                       int64_t ne1, int64_t ne2);
struct ggml_tensor* ggml_set_name(struct ggml_tensor* t, const char* name);
struct ggml_tensor* ggml_get_tensor(struct ggml_context* ctx, const char* name);
void ggml_set_input(struct ggml_tensor* t);
void ggml_set_output(struct ggml_tensor* t);

/* ops (results are F32, except get_rows / concat of I32) */
struct ggml_tensor* ggml_add(struct ggml_context* ctx, struct ggml_tensor* a, struct ggml_tensor* b);
struct ggml_tensor* ggml_mul(struct ggml_context* ctx, struct ggml_tensor* a, struct ggml_tensor* b);
struct ggml_tensor* ggml_norm(struct ggml_context* ctx, struct ggml_tensor* a, float eps);
struct ggml_tensor* ggml_silu(struct ggml_context* ctx, struct ggml_tensor* a);
struct ggml_tensor* ggml_mul_mat(struct ggml_context* ctx, struct ggml_tensor* a,
                                 struct ggml_tensor* b);
struct ggml_tensor* ggml_get_rows(struct ggml_context* ctx, struct ggml_tensor* a,
                                  struct ggml_tensor* rows);
/* dim must be the outermost dimension a and b use (a contiguous append) */
struct ggml_tensor* ggml_concat(struct ggml_context* ctx, struct ggml_tensor* a,
                                struct ggml_tensor* b, int dim);
struct ggml_tensor* ggml_custom(struct ggml_context* ctx, enum ggml_type type, int n_dims,
                                const int64_t* ne, struct ggml_tensor** srcs, int n_srcs,
                                ggml_custom_fn fn, void* userdata, size_t scratch_bytes);

struct ggml_cgraph* ggml_new_graph_custom(struct ggml_context* ctx, size_t size, bool grads);
void ggml_build_forward_expand(struct ggml_cgraph* graph, struct ggml_tensor* tensor);
int ggml_graph_n_nodes(struct ggml_cgraph* graph);
struct ggml_tensor* ggml_graph_node(struct ggml_cgraph* graph, int i);

float ggml_fp16_to_fp32(ggml_fp16_t h);
ggml_fp16_t ggml_fp32_to_fp16(float f);
void ggml_fp16_to_fp32_row(const ggml_fp16_t* x, float* y, int64_t n);
void ggml_fp32_to_fp16_row(const float* x, ggml_fp16_t* y, int64_t n);

#ifdef __cplusplus
}
#endif
#endif
