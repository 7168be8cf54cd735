// A small ggml-compatible graph runtime that executes on one HIP device.
//
// It provides the part of ggml's API that trellis.cpp's sparse-path callers use
// (shape_decoder.cpp:34-77, test_sparse_conv.cpp:46-58, trellis_model.cpp:96-186): metadata-only
// contexts, deferred graphs, a graph allocator with lifetime-based reuse, and a backend that
// runs each node on the device's stream. Generic ops (add, mul, norm, silu, mul_mat, get_rows,
// concat) run as kernels of this library or of libtrellis_sparse; the sparse ops are custom
// nodes created by the adapter in sparse.cpp.
#include <algorithm>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <deque>
#include <functional>
#include <map>
#include <memory>
#include <mutex>
#include <unordered_map>
#include <unordered_set>
#include <thread>
#include <vector>

#include <sys/mman.h>

#include "ggml-alloc.h"
#include "runtime.hpp"

// ---------------------------------------------------------------------------------------------
// helpers
// ---------------------------------------------------------------------------------------------
namespace tgr {

void fail(const std::string& msg) { throw std::runtime_error(msg); }

void hip_check(hipError_t e, const char* what) {
    if (e != hipSuccess) fail(std::string(what) + ": " + hipGetErrorString(e));
}

DeviceBuffer::DeviceBuffer(size_t bytes) : n_(bytes) {
    if (bytes) hip_check(hipMalloc(&p_, bytes), "hipMalloc");
}

namespace {
// Idle blocks per (device, stream), by size. Allocated once and never destroyed, so that buffers
// released during static destruction still find it.
struct BlockCache {
    std::mutex mu;
    std::map<std::pair<int, hipStream_t>, std::multimap<size_t, void*>> idle;
};
BlockCache& block_cache() {
    static BlockCache* c = new BlockCache;
    return *c;
}
// Block sizes: 4 KiB steps up to 1 MiB, 2 MiB steps above, so that a repeated request pattern
// (the same decoder again) is served from the cache block for block.
size_t block_bytes(size_t bytes) {
    constexpr size_t kSmall = size_t(1) << 20, kPage = size_t(4) << 10, kLarge = size_t(2) << 20;
    return bytes <= kSmall ? (bytes + kPage - 1) / kPage * kPage : (bytes + kLarge - 1) / kLarge * kLarge;
}
// Frees every idle block of device dev once the device has finished all queued work.
void free_idle_blocks(int dev) {
    hip_check(hipDeviceSynchronize(), "hipDeviceSynchronize");
    BlockCache& c = block_cache();
    std::lock_guard<std::mutex> lock(c.mu);
    for (auto& [key, blocks] : c.idle) {
        if (key.first != dev) continue;
        for (auto& [bytes, p] : blocks) (void)hipFree(p);
        blocks.clear();
    }
}
}  // namespace

DeviceBuffer::DeviceBuffer(size_t bytes, hipStream_t s) : n_(bytes), s_(s), mode_(kCached) {
    if (!bytes) return;
    hip_check(hipGetDevice(&dev_), "hipGetDevice");
    const size_t want = block_bytes(bytes);
    {
        BlockCache& c = block_cache();
        std::lock_guard<std::mutex> lock(c.mu);
        auto& idle = c.idle[{dev_, s}];
        // the smallest idle block that fits, unless it is more than twice the size needed
        auto it = idle.lower_bound(want);
        if (it != idle.end() && it->first <= 2 * want) {
            cap_ = it->first;
            p_ = it->second;
            idle.erase(it);
            return;
        }
    }
    hipError_t e = hipMalloc(&p_, want);
    if (e == hipErrorOutOfMemory) {
        (void)hipGetLastError();
        p_ = nullptr;
        free_idle_blocks(dev_);
        e = hipMalloc(&p_, want);
    }
    hip_check(e, "hipMalloc");
    cap_ = want;
}
DeviceBuffer::~DeviceBuffer() { reset(); }

void DeviceBuffer::reset() {
    if (p_) {
        if (mode_ == kCached) {
            BlockCache& c = block_cache();
            std::lock_guard<std::mutex> lock(c.mu);
            c.idle[{dev_, s_}].emplace(cap_, p_);
        } else {
            (void)hipFree(p_);
        }
    }
    p_ = nullptr;
    n_ = cap_ = 0;
}

namespace {
constexpr size_t kStageChunk = size_t(24) << 20;   // divisible by 4, 12 and 24 (element sizes)
constexpr int kMaxDevices = 64;
std::mutex g_stage_mu;
void* g_stage[2] = {nullptr, nullptr};
hipEvent_t g_stage_ev[kMaxDevices][2] = {};
// copies of produced chunks: a stream of their own per device and the event they wait for
hipStream_t g_copy_stream[kMaxDevices] = {};
hipEvent_t g_prod_ev[kMaxDevices] = {};

// Chunks of whole units (at most kStageChunk bytes; the last one what is left) through the two
// staging buffers. With produce, chunk i is first produced by produce(off, len) on s and copied
// on the device's copy stream once that work is done, so that the copy of one chunk overlaps the
// production of the next; the copies have all landed when this returns.
void download_staged(const void* src, size_t bytes, size_t unit, hipStream_t s,
                     const std::function<void(size_t, size_t)>* produce,
                     const std::function<void(const void*, size_t)>& sink) {
    if (!bytes) return;
    if (!unit || unit > kStageChunk) fail("download: bad unit");
    std::lock_guard<std::mutex> lock(g_stage_mu);
    int dev = 0;
    hip_check(hipGetDevice(&dev), "hipGetDevice");
    if (dev < 0 || dev >= kMaxDevices) fail("download: device out of range");
    for (int k = 0; k < 2; ++k) {
        if (!g_stage[k]) hip_check(hipHostMalloc(&g_stage[k], kStageChunk, hipHostMallocDefault), "hipHostMalloc");
        if (!g_stage_ev[dev][k])
            hip_check(hipEventCreateWithFlags(&g_stage_ev[dev][k], hipEventDisableTiming), "hipEventCreate");
    }
    hipStream_t cs = s;
    if (produce) {
        if (!g_copy_stream[dev])
            hip_check(hipStreamCreateWithFlags(&g_copy_stream[dev], hipStreamNonBlocking), "hipStreamCreate");
        if (!g_prod_ev[dev])
            hip_check(hipEventCreateWithFlags(&g_prod_ev[dev], hipEventDisableTiming), "hipEventCreate");
        cs = g_copy_stream[dev];
    }
    const size_t chunk = kStageChunk / unit * unit;
    const size_t nchunk = (bytes + chunk - 1) / chunk;
    auto issue = [&](size_t i) {
        const size_t off = i * chunk, len = std::min(chunk, bytes - off);
        if (produce) {
            (*produce)(off, len);
            hip_check(hipEventRecord(g_prod_ev[dev], s), "hipEventRecord");
            hip_check(hipStreamWaitEvent(cs, g_prod_ev[dev], 0), "hipStreamWaitEvent");
        }
        hip_check(hipMemcpyAsync(g_stage[i % 2], static_cast<const char*>(src) + off, len,
                                 hipMemcpyDeviceToHost, cs), "download");
        hip_check(hipEventRecord(g_stage_ev[dev][i % 2], cs), "hipEventRecord");
    };
    try {
        issue(0);
        for (size_t i = 0; i < nchunk; ++i) {
            if (i + 1 < nchunk) issue(i + 1);   // the other buffer: its chunk i-1 was taken already
            hip_check(hipEventSynchronize(g_stage_ev[dev][i % 2]), "download");
            sink(g_stage[i % 2], std::min(chunk, bytes - i * chunk));
        }
    } catch (...) {
        // copies still in flight must not land in the staging buffers under the next download
        (void)hipStreamSynchronize(cs);
        throw;
    }
}

// a sink that copies each staged chunk to the next bytes of dst on several host threads
std::function<void(const void*, size_t)> threaded_sink(void* dst) {
    const unsigned hw = std::thread::hardware_concurrency();
    const size_t nthr = std::max<size_t>(1, std::min<size_t>(8, hw ? hw : 1));
    auto done = std::make_shared<size_t>(0);
    char* out = static_cast<char*>(dst);
    return [=](const void* p, size_t n) {
        // each thread copies a 64-byte-aligned part of the chunk
        const size_t part = (n / nthr + 63) / 64 * 64;
        char* to = out + *done;
        std::vector<std::thread> th;
        for (size_t k = 1; k < nthr && k * part < n; ++k)
            th.emplace_back([=] { memcpy(to + k * part, static_cast<const char*>(p) + k * part, std::min(part, n - k * part)); });
        memcpy(to, p, std::min(part, n));
        for (auto& t : th) t.join();
        *done += n;
    };
}
}  // namespace

void advise_huge_pages(void* p, size_t bytes) {
    constexpr uintptr_t kHuge = uintptr_t(2) << 20;
    const uintptr_t a = (reinterpret_cast<uintptr_t>(p) + kHuge - 1) & ~(kHuge - 1);
    const uintptr_t e = (reinterpret_cast<uintptr_t>(p) + bytes) & ~(kHuge - 1);
    if (p && e > a) (void)madvise(reinterpret_cast<void*>(a), e - a, MADV_HUGEPAGE);
}

void download_chunks(const void* src, size_t bytes, hipStream_t s,
                     const std::function<void(const void*, size_t)>& sink) {
    download_staged(src, bytes, 1, s, nullptr, sink);
}

void download_into(void* dst, const void* src, size_t bytes, hipStream_t s) {
    download_staged(src, bytes, 1, s, nullptr, threaded_sink(dst));
}

void download_produced(void* dst, const void* src, size_t bytes, size_t unit, hipStream_t s,
                       const std::function<void(size_t, size_t)>& produce) {
    download_staged(src, bytes, unit, s, &produce, threaded_sink(dst));
}

int tsp_dtype_of(enum ggml_type t) {
    switch (t) {
        case GGML_TYPE_F32: return TSP_F32;
        case GGML_TYPE_F16: return TSP_F16;
        case GGML_TYPE_BF16: return TSP_BF16;
        default: return -1;
    }
}

bool is_contiguous(const ggml_tensor* t) {
    size_t nb = ggml_type_size(t->type);
    for (int d = 0; d < GGML_MAX_DIMS; ++d) {
        if (t->ne[d] != 1 && t->nb[d] != nb) return false;
        nb *= (size_t)t->ne[d];
    }
    return true;
}

}  // namespace tgr

using namespace tgr;

// ---------------------------------------------------------------------------------------------
// contexts and tensors
// ---------------------------------------------------------------------------------------------
struct ggml_cgraph {
    size_t size = 0;
    std::vector<ggml_tensor*> nodes;
    std::vector<ggml_tensor*> leafs;
    std::unordered_set<const ggml_tensor*> seen;
};

struct ggml_context {
    size_t mem_size = 0;
    size_t used = 0;
    std::deque<ggml_tensor> tensors;   // stable addresses
    std::deque<ggml_cgraph> graphs;
    std::unordered_map<std::string, ggml_tensor*> by_name;
    std::vector<std::shared_ptr<void>> keep;
    std::map<std::pair<const ggml_tensor*, int>, ggml_tensor*> memo;
};

namespace tgr {
void context_keep(ggml_context* ctx, std::shared_ptr<void> obj) { ctx->keep.push_back(std::move(obj)); }
ggml_tensor* context_memo_get(ggml_context* ctx, const ggml_tensor* key, int kind) {
    auto it = ctx->memo.find({key, kind});
    return it == ctx->memo.end() ? nullptr : it->second;
}
void context_memo_put(ggml_context* ctx, const ggml_tensor* key, int kind, ggml_tensor* value) {
    ctx->memo[{key, kind}] = value;
}
}  // namespace tgr

extern "C" {

void ggml_abort(const char* file, int line, const char* msg) {
    fprintf(stderr, "%s:%d: %s\n", file, line, msg);
    fflush(stderr);
    abort();
}

size_t ggml_tensor_overhead(void) { return sizeof(ggml_tensor) + 64; }

size_t ggml_graph_overhead_custom(size_t size, bool grads) {
    (void)grads;
    return sizeof(ggml_cgraph) + 3 * size * sizeof(void*) + 64;
}

struct ggml_context* ggml_init(struct ggml_init_params params) {
    if (params.mem_buffer != nullptr || !params.no_alloc)
        ggml_abort(__FILE__, __LINE__,
                   "ggml_init: this runtime keeps tensor data on the device only "
                   "(mem_buffer must be NULL and no_alloc true)");
    auto* ctx = new ggml_context;
    ctx->mem_size = params.mem_size;
    return ctx;
}

void ggml_free(struct ggml_context* ctx) { delete ctx; }

static void charge(ggml_context* ctx, size_t bytes) {
    ctx->used += bytes;
    GGML_ASSERT(ctx->used <= ctx->mem_size && "ggml context metadata budget exhausted");
}

size_t ggml_type_size(enum ggml_type type) {
    switch (type) {
        case GGML_TYPE_F32: return 4;
        case GGML_TYPE_F16: return 2;
        case GGML_TYPE_BF16: return 2;
        case GGML_TYPE_I32: return 4;
    }
    ggml_abort(__FILE__, __LINE__, "ggml_type_size: unsupported tensor type");
    return 0;
}

size_t ggml_element_size(const struct ggml_tensor* t) { return ggml_type_size(t->type); }

int64_t ggml_nelements(const struct ggml_tensor* t) {
    return t->ne[0] * t->ne[1] * t->ne[2] * t->ne[3];
}

size_t ggml_nbytes(const struct ggml_tensor* t) {
    if (ggml_nelements(t) == 0) return 0;
    size_t n = ggml_type_size(t->type);
    for (int d = 0; d < GGML_MAX_DIMS; ++d) n += (size_t)(t->ne[d] - 1) * t->nb[d];
    return n;
}

struct ggml_tensor* ggml_new_tensor(struct ggml_context* ctx, enum ggml_type type, int n_dims,
                                    const int64_t* ne) {
    GGML_ASSERT(n_dims >= 1 && n_dims <= GGML_MAX_DIMS);
    charge(ctx, ggml_tensor_overhead());
    ctx->tensors.emplace_back();
    ggml_tensor* t = &ctx->tensors.back();
    memset(t, 0, sizeof(*t));
    t->type = type;
    for (int d = 0; d < GGML_MAX_DIMS; ++d) {
        t->ne[d] = d < n_dims ? ne[d] : 1;
        GGML_ASSERT(t->ne[d] >= 0);
    }
    t->nb[0] = ggml_type_size(type);
    for (int d = 1; d < GGML_MAX_DIMS; ++d) t->nb[d] = t->nb[d - 1] * (size_t)t->ne[d - 1];
    return t;
}

struct ggml_tensor* ggml_new_tensor_1d(struct ggml_context* ctx, enum ggml_type type, int64_t ne0) {
    return ggml_new_tensor(ctx, type, 1, &ne0);
}
struct ggml_tensor* ggml_new_tensor_2d(struct ggml_context* ctx, enum ggml_type type, int64_t ne0,
                                       int64_t ne1) {
    const int64_t ne[2] = {ne0, ne1};
    return ggml_new_tensor(ctx, type, 2, ne);
}
struct ggml_tensor* ggml_new_tensor_3d(struct ggml_context* ctx, enum ggml_type type, int64_t ne0,
                                       int64_t ne1, int64_t ne2) {
    const int64_t ne[3] = {ne0, ne1, ne2};
    return ggml_new_tensor(ctx, type, 3, ne);
}

struct ggml_tensor* ggml_set_name(struct ggml_tensor* t, const char* name) {
    snprintf(t->name, sizeof(t->name), "%s", name);
    return t;
}

struct ggml_tensor* ggml_get_tensor(struct ggml_context* ctx, const char* name) {
    auto it = ctx->by_name.find(name);
    if (it != ctx->by_name.end()) return it->second;
    for (auto& t : ctx->tensors)
        if (strncmp(t.name, name, GGML_MAX_NAME) == 0) {
            ctx->by_name[name] = &t;
            return &t;
        }
    return nullptr;
}

void ggml_set_input(struct ggml_tensor* t) { t->flags |= GGML_TENSOR_FLAG_INPUT; }
void ggml_set_output(struct ggml_tensor* t) { t->flags |= GGML_TENSOR_FLAG_OUTPUT; }

// ---------------------------------------------------------------------------------------------
// ops
// ---------------------------------------------------------------------------------------------
static ggml_tensor* node(ggml_context* ctx, enum ggml_op op, enum ggml_type type, const int64_t* ne,
                         ggml_tensor* a, ggml_tensor* b) {
    ggml_tensor* t = ggml_new_tensor(ctx, type, 4, ne);
    t->op = op;
    t->src[0] = a;
    t->src[1] = b;
    return t;
}

static bool can_repeat(const ggml_tensor* b, const ggml_tensor* a) {
    for (int d = 0; d < GGML_MAX_DIMS; ++d)
        if (b->ne[d] == 0 || a->ne[d] % b->ne[d] != 0) return false;
    return true;
}

static ggml_tensor* binary(ggml_context* ctx, enum ggml_op op, ggml_tensor* a, ggml_tensor* b) {
    GGML_ASSERT(can_repeat(b, a) && "ggml_add/ggml_mul: b must broadcast over a");
    GGML_ASSERT((a->type == GGML_TYPE_F32 || a->type == GGML_TYPE_F16) &&
                (b->type == GGML_TYPE_F32 || b->type == GGML_TYPE_F16));
    return node(ctx, op, GGML_TYPE_F32, a->ne, a, b);
}

struct ggml_tensor* ggml_add(struct ggml_context* ctx, struct ggml_tensor* a, struct ggml_tensor* b) {
    return binary(ctx, GGML_OP_ADD, a, b);
}
struct ggml_tensor* ggml_mul(struct ggml_context* ctx, struct ggml_tensor* a, struct ggml_tensor* b) {
    return binary(ctx, GGML_OP_MUL, a, b);
}

struct ggml_tensor* ggml_norm(struct ggml_context* ctx, struct ggml_tensor* a, float eps) {
    GGML_ASSERT(tsp_dtype_of(a->type) >= 0);
    ggml_tensor* t = node(ctx, GGML_OP_NORM, GGML_TYPE_F32, a->ne, a, nullptr);
    memcpy(&t->op_params[0], &eps, sizeof(float));
    return t;
}

struct ggml_tensor* ggml_silu(struct ggml_context* ctx, struct ggml_tensor* a) {
    GGML_ASSERT(a->type == GGML_TYPE_F32);
    return node(ctx, GGML_OP_SILU, GGML_TYPE_F32, a->ne, a, nullptr);
}

struct ggml_tensor* ggml_mul_mat(struct ggml_context* ctx, struct ggml_tensor* a,
                                 struct ggml_tensor* b) {
    GGML_ASSERT(a->ne[0] == b->ne[0] && "ggml_mul_mat: inner dimensions differ");
    GGML_ASSERT(a->ne[2] == 1 && a->ne[3] == 1 && b->ne[2] == 1 && b->ne[3] == 1 &&
                "ggml_mul_mat: only 2-D operands are supported");
    GGML_ASSERT(tsp_dtype_of(a->type) >= 0 && tsp_dtype_of(b->type) >= 0);
    const int64_t ne[4] = {a->ne[1], b->ne[1], 1, 1};
    return node(ctx, GGML_OP_MUL_MAT, GGML_TYPE_F32, ne, a, b);
}

struct ggml_tensor* ggml_get_rows(struct ggml_context* ctx, struct ggml_tensor* a,
                                  struct ggml_tensor* rows) {
    GGML_ASSERT(rows->type == GGML_TYPE_I32 && rows->ne[1] == 1 && rows->ne[2] == 1 &&
                rows->ne[3] == 1);
    GGML_ASSERT(a->ne[2] == 1 && a->ne[3] == 1 && "ggml_get_rows: only 2-D sources");
    const int64_t ne[4] = {a->ne[0], rows->ne[0], 1, 1};
    return node(ctx, GGML_OP_GET_ROWS, a->type == GGML_TYPE_I32 ? GGML_TYPE_I32 : GGML_TYPE_F32,
                ne, a, rows);
}

struct ggml_tensor* ggml_concat(struct ggml_context* ctx, struct ggml_tensor* a,
                                struct ggml_tensor* b, int dim) {
    GGML_ASSERT(dim >= 0 && dim < GGML_MAX_DIMS && a->type == b->type);
    for (int d = 0; d < GGML_MAX_DIMS; ++d) {
        if (d != dim) GGML_ASSERT(a->ne[d] == b->ne[d] && "ggml_concat: shapes differ");
        if (d > dim) GGML_ASSERT(a->ne[d] == 1 && "ggml_concat: only along the outermost dimension");
    }
    int64_t ne[4] = {a->ne[0], a->ne[1], a->ne[2], a->ne[3]};
    ne[dim] += b->ne[dim];
    ggml_tensor* t = node(ctx, GGML_OP_CONCAT, a->type, ne, a, b);
    t->op_params[0] = dim;
    return t;
}

struct ggml_tensor* ggml_custom(struct ggml_context* ctx, enum ggml_type type, int n_dims,
                                const int64_t* ne, struct ggml_tensor** srcs, int n_srcs,
                                ggml_custom_fn fn, void* userdata, size_t scratch_bytes) {
    GGML_ASSERT(n_srcs >= 0 && n_srcs <= GGML_MAX_SRC && fn != nullptr);
    ggml_tensor* t = ggml_new_tensor(ctx, type, n_dims, ne);
    t->op = GGML_OP_CUSTOM;
    for (int i = 0; i < n_srcs; ++i) t->src[i] = srcs[i];
    t->custom_fn = fn;
    t->custom_userdata = userdata;
    t->custom_scratch = scratch_bytes;
    return t;
}

// ---------------------------------------------------------------------------------------------
// graphs
// ---------------------------------------------------------------------------------------------
struct ggml_cgraph* ggml_new_graph_custom(struct ggml_context* ctx, size_t size, bool grads) {
    charge(ctx, ggml_graph_overhead_custom(size, grads));
    ctx->graphs.emplace_back();
    ggml_cgraph* g = &ctx->graphs.back();
    g->size = size;
    return g;
}

// Depth-first, sources before consumers (ggml's visit order).
void ggml_build_forward_expand(struct ggml_cgraph* g, struct ggml_tensor* root) {
    std::vector<std::pair<ggml_tensor*, int>> stack{{root, 0}};
    while (!stack.empty()) {
        auto& [t, next] = stack.back();
        if (next == 0 && g->seen.count(t)) {
            stack.pop_back();
            continue;
        }
        if (next < GGML_MAX_SRC) {
            ggml_tensor* s = t->src[next++];
            if (s && !g->seen.count(s)) stack.push_back({s, 0});
            continue;
        }
        g->seen.insert(t);
        if (t->op == GGML_OP_NONE) {
            g->leafs.push_back(t);
        } else {
            GGML_ASSERT(g->nodes.size() < g->size && "graph node budget exhausted");
            g->nodes.push_back(t);
        }
        stack.pop_back();
    }
}

int ggml_graph_n_nodes(struct ggml_cgraph* g) { return (int)g->nodes.size(); }

struct ggml_tensor* ggml_graph_node(struct ggml_cgraph* g, int i) {
    if (i < 0) i += (int)g->nodes.size();
    GGML_ASSERT(i >= 0 && i < (int)g->nodes.size());
    return g->nodes[i];
}

// ---------------------------------------------------------------------------------------------
// backend, buffers
// ---------------------------------------------------------------------------------------------
struct ggml_backend_buffer_type {
    int device;
};

struct ggml_backend {
    int device = 0;
    hipStream_t stream = nullptr;
    ggml_backend_buffer_type buft{0};
    std::string name;
};

struct ggml_backend_buffer {
    int device = 0;
    void* base = nullptr;
    size_t size = 0;
};

ggml_backend_t ggml_backend_hip_init(int device) {
    int count = 0;
    if (hipGetDeviceCount(&count) != hipSuccess || device < 0 || device >= count) return nullptr;
    if (hipSetDevice(device) != hipSuccess) return nullptr;
    auto* b = new ggml_backend;
    b->device = device;
    b->buft.device = device;
    // a blocking stream at the default priority: it orders with the synchronous copies of
    // ggml_backend_tensor_set / _get, which run on the null stream
    if (hipStreamCreate(&b->stream) != hipSuccess) {
        delete b;
        return nullptr;
    }
    hipDeviceProp_t prop;
    b->name = "HIP" + std::to_string(device);
    if (hipGetDeviceProperties(&prop, device) == hipSuccess)
        b->name += std::string(" (") + prop.gcnArchName + ")";
    return b;
}

void ggml_backend_free(ggml_backend_t backend) {
    if (!backend) return;
    (void)hipSetDevice(backend->device);
    (void)hipStreamSynchronize(backend->stream);
    (void)hipStreamDestroy(backend->stream);
    delete backend;
}

const char* ggml_backend_name(ggml_backend_t backend) { return backend->name.c_str(); }

void ggml_backend_synchronize(ggml_backend_t backend) {
    (void)hipSetDevice(backend->device);
    hip_check(hipStreamSynchronize(backend->stream), "ggml_backend_synchronize");
}

ggml_backend_buffer_type_t ggml_backend_get_default_buffer_type(ggml_backend_t backend) {
    return &backend->buft;
}

void* ggml_backend_hip_stream(ggml_backend_t backend) { return backend->stream; }

}  // extern "C"

namespace tgr {
int backend_device(ggml_backend_t backend) { return backend->device; }
hipStream_t backend_stream(ggml_backend_t backend) { return backend->stream; }
}  // namespace tgr

extern "C" {

ggml_backend_buffer_t ggml_backend_alloc_ctx_tensors(struct ggml_context* ctx,
                                                     ggml_backend_t backend) {
    size_t total = 0;
    for (auto& t : ctx->tensors)
        if (!t.data) total += align_up(ggml_nbytes(&t));
    auto* buf = new ggml_backend_buffer;
    buf->device = backend->device;
    buf->size = total;
    if (hipSetDevice(backend->device) != hipSuccess ||
        (total && hipMalloc(&buf->base, total) != hipSuccess)) {
        delete buf;
        return nullptr;
    }
    size_t off = 0;
    for (auto& t : ctx->tensors)
        if (!t.data) {
            t.data = static_cast<char*>(buf->base) + off;
            t.buffer = buf;
            off += align_up(ggml_nbytes(&t));
        }
    return buf;
}

void ggml_backend_buffer_free(ggml_backend_buffer_t buffer) {
    if (!buffer) return;
    if (buffer->base) {
        (void)hipSetDevice(buffer->device);
        (void)hipFree(buffer->base);
    }
    delete buffer;
}

size_t ggml_backend_buffer_get_size(ggml_backend_buffer_t buffer) { return buffer->size; }

void ggml_backend_tensor_set(struct ggml_tensor* t, const void* data, size_t offset, size_t size) {
    GGML_ASSERT(t->data && "ggml_backend_tensor_set: tensor has no device memory");
    GGML_ASSERT(offset + size <= ggml_nbytes(t) && "ggml_backend_tensor_set: out of bounds");
    if (!size) return;
    if (t->buffer) (void)hipSetDevice(t->buffer->device);
    hip_check(hipMemcpy(static_cast<char*>(t->data) + offset, data, size, hipMemcpyHostToDevice),
              "ggml_backend_tensor_set");
}

void ggml_backend_tensor_get(const struct ggml_tensor* t, void* data, size_t offset, size_t size) {
    GGML_ASSERT(t->data && "ggml_backend_tensor_get: tensor has no device memory");
    GGML_ASSERT(offset + size <= ggml_nbytes(t) && "ggml_backend_tensor_get: out of bounds");
    if (!size) return;
    if (t->buffer) (void)hipSetDevice(t->buffer->device);
    hip_check(hipMemcpy(data, static_cast<const char*>(t->data) + offset, size,
                        hipMemcpyDeviceToHost),
              "ggml_backend_tensor_get");
}

// ---------------------------------------------------------------------------------------------
// graph allocator: one device buffer per graph; intermediate results share memory once their
// last consumer has run (first fit over a free list, like ggml's gallocr)
// ---------------------------------------------------------------------------------------------
struct ggml_gallocr {
    ggml_backend_buffer_type* buft = nullptr;
    ggml_backend_buffer buffer;   // base / size of the current allocation
};

namespace {
class Arena {
public:
    size_t alloc(size_t size) {
        size = align_up(std::max<size_t>(size, 1));
        auto best = free_.end();
        for (auto it = free_.begin(); it != free_.end(); ++it)
            if (it->second >= size && (best == free_.end() || it->second < best->second)) best = it;
        if (best != free_.end()) {
            const size_t off = best->first, rest = best->second - size;
            free_.erase(best);
            if (rest) free_[off + size] = rest;
            return off;
        }
        const size_t off = top_;
        top_ += size;
        peak_ = std::max(peak_, top_);
        return off;
    }
    void release(size_t off, size_t size) {
        size = align_up(std::max<size_t>(size, 1));
        auto it = free_.emplace(off, size).first;
        auto next = std::next(it);
        if (next != free_.end() && it->first + it->second == next->first) {
            it->second += next->second;
            free_.erase(next);
        }
        if (it != free_.begin()) {
            auto prev = std::prev(it);
            if (prev->first + prev->second == it->first) {
                prev->second += it->second;
                free_.erase(it);
                it = prev;
            }
        }
        if (it->first + it->second == top_) {
            top_ = it->first;
            free_.erase(it);
        }
    }
    size_t peak() const { return peak_; }

private:
    std::map<size_t, size_t> free_;
    size_t top_ = 0, peak_ = 0;
};
}  // namespace

ggml_gallocr_t ggml_gallocr_new(ggml_backend_buffer_type_t buft) {
    auto* g = new ggml_gallocr;
    g->buft = buft;
    g->buffer.device = buft->device;
    return g;
}

void ggml_gallocr_free(ggml_gallocr_t galloc) {
    if (!galloc) return;
    if (galloc->buffer.base) {
        (void)hipSetDevice(galloc->buffer.device);
        (void)hipFree(galloc->buffer.base);
    }
    delete galloc;
}

size_t ggml_gallocr_get_buffer_size(ggml_gallocr_t galloc, int buffer_id) {
    return buffer_id == 0 ? galloc->buffer.size : 0;
}

bool ggml_gallocr_alloc_graph(ggml_gallocr_t galloc, struct ggml_cgraph* g) {
    // last node index that reads each tensor
    std::unordered_map<const ggml_tensor*, int> last_use;
    std::unordered_set<const ggml_tensor*> consumed;
    for (int i = 0; i < (int)g->nodes.size(); ++i)
        for (ggml_tensor* s : g->nodes[i]->src)
            if (s) {
                last_use[s] = i;
                consumed.insert(s);
            }
    Arena arena;
    std::unordered_map<const ggml_tensor*, size_t> offset;
    std::vector<std::pair<ggml_tensor*, size_t>> scratch;   // node, offset
    for (ggml_tensor* t : g->leafs)
        if (!t->data) offset[t] = arena.alloc(ggml_nbytes(t));   // inputs live for the whole graph
    for (int i = 0; i < (int)g->nodes.size(); ++i) {
        ggml_tensor* t = g->nodes[i];
        const bool placed_here = !t->data;
        if (placed_here) offset[t] = arena.alloc(ggml_nbytes(t));
        size_t soff = 0;
        if (t->op == GGML_OP_CUSTOM && t->custom_scratch) soff = arena.alloc(t->custom_scratch);
        if (t->op == GGML_OP_CUSTOM && t->custom_scratch) {
            scratch.push_back({t, soff});
            arena.release(soff, t->custom_scratch);
        }
        // free the sources whose last consumer this node is (intermediates only)
        for (ggml_tensor* s : t->src) {
            if (!s || s->op == GGML_OP_NONE || (s->flags & GGML_TENSOR_FLAG_OUTPUT)) continue;
            auto lu = last_use.find(s);
            auto of = offset.find(s);
            if (lu != last_use.end() && lu->second == i && of != offset.end()) {
                arena.release(of->second, ggml_nbytes(s));
                last_use.erase(lu);   // release once even if s appears twice among the sources
            }
        }
        // a node nobody reads is a result: it keeps its memory
        if (placed_here && !consumed.count(t)) t->flags |= GGML_TENSOR_FLAG_OUTPUT;
    }
    const size_t need = arena.peak();
    if (need > galloc->buffer.size) {
        (void)hipSetDevice(galloc->buffer.device);
        if (galloc->buffer.base) (void)hipFree(galloc->buffer.base);
        galloc->buffer.base = nullptr;
        galloc->buffer.size = 0;
        if (hipMalloc(&galloc->buffer.base, need) != hipSuccess) {
            fprintf(stderr, "ggml_gallocr_alloc_graph: cannot allocate %zu bytes\n", need);
            return false;
        }
        galloc->buffer.size = need;
    }
    char* base = static_cast<char*>(galloc->buffer.base);
    for (auto& [t, off] : offset) {
        auto* tt = const_cast<ggml_tensor*>(t);
        tt->data = base + off;
        tt->buffer = &galloc->buffer;
    }
    for (auto& [t, off] : scratch) t->extra = base + off;
    return true;
}

// ---------------------------------------------------------------------------------------------
// compute
// ---------------------------------------------------------------------------------------------
static void run_node(ggml_tensor* t, hipStream_t s) {
    ggml_tensor* a = t->src[0];
    ggml_tensor* b = t->src[1];
    auto lib = [](int st, const char* what) {
        if (st != TSP_OK) fail(std::string(what) + ": " + tsp_last_error());
    };
    auto need_contig = [](const ggml_tensor* x) {
        if (x && !is_contiguous(x)) fail("graph compute: non-contiguous operand");
    };
    need_contig(a);
    need_contig(b);
    switch (t->op) {
        case GGML_OP_ADD:
        case GGML_OP_MUL:
            hip_check(launch_binary(t->op == GGML_OP_MUL, a, b, static_cast<float*>(t->data), s),
                      "add/mul");
            break;
        case GGML_OP_SILU:
            hip_check(launch_silu(static_cast<const float*>(a->data), static_cast<float*>(t->data),
                                  ggml_nelements(a), s),
                      "silu");
            break;
        case GGML_OP_NORM: {
            float eps;
            memcpy(&eps, &t->op_params[0], sizeof(float));
            lib(tsp_layer_norm(a->data, tsp_dtype_of(a->type), ggml_nelements(a) / a->ne[0],
                               (int)a->ne[0], nullptr, nullptr, eps, 0, t->data, TSP_F32, s),
                "norm");
            break;
        }
        case GGML_OP_MUL_MAT: {
            // F16 / BF16 weights take their input rounded to their own type (the CPU backend's
            // vec_dot type), F32 weights the input as it is
            const int adt = tsp_dtype_of(a->type), bdt = tsp_dtype_of(b->type);
            const int64_t nb = ggml_nelements(b);
            const void* x = b->data;
            int xdt = bdt;
            DeviceBuffer rounded;
            if (bdt == TSP_F32 && (adt == TSP_F16 || adt == TSP_BF16) && nb > 0) {
                rounded = DeviceBuffer((size_t)nb * 2, s);
                hip_check(launch_convert(b->data, TSP_F32, rounded.get(), adt, nb, s), "mul_mat rounding");
                x = rounded.get();
                xdt = adt;
            }
            lib(tsp_linear(x, xdt, b->ne[1], (int)b->ne[0], a->data, adt, nullptr, (int)a->ne[1], t->data,
                           TSP_F32, s),
                "mul_mat");
            break;
        }
        case GGML_OP_GET_ROWS:
            hip_check(launch_get_rows(a, static_cast<const int32_t*>(b->data), b->ne[0], t->data, s),
                      "get_rows");
            break;
        case GGML_OP_CONCAT: {
            const size_t na = ggml_nbytes(a), nb = ggml_nbytes(b);
            if (na) hip_check(hipMemcpyAsync(t->data, a->data, na, hipMemcpyDeviceToDevice, s), "concat");
            if (nb)
                hip_check(hipMemcpyAsync(static_cast<char*>(t->data) + na, b->data, nb,
                                         hipMemcpyDeviceToDevice, s),
                          "concat");
            break;
        }
        case GGML_OP_CUSTOM:
            if (t->custom_scratch && !t->extra) fail("graph compute: custom node has no scratch");
            if (t->custom_fn(t, s, t->extra, t->custom_userdata) != 0)
                fail(std::string("custom node '") + t->name + "' failed");
            break;
        default:
            fail("graph compute: unsupported op");
    }
}

enum ggml_status ggml_backend_graph_compute(ggml_backend_t backend, struct ggml_cgraph* g) {
    try {
        hip_check(hipSetDevice(backend->device), "hipSetDevice");
        for (ggml_tensor* t : g->nodes) {
            if (!t->data && ggml_nelements(t) > 0)
                fail("graph compute: node without device memory (run ggml_gallocr_alloc_graph)");
            for (ggml_tensor* src : t->src)
                if (src && !src->data && ggml_nelements(src) > 0)
                    fail(std::string("graph compute: source without device memory: ") + src->name);
            if (ggml_nelements(t) == 0) continue;
            run_node(t, backend->stream);
        }
        hip_check(hipStreamSynchronize(backend->stream), "graph compute");
    } catch (const std::exception& e) {
        fprintf(stderr, "ggml_backend_graph_compute: %s\n", e.what());
        return GGML_STATUS_FAILED;
    }
    return GGML_STATUS_SUCCESS;
}

// ---------------------------------------------------------------------------------------------
// fp16 conversion on the host (IEEE binary16, round to nearest even)
// ---------------------------------------------------------------------------------------------
float ggml_fp16_to_fp32(ggml_fp16_t h) {
    const uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    uint32_t exp = (h >> 10) & 0x1fu, man = h & 0x3ffu, bits;
    if (exp == 0x1f) {
        bits = sign | 0x7f800000u | (man << 13);
    } else if (exp != 0) {
        bits = sign | ((exp + 112u) << 23) | (man << 13);
    } else if (man == 0) {
        bits = sign;
    } else {   // subnormal: normalise
        int e = -1;
        do {
            ++e;
            man <<= 1;
        } while (!(man & 0x400u));
        bits = sign | ((uint32_t)(112 - e) << 23) | ((man & 0x3ffu) << 13);
    }
    float f;
    memcpy(&f, &bits, 4);
    return f;
}

ggml_fp16_t ggml_fp32_to_fp16(float f) {
    uint32_t x;
    memcpy(&x, &f, 4);
    const uint32_t sign = (x >> 16) & 0x8000u;
    const uint32_t ax = x & 0x7fffffffu;
    if (ax > 0x7f800000u) return (ggml_fp16_t)(sign | 0x7e00u);   // NaN
    if (ax >= 0x477ff000u) return (ggml_fp16_t)(sign | 0x7c00u);  // rounds to >= 65520: inf
    if (ax >= 0x38800000u) {                                       // normal half
        const uint32_t r = ax + 0x0fffu + ((ax >> 13) & 1u) - (112u << 23);
        return (ggml_fp16_t)(sign | (r >> 13));
    }
    if (ax < 0x33000000u) return (ggml_fp16_t)sign;                // < 2^-25: zero
    // subnormal half: value = m * 2^-24
    const uint32_t e = ax >> 23, m = (ax & 0x7fffffu) | 0x800000u;
    const int shift = (int)(126 - e);   // 14..24
    const uint32_t q = m >> shift, rem = m & ((1u << shift) - 1u), half = 1u << (shift - 1);
    const uint32_t r = q + ((rem > half || (rem == half && (q & 1u))) ? 1u : 0u);
    return (ggml_fp16_t)(sign | r);
}

void ggml_fp16_to_fp32_row(const ggml_fp16_t* x, float* y, int64_t n) {
    for (int64_t i = 0; i < n; ++i) y[i] = ggml_fp16_to_fp32(x[i]);
}

void ggml_fp32_to_fp16_row(const float* x, ggml_fp16_t* y, int64_t n) {
    for (int64_t i = 0; i < n; ++i) y[i] = ggml_fp32_to_fp16(x[i]);
}

}  // extern "C"
