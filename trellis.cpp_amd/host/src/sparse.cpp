// trellis::build_neighbor_table / sparse_submconv / sparse_convnext / sparse_c2s
// (include/sparse.h:14-35, src/sparse.cpp:21-336 of the reference) on libtrellis_sparse.
//
// The reference expresses a conv as 27 x (get_rows -> mul_mat -> add) graph nodes and a
// ConvNeXt block as ~10 more; here each is ONE custom node that runs the fused kernels:
//   * a conv plan node per neighbour table and graph context (the tile row sets the matrix-core
//     kernel stages in LDS), shared by every conv that reads the same table;
//   * a conv node (ops::run_conv);
//   * a ConvNeXt node (ops::run_convnext): conv, LayerNorm(1e-6)+affine, the two linears with
//     SiLU, and the residual, chunked over voxels so the [nr, 4C] hidden stays bounded.
// sparse_c2s runs the whole up-block on the device (ops::run_c2s) and reads back its results.
#include "sparse.h"

#include <cstdio>
#include <cstring>
#include <memory>
#include <stdexcept>

#include "ggml-backend.h"
#include "ggml.h"
#include "runtime.hpp"
#include "sparse_ops.hpp"
#include "trellis_model.h"

namespace trellis {

bool g_sparse_cast_f32 = false;

namespace {

using ops::Carve;
using tgr::DeviceBuffer;
using tgr::fail;
using tgr::hip_check;

enum { kMemoPlan = 1 };

// ---- conv plan node ----------------------------------------------------------------------------
struct PlanArgs {
    int64_t n;
};

int plan_fn(ggml_tensor* dst, void* stream, void*, void* ud) {
    const auto* a = static_cast<const PlanArgs*>(ud);
    const int st = tsp_conv_plan_build(static_cast<const int32_t*>(dst->src[0]->data), a->n, dst->data,
                                       ggml_nbytes(dst), stream);
    if (st != TSP_OK) fprintf(stderr, "conv plan: %s\n", tsp_last_error());
    return st;
}

ggml_tensor* plan_node(ggml_context* ctx, ggml_tensor* nbr, int64_t n) {
    if (ggml_tensor* p = tgr::context_memo_get(ctx, nbr, kMemoPlan)) return p;
    auto args = std::make_shared<PlanArgs>(PlanArgs{n});
    tgr::context_keep(ctx, args);
    const int64_t ne[1] = {(int64_t)(tsp_conv_plan_bytes(n) / 4)};
    ggml_tensor* srcs[1] = {nbr};
    ggml_tensor* p = ggml_custom(ctx, GGML_TYPE_I32, 1, ne, srcs, 1, plan_fn, args.get(), 0);
    ggml_set_name(p, "conv_plan");
    tgr::context_memo_put(ctx, nbr, kMemoPlan, p);
    return p;
}

void check_graph_inputs(const ggml_tensor* feats, const ggml_tensor* nbr, int ci, int64_t n,
                        const std::string& prefix) {
    if (feats->ne[0] != ci || feats->ne[1] != n || feats->ne[2] != 1 || feats->ne[3] != 1)
        fail(prefix + ": feats must be ggml [" + std::to_string(ci) + ", " + std::to_string(n) + "]");
    if (tgr::tsp_dtype_of(feats->type) < 0) fail(prefix + ": feats must be F32, F16 or BF16");
    if (nbr->type != GGML_TYPE_I32 || ggml_nelements(nbr) != 27 * n)
        fail(prefix + ": nbr must be I32 with 27*N elements");
}

// ---- conv node ---------------------------------------------------------------------------------
struct ConvArgs {
    ops::Conv conv;
    int64_t n;
};

int conv_fn(ggml_tensor* dst, void* stream, void* scratch, void* ud) {
    const auto* a = static_cast<const ConvArgs*>(ud);
    try {
        Carve sc(scratch);
        const ggml_tensor* f = dst->src[0];
        ops::run_conv(a->conv, f->data, tgr::tsp_dtype_of(f->type), a->n,
                      static_cast<const int32_t*>(dst->src[1]->data), dst->src[2] ? dst->src[2]->data : nullptr,
                      static_cast<float*>(dst->data), sc, static_cast<hipStream_t>(stream));
    } catch (const std::exception& e) {
        fprintf(stderr, "sparse_submconv: %s\n", e.what());
        return 1;
    }
    return 0;
}

// ---- ConvNeXt node -----------------------------------------------------------------------------
int convnext_fn(ggml_tensor* dst, void* stream, void* scratch, void* ud) {
    const auto* a = static_cast<const ops::ConvNext*>(ud);
    try {
        Carve sc(scratch);
        const ggml_tensor* f = dst->src[0];
        ops::run_convnext(*a, f->data, tgr::tsp_dtype_of(f->type), static_cast<const int32_t*>(dst->src[1]->data),
                          dst->src[2] ? dst->src[2]->data : nullptr, static_cast<float*>(dst->data), sc,
                          static_cast<hipStream_t>(stream));
    } catch (const std::exception& e) {
        fprintf(stderr, "sparse_convnext: %s\n", e.what());
        return 1;
    }
    return 0;
}

}  // namespace

// -------------------------------------------------------------------------------------------------
std::vector<int32_t> build_neighbor_table(const std::vector<std::array<int, 3>>& coords) {
    static_assert(sizeof(std::array<int, 3>) == 12, "coords must be packed int32 triples");
    const int64_t n = (int64_t)coords.size();
    std::vector<int32_t> nbr((size_t)27 * n);
    if (n == 0) return nbr;
    DeviceBuffer d_coords((size_t)n * 12);
    hip_check(hipMemcpy(d_coords.get(), coords.data(), (size_t)n * 12, hipMemcpyHostToDevice),
              "build_neighbor_table upload");
    ops::Table t;
    ops::build_table(d_coords.as<int32_t>(), n, t, nullptr);
    hip_check(hipMemcpy(nbr.data(), t.nbr.get(), nbr.size() * 4, hipMemcpyDeviceToHost),
              "build_neighbor_table download");
    return nbr;
}

ggml_tensor* sparse_submconv(ggml_context* ctx, const Model& m, const std::string& prefix,
                             ggml_tensor* feats, ggml_tensor* nbr, int N) {
    auto args = std::make_shared<ConvArgs>(ConvArgs{ops::conv_of(m, prefix), N});
    const ops::Conv& c = args->conv;
    check_graph_inputs(feats, nbr, c.ci, N, prefix);
    tgr::context_keep(ctx, args);
    ggml_tensor* srcs[3] = {feats, nbr, c.mfma ? plan_node(ctx, nbr, N) : nullptr};
    const int64_t ne[2] = {c.co, N};
    ggml_tensor* t = ggml_custom(ctx, GGML_TYPE_F32, 2, ne, srcs, c.mfma ? 3 : 2, conv_fn, args.get(),
                                 ops::conv_scratch(c, N, tgr::tsp_dtype_of(feats->type)));
    ggml_set_name(t, (prefix + ".out").substr(0, GGML_MAX_NAME - 1).c_str());
    return t;
}

ggml_tensor* sparse_convnext(ggml_context* ctx, const Model& m, const std::string& prefix,
                             ggml_tensor* feats, ggml_tensor* nbr, int N) {
    auto a = std::make_shared<ops::ConvNext>(ops::convnext_of(m, prefix, N));
    check_graph_inputs(feats, nbr, a->c, N, prefix);
    tgr::context_keep(ctx, a);
    ggml_tensor* srcs[3] = {feats, nbr, a->conv.mfma ? plan_node(ctx, nbr, N) : nullptr};
    const int64_t ne[2] = {a->c, N};
    ggml_tensor* t = ggml_custom(ctx, GGML_TYPE_F32, 2, ne, srcs, a->conv.mfma ? 3 : 2, convnext_fn, a.get(),
                                 ops::convnext_scratch(*a, tgr::tsp_dtype_of(feats->type)));
    ggml_set_name(t, (prefix + ".out").substr(0, GGML_MAX_NAME - 1).c_str());
    return t;
}

C2SResult sparse_c2s(const Model& m, const std::string& prefix, const std::vector<float>& feats_in,
                     int Cin, const std::vector<std::array<int, 3>>& coords, int Cout,
                     const std::vector<uint8_t>* ext_subdiv) {
    const int64_t n = (int64_t)coords.size();
    if ((int64_t)feats_in.size() != n * Cin) fail(prefix + ": feats_in must hold Cin*N floats");
    C2SResult r;
    r.C = Cout;
    if (n == 0) return r;
    hip_check(hipSetDevice(tgr::backend_device(m.backend)), "hipSetDevice");
    hipStream_t s = tgr::backend_stream(m.backend);
    DeviceBuffer d_coords((size_t)n * 12), d_x((size_t)n * Cin * 4);
    hip_check(hipMemcpy(d_coords.get(), coords.data(), (size_t)n * 12, hipMemcpyHostToDevice), "c2s upload");
    hip_check(hipMemcpy(d_x.get(), feats_in.data(), (size_t)n * Cin * 4, hipMemcpyHostToDevice), "c2s upload");
    ops::Table parent;
    ops::build_table(d_coords.as<int32_t>(), n, parent, s);
    ops::C2SOut o = ops::run_c2s(m, prefix, d_x.as<float>(), d_coords.as<int32_t>(), parent, Cin, Cout,
                                 ext_subdiv, s);
    r.subdiv = std::move(o.mask);
    r.feats.resize((size_t)o.m * Cout);
    r.coords.resize((size_t)o.m);
    if (o.m) {
        hip_check(hipMemcpy(r.feats.data(), o.feats.get(), r.feats.size() * 4, hipMemcpyDeviceToHost),
                  "c2s readback");
        hip_check(hipMemcpy(r.coords.data(), o.coords.get(), (size_t)o.m * 12, hipMemcpyDeviceToHost),
                  "c2s readback");
    }
    return r;
}

}  // namespace trellis
