// trellis::build_neighbor_table / sparse_submconv / sparse_convnext / sparse_c2s
// (include/sparse.h:14-35, src/sparse.cpp:21-336 of the reference) on libtrellis_sparse.
//
// The reference expresses a conv as 27 x (get_rows -> mul_mat -> add) graph nodes and a
// ConvNeXt block as ~10 more; here each is ONE custom node that runs the fused kernels:
//   * a conv plan node per neighbour table and graph context (the tile row sets the matrix-core
//     kernel stages in LDS), shared by every conv that reads the same table;
//   * a conv node: F32 activations rounded to the weights' 16-bit type (what ggml's F16 mul_mat
//     does to its F32 operand), weights packed for the MFMA operand order, one planned conv
//     with fp32 accumulation; fp32 VALU conv when g_sparse_cast_f32 is set or the channel counts
//     do not fit the matrix-core tiles;
//   * a ConvNeXt node: conv, LayerNorm(1e-6)+affine in place, the two linears with SiLU, and
//     the residual, chunked over voxels so the [nr, 4C] hidden stays bounded.
// sparse_c2s runs the whole up-block on the device (rulebooks, mask, subdivision, both convs,
// the octant gather and the skip) and reads back only its results.
#include "sparse.h"

#include <algorithm>
#include <cstring>
#include <stdexcept>

#include "ggml-backend.h"
#include "ggml.h"
#include "runtime.hpp"
#include "trellis_model.h"

namespace trellis {

bool g_sparse_cast_f32 = false;

namespace {

using tgr::align_up;
using tgr::DeviceBuffer;
using tgr::fail;
using tgr::hip_check;

void lib(int st, const std::string& what) {
    if (st != TSP_OK) fail(what + ": " + tsp_last_error());
}

// Scratch carving: the same walk sizes a buffer (a default-constructed Carve: nothing runs)
// and, over the real buffer, hands out its pieces while the work runs.
struct Carve {
    char* base = nullptr;
    size_t off = 0;
    bool sizing = true;
    Carve() = default;
    explicit Carve(void* b) : base(static_cast<char*>(b)), sizing(false) {}
    bool running() const { return !sizing; }
    void* take(size_t bytes) {
        void* p = sizing ? nullptr : base + off;
        off += align_up(bytes);
        return p;
    }
};

enum { kMemoPlan = 1 };

// A conv's weights as the graph sees them.
struct Conv {
    const ggml_tensor* w = nullptr;   // ggml [Ci, 27, Co]
    const ggml_tensor* b = nullptr;   // [Co]
    int ci = 0, co = 0, wdt = 0;
    bool mfma = false;
};

Conv conv_of(const Model& m, const std::string& prefix) {
    Conv c;
    c.w = m.get(prefix + ".weight");
    c.b = m.get(prefix + ".bias");
    if (c.w->ne[1] != 27 || c.w->ne[3] != 1)
        fail(prefix + ".weight: expected ggml shape [Ci, 27, Co]");
    c.ci = (int)c.w->ne[0];
    c.co = (int)c.w->ne[2];
    if (ggml_nelements(c.b) != c.co) fail(prefix + ".bias: expected " + std::to_string(c.co) + " elements");
    c.wdt = tgr::tsp_dtype_of(c.w->type);
    if (c.wdt < 0) fail(prefix + ".weight: unsupported tensor type");
    c.mfma = !g_sparse_cast_f32 && (c.wdt == TSP_F16 || c.wdt == TSP_BF16) && c.ci % 16 == 0 &&
             c.co % 64 == 0;
    return c;
}

// Float32 view of a 1-D parameter (converted into scratch when stored in 16 bits).
const float* f32_param(const ggml_tensor* t, Carve& sc, hipStream_t s) {
    if (t->type == GGML_TYPE_F32) return static_cast<const float*>(t->data);
    void* p = sc.take((size_t)ggml_nelements(t) * 4);
    if (sc.running()) hip_check(tgr::launch_convert(t->data, tgr::tsp_dtype_of(t->type), p, TSP_F32,
                                         ggml_nelements(t), s),
                     "parameter conversion");
    return static_cast<const float*>(p);
}

// out [n][co] f32 = conv(feats [n][ci] of dtype fdt). Walks `sc` the same way when sizing.
void run_conv(const Conv& c, const void* feats, int fdt, int64_t n, const int32_t* nbr,
              const void* plan, float* out, Carve& sc, hipStream_t s) {
    const float* bias = f32_param(c.b, sc, s);
    if (c.mfma) {
        const void* x = feats;
        if (fdt != c.wdt) {
            void* x16 = sc.take((size_t)n * c.ci * 2);
            if (sc.running()) hip_check(tgr::launch_convert(feats, fdt, x16, c.wdt, n * c.ci, s), "conv input rounding");
            x = x16;
        }
        void* packed = sc.take((size_t)27 * c.ci * c.co * 2);
        if (!sc.running()) return;
        lib(tsp_conv_weight_pack(c.w->data, c.wdt, c.ci, c.co, packed, s), "weight pack");
        lib(tsp_subm_conv3x3_planned(x, c.wdt, n, c.ci, nbr, plan, packed, bias, c.co, out, TSP_F32, s),
            "sparse conv");
    } else {
        if (!sc.running()) return;
        lib(tsp_subm_conv3x3(feats, fdt, n, c.ci, nbr, c.w->data, c.wdt, bias, c.co, out, TSP_F32,
                             TSP_ALGO_AUTO, s),
            "sparse conv");
    }
}

size_t conv_scratch(const Conv& c, int64_t n, int fdt) {
    Carve sz;
    run_conv(c, nullptr, fdt, n, nullptr, nullptr, nullptr, sz, nullptr);
    return sz.off;
}

// ---- conv plan node --------------------------------------------------------------------------
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
    const size_t bytes = tsp_conv_plan_bytes(n);
    const int64_t ne[1] = {(int64_t)(bytes / 4)};
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

// ---- conv node -------------------------------------------------------------------------------
struct ConvArgs {
    Conv conv;
    int64_t n;
};

int conv_fn(ggml_tensor* dst, void* stream, void* scratch, void* ud) {
    const auto* a = static_cast<const ConvArgs*>(ud);
    try {
        Carve sc(scratch);
        const ggml_tensor* f = dst->src[0];
        run_conv(a->conv, f->data, tgr::tsp_dtype_of(f->type), a->n,
                 static_cast<const int32_t*>(dst->src[1]->data), dst->src[2] ? dst->src[2]->data : nullptr,
                 static_cast<float*>(dst->data), sc, static_cast<hipStream_t>(stream));
    } catch (const std::exception& e) {
        fprintf(stderr, "sparse_submconv: %s\n", e.what());
        return 1;
    }
    return 0;
}

// ---- ConvNeXt node ---------------------------------------------------------------------------
struct ConvNextArgs {
    Conv conv;
    const ggml_tensor *nw, *nb, *w0, *b0, *w2, *b2;
    int64_t n;
    int c;
    int64_t chunk;
};

// Sizes the block's scratch (a sizing Carve) or runs it.
void run_convnext(const ConvNextArgs& a, const void* feats, int fdt, const int32_t* nbr,
                  const void* plan, float* out, Carve& sc, hipStream_t s) {
    const int c = a.c;
    float* h = static_cast<float*>(sc.take((size_t)a.n * c * 4));
    float* hid = static_cast<float*>(sc.take((size_t)a.chunk * 4 * c * 4));
    const float* gamma = f32_param(a.nw, sc, s);
    const float* beta = f32_param(a.nb, sc, s);
    const float* bias0 = f32_param(a.b0, sc, s);
    const float* bias2 = f32_param(a.b2, sc, s);
    run_conv(a.conv, feats, fdt, a.n, nbr, plan, h, sc, s);
    if (!sc.running()) return;
    lib(tsp_layer_norm(h, TSP_F32, a.n, c, gamma, beta, 1e-6f, 0, h, TSP_F32, s), "convnext norm");
    const int w0dt = tgr::tsp_dtype_of(a.w0->type), w2dt = tgr::tsp_dtype_of(a.w2->type);
    const size_t fes = fdt == TSP_F32 ? 4 : 2;
    for (int64_t r0 = 0; r0 < a.n; r0 += a.chunk) {
        const int64_t nr = std::min(a.chunk, a.n - r0);
        lib(tsp_linear(h + r0 * c, TSP_F32, nr, c, a.w0->data, w0dt, bias0, 4 * c, hid, TSP_F32, s),
            "convnext mlp.0");
        hip_check(tgr::launch_silu(hid, hid, nr * 4 * c, s), "convnext silu");
        lib(tsp_linear(hid, TSP_F32, nr, 4 * c, a.w2->data, w2dt, bias2, c, out + r0 * c, TSP_F32, s),
            "convnext mlp.2");
        hip_check(tgr::launch_add_inplace(out + r0 * c,
                                          static_cast<const char*>(feats) + (size_t)r0 * c * fes,
                                          fdt, nr * c, s),
                  "convnext residual");
    }
}

int convnext_fn(ggml_tensor* dst, void* stream, void* scratch, void* ud) {
    const auto* a = static_cast<const ConvNextArgs*>(ud);
    try {
        Carve sc(scratch);
        const ggml_tensor* f = dst->src[0];
        run_convnext(*a, f->data, tgr::tsp_dtype_of(f->type), static_cast<const int32_t*>(dst->src[1]->data),
                     dst->src[2] ? dst->src[2]->data : nullptr, static_cast<float*>(dst->data), sc,
                     static_cast<hipStream_t>(stream));
    } catch (const std::exception& e) {
        fprintf(stderr, "sparse_convnext: %s\n", e.what());
        return 1;
    }
    return 0;
}

const ggml_tensor* vec_param(const Model& m, const std::string& name, int64_t n) {
    const ggml_tensor* t = m.get(name);
    if (ggml_nelements(t) != n || tgr::tsp_dtype_of(t->type) < 0)
        fail(name + ": expected " + std::to_string(n) + " floating-point elements");
    return t;
}

const ggml_tensor* mat_param(const Model& m, const std::string& name, int64_t k, int64_t rows) {
    const ggml_tensor* t = m.get(name);
    if (t->ne[0] != k || t->ne[1] != rows || t->ne[2] != 1 || t->ne[3] != 1 ||
        tgr::tsp_dtype_of(t->type) < 0)
        fail(name + ": expected ggml shape [" + std::to_string(k) + ", " + std::to_string(rows) + "]");
    return t;
}

}  // namespace

// ---------------------------------------------------------------------------------------------
std::vector<int32_t> build_neighbor_table(const std::vector<std::array<int, 3>>& coords) {
    static_assert(sizeof(std::array<int, 3>) == 12, "coords must be packed int32 triples");
    const int64_t n = (int64_t)coords.size();
    std::vector<int32_t> nbr((size_t)27 * n);
    if (n == 0) return nbr;
    DeviceBuffer d_coords((size_t)n * 12), d_nbr((size_t)n * 27 * 4),
        d_ws(tsp_rulebook_workspace_bytes(n)), d_status(4);
    hip_check(hipMemcpy(d_coords.get(), coords.data(), (size_t)n * 12, hipMemcpyHostToDevice),
              "build_neighbor_table upload");
    hip_check(hipMemset(d_status.get(), 0, 4), "build_neighbor_table");
    lib(tsp_rulebook_build(d_coords.as<int32_t>(), n, d_nbr.as<int32_t>(), d_ws.get(), d_ws.size(),
                           d_status.as<int32_t>(), nullptr),
        "build_neighbor_table");
    int32_t status = 0;
    hip_check(hipMemcpy(&status, d_status.get(), 4, hipMemcpyDeviceToHost), "build_neighbor_table");
    if (status) fail("build_neighbor_table: a coordinate lies outside [0, 2^21-3]");
    hip_check(hipMemcpy(nbr.data(), d_nbr.get(), nbr.size() * 4, hipMemcpyDeviceToHost),
              "build_neighbor_table download");
    return nbr;
}

ggml_tensor* sparse_submconv(ggml_context* ctx, const Model& m, const std::string& prefix,
                             ggml_tensor* feats, ggml_tensor* nbr, int N) {
    auto args = std::make_shared<ConvArgs>(ConvArgs{conv_of(m, prefix), N});
    const Conv& c = args->conv;
    check_graph_inputs(feats, nbr, c.ci, N, prefix);
    tgr::context_keep(ctx, args);
    ggml_tensor* srcs[3] = {feats, nbr, c.mfma ? plan_node(ctx, nbr, N) : nullptr};
    const int64_t ne[2] = {c.co, N};
    ggml_tensor* t = ggml_custom(ctx, GGML_TYPE_F32, 2, ne, srcs, c.mfma ? 3 : 2, conv_fn,
                                 args.get(), conv_scratch(c, N, tgr::tsp_dtype_of(feats->type)));
    ggml_set_name(t, (prefix + ".out").substr(0, GGML_MAX_NAME - 1).c_str());
    return t;
}

ggml_tensor* sparse_convnext(ggml_context* ctx, const Model& m, const std::string& prefix,
                             ggml_tensor* feats, ggml_tensor* nbr, int N) {
    auto a = std::make_shared<ConvNextArgs>();
    a->conv = conv_of(m, prefix + ".conv");
    const int c = a->conv.co;
    if (a->conv.ci != c) fail(prefix + ".conv: a ConvNeXt conv keeps the channel count");
    check_graph_inputs(feats, nbr, c, N, prefix);
    a->nw = vec_param(m, prefix + ".norm.weight", c);
    a->nb = vec_param(m, prefix + ".norm.bias", c);
    a->w0 = mat_param(m, prefix + ".mlp.0.weight", c, 4 * (int64_t)c);
    a->b0 = vec_param(m, prefix + ".mlp.0.bias", 4 * (int64_t)c);
    a->w2 = mat_param(m, prefix + ".mlp.2.weight", 4 * (int64_t)c, c);
    a->b2 = vec_param(m, prefix + ".mlp.2.bias", c);
    a->n = N;
    a->c = c;
    // the [chunk, 4C] f32 hidden is bounded to 1 GiB
    a->chunk = std::max<int64_t>(1, std::min<int64_t>(N, (int64_t(1) << 30) / (16 * (int64_t)c)));
    tgr::context_keep(ctx, a);
    Carve sz;
    run_convnext(*a, nullptr, tgr::tsp_dtype_of(feats->type), nullptr, nullptr, nullptr, sz, nullptr);
    ggml_tensor* srcs[3] = {feats, nbr, a->conv.mfma ? plan_node(ctx, nbr, N) : nullptr};
    const int64_t ne[2] = {c, N};
    ggml_tensor* t = ggml_custom(ctx, GGML_TYPE_F32, 2, ne, srcs, a->conv.mfma ? 3 : 2, convnext_fn,
                                 a.get(), sz.off);
    ggml_set_name(t, (prefix + ".out").substr(0, GGML_MAX_NAME - 1).c_str());
    return t;
}

// ---------------------------------------------------------------------------------------------
C2SResult sparse_c2s(const Model& m, const std::string& prefix, const std::vector<float>& feats_in,
                     int Cin, const std::vector<std::array<int, 3>>& coords, int Cout,
                     const std::vector<uint8_t>* ext_subdiv) {
    const int64_t n = (int64_t)coords.size();
    if (Cin <= 0 || Cin % 8 != 0 || Cout <= 0 || Cout % (Cin / 8) != 0)
        fail(prefix + ": C2S needs Cin % 8 == 0 and Cout % (Cin/8) == 0");
    if ((int64_t)feats_in.size() != n * Cin) fail(prefix + ": feats_in must hold Cin*N floats");
    if (ext_subdiv && (int64_t)ext_subdiv->size() != 8 * n) fail(prefix + ": ext_subdiv must hold 8*N entries");
    C2SResult r;
    r.C = Cout;
    if (n == 0) return r;

    Conv conv1 = conv_of(m, prefix + ".conv1"), conv2 = conv_of(m, prefix + ".conv2");
    if (conv1.ci != Cin || conv1.co != 8 * Cout || conv2.ci != Cout || conv2.co != Cout)
        fail(prefix + ": conv1 must map Cin -> 8*Cout and conv2 Cout -> Cout");
    const ggml_tensor* n1w = vec_param(m, prefix + ".norm1.weight", Cin);
    const ggml_tensor* n1b = vec_param(m, prefix + ".norm1.bias", Cin);

    hip_check(hipSetDevice(tgr::backend_device(m.backend)), "hipSetDevice");
    hipStream_t s = tgr::backend_stream(m.backend);

    // ---- inputs, parent rulebook, subdivision mask
    DeviceBuffer d_coords((size_t)n * 12), d_x((size_t)n * Cin * 4), d_mask((size_t)8 * n);
    hip_check(hipMemcpy(d_coords.get(), coords.data(), (size_t)n * 12, hipMemcpyHostToDevice), "c2s upload");
    hip_check(hipMemcpy(d_x.get(), feats_in.data(), (size_t)n * Cin * 4, hipMemcpyHostToDevice), "c2s upload");
    DeviceBuffer d_status(4);
    hip_check(hipMemset(d_status.get(), 0, 4), "c2s");
    auto rulebook = [&](const DeviceBuffer& xyz, int64_t cnt, DeviceBuffer& out) {
        DeviceBuffer ws(tsp_rulebook_workspace_bytes(cnt));
        lib(tsp_rulebook_build(xyz.as<int32_t>(), cnt, out.as<int32_t>(), ws.get(), ws.size(),
                               d_status.as<int32_t>(), s),
            prefix + " rulebook");
        hip_check(hipStreamSynchronize(s), "c2s rulebook");   // before `ws` is freed
    };
    DeviceBuffer d_nbr((size_t)27 * n * 4);
    rulebook(d_coords, n, d_nbr);
    if (ext_subdiv) {
        hip_check(hipMemcpy(d_mask.get(), ext_subdiv->data(), (size_t)8 * n, hipMemcpyHostToDevice),
                  "c2s mask upload");
    } else {
        const ggml_tensor* wsub = mat_param(m, prefix + ".to_subdiv.weight", Cin, 8);
        const ggml_tensor* bsub = vec_param(m, prefix + ".to_subdiv.bias", 8);
        DeviceBuffer d_logits((size_t)8 * n * 4), d_b(8 * 4);
        Carve sc(d_b.get());
        const float* b = bsub->type == GGML_TYPE_F32 ? static_cast<const float*>(bsub->data)
                                                     : f32_param(bsub, sc, s);
        lib(tsp_linear(d_x.get(), TSP_F32, n, Cin, wsub->data, tgr::tsp_dtype_of(wsub->type), b, 8,
                       d_logits.get(), TSP_F32, s),
            prefix + ".to_subdiv");
        lib(tsp_mask_positive(d_logits.as<float>(), 8 * n, d_mask.as<uint8_t>(), s), prefix + " mask");
        hip_check(hipStreamSynchronize(s), "c2s mask");
    }

    // ---- children
    DeviceBuffer d_mstart((size_t)(n + 1) * 4), d_child((size_t)8 * n * 12), d_gidx((size_t)8 * n * 4),
        d_m(8), d_sws(tsp_subdivide_workspace_bytes(n));
    lib(tsp_subdivide(d_mask.as<uint8_t>(), d_coords.as<int32_t>(), n, d_mstart.as<int32_t>(),
                      d_child.as<int32_t>(), d_gidx.as<int32_t>(), d_m.as<int64_t>(), d_sws.get(),
                      d_sws.size(), s),
        prefix + " subdivide");
    int64_t mm = 0;
    hip_check(hipMemcpyAsync(&mm, d_m.get(), 8, hipMemcpyDeviceToHost, s), "c2s");
    hip_check(hipStreamSynchronize(s), "c2s");
    r.subdiv.resize((size_t)8 * n);
    hip_check(hipMemcpy(r.subdiv.data(), d_mask.get(), (size_t)8 * n, hipMemcpyDeviceToHost), "c2s mask");
    if (mm == 0) return r;

    // ---- conv1 on the parents: LN(norm1)+SiLU written straight in the conv's input dtype
    Carve sz;
    const int in1 = conv1.mfma ? conv1.wdt : TSP_F32, in2 = conv2.mfma ? conv2.wdt : TSP_F32;
    const size_t es1 = in1 == TSP_F32 ? 4 : 2, es2 = in2 == TSP_F32 ? 4 : 2;
    sz.take((size_t)n * Cin * es1);                       // h0
    sz.take((size_t)n * 8 * Cout * 4);                    // conv1 out
    sz.take(conv1.mfma ? tsp_conv_plan_bytes(n) : 0);     // plan 1
    sz.take(conv_scratch(conv1, n, in1));
    sz.take((size_t)mm * Cout * 4);                       // gathered
    sz.take((size_t)mm * Cout * es2);                     // normed
    sz.take((size_t)27 * mm * 4);                         // child table
    sz.take(conv2.mfma ? tsp_conv_plan_bytes(mm) : 0);    // plan 2
    sz.take(conv_scratch(conv2, mm, in2));
    sz.take((size_t)mm * Cout * 4);                       // out
    sz.take(2 * (size_t)Cin * 4);                         // norm1 params as f32
    DeviceBuffer work(sz.off);
    Carve w(work.get());
    void* h0 = w.take((size_t)n * Cin * es1);
    float* h1 = static_cast<float*>(w.take((size_t)n * 8 * Cout * 4));
    void* plan1 = w.take(conv1.mfma ? tsp_conv_plan_bytes(n) : 0);
    Carve sc1(w.take(conv_scratch(conv1, n, in1)));
    float* g = static_cast<float*>(w.take((size_t)mm * Cout * 4));
    void* h2 = w.take((size_t)mm * Cout * es2);
    int32_t* nbr2 = static_cast<int32_t*>(w.take((size_t)27 * mm * 4));
    void* plan2 = w.take(conv2.mfma ? tsp_conv_plan_bytes(mm) : 0);
    Carve sc2(w.take(conv_scratch(conv2, mm, in2)));
    float* out = static_cast<float*>(w.take((size_t)mm * Cout * 4));
    Carve scp(w.take(2 * (size_t)Cin * 4));
    const float* g1 = f32_param(n1w, scp, s);
    const float* b1 = f32_param(n1b, scp, s);

    lib(tsp_layer_norm(d_x.get(), TSP_F32, n, Cin, g1, b1, 1e-6f, 1, h0, in1, s), prefix + ".norm1");
    if (conv1.mfma)
        lib(tsp_conv_plan_build(d_nbr.as<int32_t>(), n, plan1, tsp_conv_plan_bytes(n), s), prefix + " plan");
    run_conv(conv1, h0, in1, n, d_nbr.as<int32_t>(), plan1, h1, sc1, s);

    // ---- channel -> spatial, norm2 (no affine) + SiLU, conv2 on the children, skip
    lib(tsp_c2s_gather(h1, TSP_F32, d_gidx.as<int32_t>(), mm, Cout, g, s), prefix + " gather");
    lib(tsp_layer_norm(g, TSP_F32, mm, Cout, nullptr, nullptr, 1e-6f, 1, h2, in2, s), prefix + " norm2");
    {
        DeviceBuffer ws(tsp_rulebook_workspace_bytes(mm));
        lib(tsp_rulebook_build(d_child.as<int32_t>(), mm, nbr2, ws.get(), ws.size(), d_status.as<int32_t>(), s),
            prefix + " child rulebook");
        hip_check(hipStreamSynchronize(s), "c2s child rulebook");
    }
    if (conv2.mfma) lib(tsp_conv_plan_build(nbr2, mm, plan2, tsp_conv_plan_bytes(mm), s), prefix + " plan");
    run_conv(conv2, h2, in2, mm, nbr2, plan2, out, sc2, s);
    lib(tsp_c2s_skip_add(d_x.get(), TSP_F32, d_gidx.as<int32_t>(), mm, Cin, Cout, out, TSP_F32, s),
        prefix + " skip");

    int32_t status = 0;
    hip_check(hipMemcpyAsync(&status, d_status.get(), 4, hipMemcpyDeviceToHost, s), "c2s");
    hip_check(hipStreamSynchronize(s), "c2s");
    if (status) fail(prefix + ": a coordinate lies outside [0, 2^21-3]");
    r.feats.resize((size_t)mm * Cout);
    r.coords.resize((size_t)mm);
    hip_check(hipMemcpy(r.feats.data(), out, r.feats.size() * 4, hipMemcpyDeviceToHost), "c2s readback");
    hip_check(hipMemcpy(r.coords.data(), d_child.get(), (size_t)mm * 12, hipMemcpyDeviceToHost), "c2s readback");
    return r;
}

}  // namespace trellis
