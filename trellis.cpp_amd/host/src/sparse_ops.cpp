// Device-level pieces of the sparse path on libtrellis_sparse (reference: src/sparse.cpp:61-336).
#include "sparse_ops.hpp"

#include <algorithm>
#include <cstring>
#include <mutex>
#include <stdexcept>
#include <unordered_map>

#include "sparse.h"

namespace trellis {
namespace ops {

using tgr::DeviceBuffer;
using tgr::fail;
using tgr::hip_check;

void lib(int st, const std::string& what) {
    if (st != TSP_OK) fail(what + ": " + tsp_last_error());
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

const float* f32_param(const ggml_tensor* t, Carve& sc, hipStream_t s) {
    if (t->type == GGML_TYPE_F32) return static_cast<const float*>(t->data);
    void* p = sc.take((size_t)ggml_nelements(t) * 4);
    if (sc.running())
        hip_check(tgr::launch_convert(t->data, tgr::tsp_dtype_of(t->type), p, TSP_F32, ggml_nelements(t), s),
                  "parameter conversion");
    return static_cast<const float*>(p);
}

// ---- packed weights ------------------------------------------------------------------------------
// The weights of a loaded Model (registered by Model::load, dropped by Model::free) are packed
// on first use and kept: a conv weight for the matrix-core kernel, a ConvNeXt block's mlp.0 and
// mlp.2 (keyed by mlp.0) for the one-kernel MLP. Decodes after the first pack nothing. Other
// weight tensors (a caller's own buffers, which may be freed and their memory reused) are not
// cached. In a sizing pass (where only null or not matters to the workspace sizes) a stand-in.
// A pack runs on the first caller's stream, which is synchronised before the copy is published,
// so that a caller on another stream never reads it unfinished.
namespace {
std::mutex g_packed_mu;
std::unordered_map<const void*, void*> g_packed;       // a model tensor's data -> its packed copy or null
std::unordered_map<const void*, void*> g_packed_mlp;   // a block's mlp.0 data -> its packed MLP

// The cached copy of `key` in `cache` (a registered model tensor), packed by pack(p, s) into
// `bytes` on first use; null when key is no model tensor. Called with g_packed_mu held.
template <class Pack>
const void* cached_pack(std::unordered_map<const void*, void*>& cache, const void* key, size_t bytes,
                        bool running, hipStream_t s, Pack pack) {
    if (g_packed.find(key) == g_packed.end()) return nullptr;
    if (!running) return reinterpret_cast<const void*>(uintptr_t(256));
    void*& slot = cache[key];
    if (!slot) {
        void* p = nullptr;
        hip_check(hipMalloc(&p, bytes), "packed weights");
        pack(p, s);
        hip_check(hipStreamSynchronize(s), "weight pack");
        slot = p;
    }
    return slot;
}
}  // namespace

void register_model_weights(const std::vector<const void*>& data) {
    std::lock_guard<std::mutex> lock(g_packed_mu);
    for (const void* d : data) g_packed.emplace(d, nullptr);
}

void forget_model_weights(const std::vector<const void*>& data) {
    std::lock_guard<std::mutex> lock(g_packed_mu);
    for (const void* d : data) {
        for (auto* cache : {&g_packed, &g_packed_mlp}) {
            auto it = cache->find(d);
            if (it == cache->end()) continue;
            if (it->second) (void)hipFree(it->second);
            cache->erase(it);
        }
    }
}

const void* packed_weights(const Conv& c, bool running, hipStream_t s) {
    if (!c.mfma) return nullptr;
    std::lock_guard<std::mutex> lock(g_packed_mu);
    return cached_pack(g_packed, c.w->data, tsp_conv_weight_packed_bytes(c.ci, c.co), running, s,
                       [&](void* p, hipStream_t st) {
                           lib(tsp_conv_weight_pack(c.w->data, c.wdt, c.ci, c.co, p, st), "weight pack");
                       });
}

const void* packed_mlp(const ConvNext& a, bool running, hipStream_t s) {
    const int dt = tgr::tsp_dtype_of(a.w0->type);
    // the shapes and types of the one-kernel MLP (tsp_convnext_mlp_pack)
    if (a.c != 128 || (dt != TSP_F16 && dt != TSP_BF16) || tgr::tsp_dtype_of(a.w2->type) != dt) return nullptr;
    std::lock_guard<std::mutex> lock(g_packed_mu);
    if (g_packed.find(a.w2->data) == g_packed.end()) return nullptr;
    return cached_pack(g_packed_mlp, a.w0->data, tsp_convnext_mlp_packed_bytes(a.c), running, s,
                       [&](void* p, hipStream_t st) {
                           lib(tsp_convnext_mlp_pack(a.w0->data, a.w2->data, dt, a.c, p, st), "MLP pack");
                       });
}

int act_dtype(int wdt, bool conv_weight) {
    if (wdt == TSP_F16) return conv_weight && g_sparse_cast_f32 ? TSP_F32 : TSP_F16;
    return wdt;
}

// ---- conv --------------------------------------------------------------------------------------
Conv conv_of(const Model& m, const std::string& prefix) {
    Conv c;
    c.w = m.get(prefix + ".weight");
    c.b = m.get(prefix + ".bias");
    if (c.w->ne[1] != 27 || c.w->ne[3] != 1) fail(prefix + ".weight: expected ggml shape [Ci, 27, Co]");
    c.ci = (int)c.w->ne[0];
    c.co = (int)c.w->ne[2];
    if (ggml_nelements(c.b) != c.co) fail(prefix + ".bias: expected " + std::to_string(c.co) + " elements");
    c.wdt = tgr::tsp_dtype_of(c.w->type);
    if (c.wdt < 0) fail(prefix + ".weight: unsupported tensor type");
    c.xdt = act_dtype(c.wdt, true);
    c.mfma = c.xdt != TSP_F32 && c.ci % 16 == 0 && c.co % 64 == 0;
    return c;
}

// F32 activations are rounded to c.xdt, as ggml's mul_mat rounds its F32 operand to the weights'
// type (sparse.cpp:74); the matrix-core kernel runs where the channel counts fit its tiles, the
// VALU kernel elsewhere (on the rounded input, or under g_sparse_cast_f32 on the F32 input and
// the weights' exact values). The padding row is formed from the unrounded row 0 (sparse.cpp:81-85
// pads the F32 input).
void run_conv(const Conv& c, const void* x, int xdt, int64_t n, const int32_t* nbr, const void* plan,
              float* out, Carve& sc, hipStream_t s) {
    const float* bias = f32_param(c.b, sc, s);
    const float* row0 = xdt == TSP_F32 && c.xdt != TSP_F32 ? static_cast<const float*>(x) : nullptr;
    const void* xr = x;
    if (xdt != c.xdt) {
        if (xdt != TSP_F32) fail("sparse conv: 16-bit input of another type than the weights'");
        void* p = sc.take((size_t)n * c.ci * 2);
        if (sc.running()) hip_check(tgr::launch_convert(x, xdt, p, c.xdt, n * c.ci, s), "conv input rounding");
        xr = p;
    }
    if (c.mfma) {
        const void* packed = packed_weights(c, sc.running(), s);
        void* own = packed ? nullptr : sc.take(tsp_conv_weight_packed_bytes(c.ci, c.co));
        if (!sc.running()) return;
        if (!plan) fail("sparse conv: the matrix-core path needs a conv plan");
        if (own) {
            lib(tsp_conv_weight_pack(c.w->data, c.wdt, c.ci, c.co, own, s), "weight pack");
            packed = own;
        }
        lib(tsp_subm_conv3x3_planned_ex(xr, c.xdt, n, c.ci, nbr, plan, packed, bias, c.co, out, TSP_F32, 0, row0, s),
            "sparse conv");
    } else {
        if (!sc.running()) return;
        lib(tsp_subm_conv3x3_ex(xr, c.xdt, n, c.ci, nbr, c.w->data, c.wdt, bias, c.co, out, TSP_F32, TSP_ALGO_AUTO,
                                0, row0, s),
            "sparse conv");
    }
}

size_t conv_scratch(const Conv& c, int64_t n, int xdt) {
    Carve sz;
    run_conv(c, nullptr, xdt, n, nullptr, nullptr, nullptr, sz, nullptr);
    return sz.off;
}

// ---- ConvNeXt block (sparse.cpp:94-137) --------------------------------------------------------
ConvNext convnext_of(const Model& m, const std::string& prefix, int64_t n) {
    ConvNext a;
    a.conv = conv_of(m, prefix + ".conv");
    const int c = a.conv.co;
    if (a.conv.ci != c) fail(prefix + ".conv: a ConvNeXt conv keeps the channel count");
    a.nw = vec_param(m, prefix + ".norm.weight", c);
    a.nb = vec_param(m, prefix + ".norm.bias", c);
    a.w0 = mat_param(m, prefix + ".mlp.0.weight", c, 4 * (int64_t)c);
    a.b0 = vec_param(m, prefix + ".mlp.0.bias", 4 * (int64_t)c);
    a.w2 = mat_param(m, prefix + ".mlp.2.weight", 4 * (int64_t)c, c);
    a.b2 = vec_param(m, prefix + ".mlp.2.bias", c);
    a.n = n;
    a.c = c;
    return a;
}

// The block is one tsp_convnext call; 16-bit vectors are converted to f32 in the scratch first.
void run_convnext(const ConvNext& a, const void* x, int xdt, const int32_t* nbr, const void* plan,
                  float* out, Carve& sc, hipStream_t s, const void* x16, void* out16, int out16_dtype) {
    tsp_convnext_weights w{};
    w.conv_weight = a.conv.w->data;
    w.conv_dtype = a.conv.wdt;
    w.conv_bias = f32_param(a.conv.b, sc, s);
    w.conv_packed = packed_weights(a.conv, sc.running(), s);
    w.norm_weight = f32_param(a.nw, sc, s);
    w.norm_bias = f32_param(a.nb, sc, s);
    w.mlp0_weight = a.w0->data;
    w.mlp0_dtype = tgr::tsp_dtype_of(a.w0->type);
    w.mlp0_bias = f32_param(a.b0, sc, s);
    w.mlp2_weight = a.w2->data;
    w.mlp2_dtype = tgr::tsp_dtype_of(a.w2->type);
    w.mlp2_bias = f32_param(a.b2, sc, s);
    w.mlp_packed = packed_mlp(a, sc.running(), s);
    const int flags = g_sparse_cast_f32 ? TSP_BLOCK_CAST_F32 : 0;
    // a plan comes with every matrix-core conv (the callers build it where conv.mfma)
    const size_t nb = tsp_convnext_workspace_bytes(a.n, a.c, xdt, &w, a.conv.mfma, flags);
    void* ws = sc.take(nb);
    if (!sc.running()) return;
    if (a.conv.mfma && !plan) fail("sparse_convnext: the matrix-core path needs a conv plan");
    lib(tsp_convnext_ex(x, xdt, x16, a.n, a.c, nbr, a.conv.mfma ? plan : nullptr, &w, out, out16, out16_dtype, ws, nb,
                        flags, s),
        "sparse_convnext");
}

size_t convnext_scratch(const ConvNext& a, int xdt) {
    Carve sz;
    run_convnext(a, nullptr, xdt, nullptr, nullptr, nullptr, sz, nullptr);
    return sz.off;
}

// ---- tables --------------------------------------------------------------------------------------
void build_table(const int32_t* d_coords, int64_t n, Table& t, hipStream_t s, int32_t* d_status,
                 bool morton_plan) {
    t.n = n;
    t.coords = morton_plan ? d_coords : nullptr;
    t.plan = DeviceBuffer();
    t.nbr = DeviceBuffer((size_t)27 * n * 4, s);
    if (n == 0) return;
    DeviceBuffer ws(tsp_rulebook_workspace_bytes(n), s), status(d_status ? 0 : 4, s);
    if (!d_status) hip_check(hipMemsetAsync(status.get(), 0, 4, s), "rulebook");
    if (morton_plan) {
        // the table and its Morton-ordered plan from one cell grid
        const size_t bytes = tsp_conv_plan_bytes(n);
        t.plan = DeviceBuffer(bytes, s);
        lib(tsp_rulebook_build_planned(d_coords, n, t.nbr.as<int32_t>(), ws.get(), ws.size(),
                                       d_status ? d_status : status.as<int32_t>(), t.plan.get(), bytes, s),
            "rulebook");
    } else {
        lib(tsp_rulebook_build(d_coords, n, t.nbr.as<int32_t>(), ws.get(), ws.size(),
                               d_status ? d_status : status.as<int32_t>(), s),
            "rulebook");
    }
    if (d_status) return;
    int32_t st = 0;
    hip_check(hipMemcpyAsync(&st, status.get(), 4, hipMemcpyDeviceToHost, s), "rulebook");
    hip_check(hipStreamSynchronize(s), "rulebook");
    if (st) fail("neighbour table: a coordinate lies outside [0, 2^21-3]");
}

void Table::ensure_plan(hipStream_t s) {
    if (plan.get() || n == 0) return;
    const size_t bytes = tsp_conv_plan_bytes(n);
    plan = DeviceBuffer(bytes, s);
    if (coords)
        lib(tsp_conv_plan_build_ordered(nbr.as<int32_t>(), coords, n, plan.get(), bytes, s), "conv plan");
    else
        lib(tsp_conv_plan_build(nbr.as<int32_t>(), n, plan.get(), bytes, s), "conv plan");
}

// ---- C2S up-block (sparse.cpp:172-336) -----------------------------------------------------------
int64_t count_nonzero(const uint8_t* p, size_t n) {
    // eight bytes at a time: a byte's high bit is set in z exactly when the byte is zero
    constexpr uint64_t kLow7 = 0x7f7f7f7f7f7f7f7full;
    int64_t zeros = 0;
    size_t i = 0;
    for (; i + 8 <= n; i += 8) {
        uint64_t w;
        memcpy(&w, p + i, 8);
        const uint64_t z = ~(((w & kLow7) + kLow7) | w | kLow7);
        zeros += __builtin_popcountll(z);
    }
    for (; i < n; ++i) zeros += p[i] == 0;
    return (int64_t)n - zeros;
}

C2SOut run_c2s(const Model& m, const std::string& prefix, const float* d_x, const int32_t* d_coords,
               Table& parent, int cin, int cout, const std::vector<uint8_t>* ext_mask, hipStream_t s,
               int32_t* d_status, bool want_mask, int64_t ext_count, int out16_dtype, bool defer_conv2) {
    const int64_t n = parent.n;
    if (cin <= 0 || cin % 8 != 0 || cout <= 0 || cout % (cin / 8) != 0)
        fail(prefix + ": C2S needs Cin % 8 == 0 and Cout % (Cin/8) == 0");
    if (ext_mask && (int64_t)ext_mask->size() != 8 * n) fail(prefix + ": ext_subdiv must hold 8*N entries");
    C2SOut r;
    if (want_mask) r.mask.resize((size_t)8 * n);
    if (n == 0) return r;
    const Conv conv1 = conv_of(m, prefix + ".conv1"), conv2 = conv_of(m, prefix + ".conv2");
    if (conv1.ci != cin || conv1.co != 8 * cout || conv2.ci != cout || conv2.co != cout)
        fail(prefix + ": conv1 must map Cin -> 8*Cout and conv2 Cout -> Cout");
    const ggml_tensor* n1w = vec_param(m, prefix + ".norm1.weight", cin);
    const ggml_tensor* n1b = vec_param(m, prefix + ".norm1.bias", cin);

    // subdivision mask: the caller's, or to_subdiv logits > 0 (sparse.cpp:184-199, 215)
    // temporaries are stream-ordered on s: freed in queue order, no wait at the end
    DeviceBuffer d_mask((size_t)8 * n, s);
    if (ext_mask) {
        hip_check(hipMemcpyAsync(d_mask.get(), ext_mask->data(), (size_t)8 * n, hipMemcpyHostToDevice, s),
                  "c2s mask upload");
    } else {
        const ggml_tensor* wsub = mat_param(m, prefix + ".to_subdiv.weight", cin, 8);
        const ggml_tensor* bsub = vec_param(m, prefix + ".to_subdiv.bias", 8);
        const int wsdt = tgr::tsp_dtype_of(wsub->type), xsdt = act_dtype(wsdt, false);
        DeviceBuffer d_logits((size_t)8 * n * 4, s), d_b(256, s);
        DeviceBuffer d_xs(xsdt != TSP_F32 ? (size_t)n * cin * 2 : 0, s);
        Carve sc(d_b.get());
        if (xsdt != TSP_F32)
            hip_check(tgr::launch_convert(d_x, TSP_F32, d_xs.get(), xsdt, n * cin, s), "to_subdiv rounding");
        lib(tsp_linear(xsdt != TSP_F32 ? d_xs.get() : static_cast<const void*>(d_x), xsdt, n, cin, wsub->data,
                       wsdt, f32_param(bsub, sc, s), 8, d_logits.get(), TSP_F32, s),
            prefix + ".to_subdiv");
        lib(tsp_mask_positive(d_logits.as<float>(), 8 * n, d_mask.as<uint8_t>(), s), prefix + " mask");
    }

    // children, parent-major and octant-ascending (sparse.cpp:205-222)
    DeviceBuffer d_mstart((size_t)(n + 1) * 4, s), d_child((size_t)8 * n * 12, s), d_gidx((size_t)8 * n * 4, s),
        d_m(8, s), d_sws(tsp_subdivide_workspace_bytes(n), s);
    lib(tsp_subdivide(d_mask.as<uint8_t>(), d_coords, n, d_mstart.as<int32_t>(), d_child.as<int32_t>(),
                      d_gidx.as<int32_t>(), d_m.as<int64_t>(), d_sws.get(), d_sws.size(), s),
        prefix + " subdivide");
    int64_t mm = 0;
    if (ext_mask) {
        // the child count is the caller's mask's: no need to wait for the device
        mm = ext_count >= 0 ? ext_count : count_nonzero(ext_mask->data(), ext_mask->size());
        if (want_mask) std::copy(ext_mask->begin(), ext_mask->end(), r.mask.begin());
    } else {
        hip_check(hipMemcpyAsync(&mm, d_m.get(), 8, hipMemcpyDeviceToHost, s), "c2s");
        if (want_mask)
            hip_check(hipMemcpyAsync(r.mask.data(), d_mask.get(), (size_t)8 * n, hipMemcpyDeviceToHost, s),
                      "c2s mask");
        hip_check(hipStreamSynchronize(s), "c2s");
    }
    r.m = mm;
    r.coords = DeviceBuffer((size_t)mm * 12, s);
    r.feats = DeviceBuffer((size_t)mm * cout * 4, s);
    if (out16_dtype >= 0) r.feats16 = DeviceBuffer((size_t)mm * cout * 2, s);
    if (mm == 0) return r;
    hip_check(hipMemcpyAsync(r.coords.get(), d_child.get(), (size_t)mm * 12, hipMemcpyDeviceToDevice, s),
              "c2s");

    // the children's table (and plans where a conv runs on the matrix cores), then the block's
    // features in one tsp_c2s call: norm1 + SiLU, conv1 with the octant gather, norm2 + SiLU,
    // conv2 (its absent taps read hn's zero padding column, sparse.cpp:289-306) with the skip
    // (a deferred conv2 takes tiles of consecutive rows: ranges of rows are then ranges of tiles)
    build_table(r.coords.as<int32_t>(), mm, r.table, s, d_status, /*morton_plan=*/!defer_conv2);   // r.coords outlives it
    if (conv1.mfma) parent.ensure_plan(s);
    if (conv2.mfma) r.table.ensure_plan(s);
    const ggml_tensor* c1b = conv1.b;
    const ggml_tensor* c2b = conv2.b;
    DeviceBuffer pbuf((size_t)(2 * cin + 9 * cout) * 4 + 4 * 256, s);
    Carve scp(pbuf.get());
    tsp_c2s_weights w{};
    w.norm1_weight = f32_param(n1w, scp, s);
    w.norm1_bias = f32_param(n1b, scp, s);
    w.conv1_weight = conv1.w->data;
    w.conv1_dtype = conv1.wdt;
    w.conv1_bias = f32_param(c1b, scp, s);
    w.conv2_weight = conv2.w->data;
    w.conv2_dtype = conv2.wdt;
    w.conv2_bias = f32_param(c2b, scp, s);
    w.conv1_packed = packed_weights(conv1, true, s);
    w.conv2_packed = packed_weights(conv2, true, s);
    const int flags = g_sparse_cast_f32 ? TSP_BLOCK_CAST_F32 : 0;
    const size_t nb = tsp_c2s_workspace_bytes(n, mm, cin, cout, &w, conv1.mfma, conv2.mfma, flags);
    DeviceBuffer work(nb, s);
    // the buffers a deferred conv2 still reads (stream-ordered: released after its last call)
    struct Kept {
        DeviceBuffer mask, mstart, gidx, params, work;
        tsp_c2s_weights w;
        bool whole = false;   // conv2 ran over every tile (its ranges are then done)
    };
    auto kept = std::make_shared<Kept>();
    // (device pointers: the tables' and the outputs' buffers keep their addresses when moved)
    const int32_t* pnbr = parent.nbr.as<int32_t>();
    const void* pplan = conv1.mfma ? parent.plan.get() : nullptr;
    const int32_t* cnbr = r.table.nbr.as<int32_t>();
    const void* cplan = conv2.mfma ? r.table.plan.get() : nullptr;
    float* feats = r.feats.as<float>();
    void* feats16 = out16_dtype >= 0 ? r.feats16.get() : nullptr;
    const int o16 = out16_dtype >= 0 ? out16_dtype : TSP_BF16;
    auto part = [=](int p, int64_t t0, int64_t nt) {
        return tsp_c2s_part(d_x, n, cin, pnbr, pplan, kept->mask.as<uint8_t>(), kept->mstart.as<int32_t>(),
                            kept->gidx.as<int32_t>(), mm, cout, cnbr, cplan, &kept->w, feats, feats16, o16,
                            kept->work.get(), nb, flags, p, t0, nt, s);
    };
    kept->mask = std::move(d_mask);
    kept->mstart = std::move(d_mstart);
    kept->gidx = std::move(d_gidx);
    kept->params = std::move(pbuf);
    kept->work = std::move(work);
    kept->w = w;
    if (!defer_conv2) {
        lib(part(TSP_C2S_PART_FRONT | TSP_C2S_PART_CONV2, 0, -1), prefix);
        return r;
    }
    lib(part(TSP_C2S_PART_FRONT, 0, -1), prefix);
    r.conv2_rows = [kept, part, prefix, mm](int64_t r0, int64_t r1) {
        if (kept->whole) return;
        const int64_t t0 = r0 / 512, t1 = std::min((r1 + 511) / 512, (mm + 511) / 512);
        const int st = part(TSP_C2S_PART_CONV2, t0, t1 - t0);
        if (st != TSP_ERR_UNSUPPORTED) {
            lib(st, prefix + " conv2");
            return;
        }
        // conv2 that does not run by tiles (no matrix-core conv2 with the skip in its stores): all
        // rows at once
        lib(part(TSP_C2S_PART_CONV2, 0, -1), prefix + " conv2");
        kept->whole = true;
    };
    return r;
}

// ---- per-voxel linear (shape_decoder.cpp:63-77) --------------------------------------------------
void run_linear(const Model& m, const std::string& prefix, const float* d_x, int64_t n, int ci, int co,
                bool pre_norm, float eps, float* d_out, hipStream_t s) {
    const ggml_tensor* w = mat_param(m, prefix + ".weight", ci, co);
    const ggml_tensor* b = vec_param(m, prefix + ".bias", co);
    const int wdt = tgr::tsp_dtype_of(w->type);
    const int xdt = act_dtype(wdt, false);
    DeviceBuffer pb((size_t)co * 4 + 256, s);
    Carve sc(pb.get());
    const float* bias = f32_param(b, sc, s);
    // a narrow head after a LayerNorm runs as one pass over x (shapes it does not take fall back);
    // it rounds the normalised values to xdt as the LN's output would be
    if (pre_norm && co <= 8) {
        const hipError_t e = tgr::launch_norm_linear(d_x, n, ci, eps, w->data, wdt, bias, co, d_out, s);
        if (e != hipErrorInvalidValue) {
            hip_check(e, (prefix + " head").c_str());
            return;
        }
    }
    DeviceBuffer tmp((pre_norm || xdt != TSP_F32) ? (size_t)n * ci * (xdt != TSP_F32 ? 2 : 4) : 0, s);
    const void* x = d_x;
    if (pre_norm) {
        lib(tsp_layer_norm(d_x, TSP_F32, n, ci, nullptr, nullptr, eps, 0, tmp.get(), xdt, s), prefix + " norm");
        x = tmp.get();
    } else if (xdt != TSP_F32) {
        hip_check(tgr::launch_convert(d_x, TSP_F32, tmp.get(), xdt, n * ci, s), (prefix + " rounding").c_str());
        x = tmp.get();
    }
    lib(tsp_linear(x, xdt, n, ci, w->data, wdt, bias, co, d_out, TSP_F32, s), prefix);
}

}  // namespace ops
}  // namespace trellis
