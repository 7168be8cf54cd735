// Device-level pieces of the sparse path on libtrellis_sparse (reference: src/sparse.cpp:61-336).
#include "sparse_ops.hpp"

#include <algorithm>
#include <cstring>
#include <stdexcept>

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
// pads the F32 input). A caller that passes input already in c.xdt (rounded from F32 as it was
// written) leaves the padding row to that row 0: the two differ only where a finite F32 value
// overflows the 16-bit range.
void run_conv(const Conv& c, const void* x, int xdt, int64_t n, const int32_t* nbr, const void* plan,
              float* out, Carve& sc, hipStream_t s, const ConvStores& st) {
    const float* bias = f32_param(c.b, sc, s);
    const int flags = st.zero_pad ? TSP_CONV_ZERO_PAD : 0;
    const float* row0 = xdt == TSP_F32 && c.xdt != TSP_F32 ? static_cast<const float*>(x) : nullptr;
    const void* xr = x;
    if (xdt != c.xdt) {
        if (xdt != TSP_F32) fail("sparse conv: 16-bit input of another type than the weights'");
        void* p = sc.take((size_t)n * c.ci * 2);
        if (sc.running()) hip_check(tgr::launch_convert(x, xdt, p, c.xdt, n * c.ci, s), "conv input rounding");
        xr = p;
    }
    if (c.mfma) {
        const void* x16 = xr;
        void* packed = sc.take((size_t)27 * c.ci * c.co * 2);
        if (!sc.running()) return;
        if (!plan) fail("sparse conv: the matrix-core path needs a conv plan");
        lib(tsp_conv_weight_pack(c.w->data, c.wdt, c.ci, c.co, packed, s), "weight pack");
        if (st.ocout)
            lib(tsp_subm_conv3x3_planned_octants(x16, c.wdt, n, c.ci, nbr, plan, packed, bias, st.ocout,
                                                 st.omask, st.omstart, out, s),
                "sparse conv (octant stores)");
        else if (st.skip_cin)   // always an exact zero padding row: the C2S conv2
            lib(tsp_subm_conv3x3_planned_skip(x16, c.wdt, n, c.ci, nbr, plan, packed, bias, c.co, st.skip_x,
                                              st.skip_cin, st.skip_gidx, out, s),
                "sparse conv (skip stores)");
        else
            lib(tsp_subm_conv3x3_planned_ex(x16, c.wdt, n, c.ci, nbr, plan, packed, bias, c.co, out, TSP_F32,
                                            flags, row0, s),
                "sparse conv");
    } else {
        if (st.ocout || st.skip_cin) fail("sparse conv: fused stores need the matrix-core path");
        if (!sc.running()) return;
        lib(tsp_subm_conv3x3_ex(xr, c.xdt, n, c.ci, nbr, c.w->data, c.wdt, bias, c.co, out, TSP_F32,
                                TSP_ALGO_NARROW, flags, row0, s),
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
    // the [chunk, 4C] f32 hidden is bounded to 1 GiB
    a.chunk = std::max<int64_t>(1, std::min<int64_t>(n, (int64_t(1) << 30) / (16 * (int64_t)c)));
    a.adt0 = act_dtype(tgr::tsp_dtype_of(a.w0->type), false);
    a.adt2 = act_dtype(tgr::tsp_dtype_of(a.w2->type), false);
    return a;
}

void run_convnext(const ConvNext& a, const void* x, int xdt, const int32_t* nbr, const void* plan,
                  float* out, Carve& sc, hipStream_t s) {
    const int c = a.c;
    const int w0dt = tgr::tsp_dtype_of(a.w0->type), w2dt = tgr::tsp_dtype_of(a.w2->type);
    // each linear's input rounded to its act_dtype (LN + affine output -> adt0, SiLU output -> adt2)
    const int adt0 = a.adt0, adt2 = a.adt2;
    const size_t aes = adt0 == TSP_F32 ? 4 : 2;
    float* h = static_cast<float*>(sc.take((size_t)a.n * c * 4));
    void* hn = adt0 != TSP_F32 ? sc.take((size_t)a.n * c * 2) : h;
    float* hid = static_cast<float*>(sc.take((size_t)a.chunk * 4 * c * 4));
    void* hid_in = adt2 != TSP_F32 ? sc.take((size_t)a.chunk * 4 * c * 2) : hid;
    const float* gamma = f32_param(a.nw, sc, s);
    const float* beta = f32_param(a.nb, sc, s);
    const float* bias0 = f32_param(a.b0, sc, s);
    const float* bias2 = f32_param(a.b2, sc, s);
    run_conv(a.conv, x, xdt, a.n, nbr, plan, h, sc, s);
    if (!sc.running()) return;
    lib(tsp_layer_norm(h, TSP_F32, a.n, c, gamma, beta, 1e-6f, 0, hn, adt0, s), "convnext norm");
    const size_t xes = xdt == TSP_F32 ? 4 : 2;
    for (int64_t r0 = 0; r0 < a.n; r0 += a.chunk) {
        const int64_t nr = std::min(a.chunk, a.n - r0);
        const void* hin = static_cast<const char*>(hn) + (size_t)r0 * c * aes;
        const void* xr = static_cast<const char*>(x) + (size_t)r0 * c * xes;
        float* yr = out + r0 * c;
        // 16-bit MLP: mlp.0 with its bias and SiLU, and mlp.2 with its bias and the f32 block input,
        // each one library GEMM; the unfused sequence where a shape has no such GEMM
        int st = TSP_ERR_UNSUPPORTED;
        if (adt0 != TSP_F32 && adt2 != TSP_F32)
            st = tsp_linear_ex(hin, adt0, nr, c, a.w0->data, w0dt, bias0, 4 * c, TSP_ACT_SILU, nullptr,
                               hid_in, adt2, s);
        if (st != TSP_ERR_UNSUPPORTED) {
            lib(st, "convnext mlp.0");
        } else {
            lib(tsp_linear(hin, adt0, nr, c, a.w0->data, w0dt, bias0, 4 * c, hid, TSP_F32, s), "convnext mlp.0");
            hip_check(tgr::launch_silu_to(hid, hid_in, adt2, nr * 4 * c, s), "convnext silu");
        }
        st = TSP_ERR_UNSUPPORTED;
        if (adt2 != TSP_F32 && xdt == TSP_F32)
            st = tsp_linear_ex(hid_in, adt2, nr, 4 * c, a.w2->data, w2dt, bias2, c, TSP_ACT_NONE,
                               static_cast<const float*>(xr), yr, TSP_F32, s);
        if (st != TSP_ERR_UNSUPPORTED) {
            lib(st, "convnext mlp.2");
        } else {
            lib(tsp_linear(hid_in, adt2, nr, 4 * c, a.w2->data, w2dt, bias2, c, yr, TSP_F32, s), "convnext mlp.2");
            hip_check(tgr::launch_add_inplace(yr, xr, xdt, nr * c, s), "convnext residual");
        }
    }
}

size_t convnext_scratch(const ConvNext& a, int xdt) {
    Carve sz;
    run_convnext(a, nullptr, xdt, nullptr, nullptr, nullptr, sz, nullptr);
    return sz.off;
}

// ---- tables --------------------------------------------------------------------------------------
void build_table(const int32_t* d_coords, int64_t n, Table& t, hipStream_t s, int32_t* d_status) {
    t.n = n;
    t.coords = nullptr;
    t.plan = DeviceBuffer();
    t.nbr = DeviceBuffer((size_t)27 * n * 4, s);
    if (n == 0) return;
    DeviceBuffer ws(tsp_rulebook_workspace_bytes(n), s), status(d_status ? 0 : 4, s);
    if (!d_status) hip_check(hipMemsetAsync(status.get(), 0, 4, s), "rulebook");
    lib(tsp_rulebook_build(d_coords, n, t.nbr.as<int32_t>(), ws.get(), ws.size(),
                           d_status ? d_status : status.as<int32_t>(), s),
        "rulebook");
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
               int32_t* d_status, bool want_mask, int64_t ext_count) {
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
    if (mm == 0) return r;
    hip_check(hipMemcpyAsync(r.coords.get(), d_child.get(), (size_t)mm * 12, hipMemcpyDeviceToDevice, s),
              "c2s");

    // conv1 on the parents: LN(norm1)+SiLU written straight in the conv's input dtype. On the
    // matrix cores (cout % 64 == 0) its stores do the octant gather, and the [n][8 cout]
    // intermediate is never written.
    // norm1 / norm2 (+ SiLU) write the convs' inputs rounded as the convs take them
    const int in1 = conv1.xdt, in2 = conv2.xdt;
    const size_t es1 = in1 == TSP_F32 ? 4 : 2, es2 = in2 == TSP_F32 ? 4 : 2;
    const size_t s1 = conv_scratch(conv1, n, in1), s2 = conv_scratch(conv2, mm, in2);
    const bool octant_stores = conv1.mfma && cout % 64 == 0;
    Carve sz;
    sz.take((size_t)n * cin * es1);
    sz.take(octant_stores ? 0 : (size_t)n * 8 * cout * 4);
    sz.take(s1);
    sz.take((size_t)mm * cout * 4);
    sz.take((size_t)mm * cout * es2);
    sz.take(s2);
    sz.take(2 * (size_t)cin * 4);
    DeviceBuffer work(sz.off, s);
    Carve w(work.get());
    void* h0 = w.take((size_t)n * cin * es1);
    float* h1 = static_cast<float*>(w.take(octant_stores ? 0 : (size_t)n * 8 * cout * 4));
    Carve sc1(w.take(s1));
    float* g = static_cast<float*>(w.take((size_t)mm * cout * 4));
    void* h2 = w.take((size_t)mm * cout * es2);
    Carve sc2(w.take(s2));
    Carve scp(w.take(2 * (size_t)cin * 4));
    const float* g1 = f32_param(n1w, scp, s);
    const float* b1 = f32_param(n1b, scp, s);

    lib(tsp_layer_norm(d_x, TSP_F32, n, cin, g1, b1, 1e-6f, 1, h0, in1, s), prefix + ".norm1");
    if (conv1.mfma) parent.ensure_plan(s);
    if (octant_stores) {
        ConvStores st;
        st.omask = d_mask.as<uint8_t>();
        st.omstart = d_mstart.as<int32_t>();
        st.ocout = cout;
        run_conv(conv1, h0, in1, n, parent.nbr.as<int32_t>(), parent.plan.get(), g, sc1, s, st);
    } else {
        run_conv(conv1, h0, in1, n, parent.nbr.as<int32_t>(), parent.plan.get(), h1, sc1, s);
        // channel -> spatial gather
        lib(tsp_c2s_gather(h1, TSP_F32, d_gidx.as<int32_t>(), mm, cout, g, s), prefix + " gather");
    }

    // norm2 (no affine) + SiLU, conv2 on the children, skip
    lib(tsp_layer_norm(g, TSP_F32, mm, cout, nullptr, nullptr, 1e-6f, 1, h2, in2, s), prefix + " norm2");
    build_table(r.coords.as<int32_t>(), mm, r.table, s, d_status);
    if (conv2.mfma) r.table.ensure_plan(s);
    // the skip: added by conv2's stores on the matrix cores (repeat R % 4 == 0), else its own pass
    // conv2's absent taps read hn's zero padding column (sparse.cpp:289-306)
    if (conv2.mfma && (cout / (cin / 8)) % 4 == 0) {
        ConvStores st;
        st.skip_x = d_x;
        st.skip_gidx = d_gidx.as<int32_t>();
        st.skip_cin = cin;
        st.zero_pad = true;
        run_conv(conv2, h2, in2, mm, r.table.nbr.as<int32_t>(), r.table.plan.get(), r.feats.as<float>(), sc2, s,
                 st);
    } else {
        ConvStores st;
        st.zero_pad = true;
        run_conv(conv2, h2, in2, mm, r.table.nbr.as<int32_t>(), r.table.plan.get(), r.feats.as<float>(), sc2, s,
                 st);
        lib(tsp_c2s_skip_add(d_x, TSP_F32, d_gidx.as<int32_t>(), mm, cin, cout, r.feats.get(), TSP_F32, s),
            prefix + " skip");
    }
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
