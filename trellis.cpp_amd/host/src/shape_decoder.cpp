// The sparse U-Net VAE decoders (reference: src/shape_decoder.cpp:79-138) with every stage
// resident on the device: features, coordinates, neighbour tables and conv plans never leave
// HBM between stages; only the subdivision masks (which the texture decoder needs) and the
// final result are read back.
//
// The network is read off the model instead of a fixed table: stage s holds ConvNeXt blocks
// `blocks.s.j` (those with a `.conv.weight`) followed by one C2S block (the first `blocks.s.j`
// with a `.conv1.weight`); the channel counts come from the weight shapes. For the TRELLIS.2
// decoders this is 4 stages of {4, 16, 8, 4} blocks at 1024 -> 512 -> 256 -> 128 -> 64 channels
// (shape_decoder.cpp:88-90).
#include "shape_decoder.h"

#include <cstdio>
#include <cstdlib>
#include <functional>
#include <future>
#include <string>

#include "ggml.h"
#include "npy_io.hpp"
#include "runtime.hpp"
#include "sparse_ops.hpp"
#include "trellis_model.h"

namespace trellis {
namespace {

using tgr::DeviceBuffer;
using tgr::fail;
using tgr::hip_check;

struct Stage {
    std::vector<std::string> convnext;   // block prefixes
    std::string c2s;
    int cin = 0, cout = 0;
};

std::vector<Stage> stages_of(const Model& m) {
    std::vector<Stage> st;
    for (int s = 0;; ++s) {
        Stage g;
        for (int j = 0;; ++j) {
            const std::string p = "blocks." + std::to_string(s) + "." + std::to_string(j);
            if (m.has(p + ".conv.weight")) {
                g.convnext.push_back(p);
            } else if (m.has(p + ".conv1.weight")) {
                g.c2s = p;
                const ggml_tensor* w1 = m.get(p + ".conv1.weight");
                const ggml_tensor* w2 = m.get(p + ".conv2.weight");
                g.cin = (int)w1->ne[0];
                g.cout = (int)w2->ne[2];
                break;
            } else {
                break;
            }
        }
        if (g.c2s.empty()) {
            if (!g.convnext.empty()) fail("decoder: stage " + std::to_string(s) + " has no C2S block");
            break;
        }
        st.push_back(std::move(g));
    }
    if (st.empty()) fail("decoder: the model has no blocks.<stage>.<block> weights");
    return st;
}

// Debug output for checking a decode at sizes the checker cannot run whole: with
// TRELLIS_DECODER_DUMP=<dir>, each level's voxel coordinates go to <dir>/level<s>_coords.npy
// (int32 [N_s, 3]) and the last stage's input features to <dir>/level<S-1>_in.npy (f32
// [N, C]). The copies synchronise the stream; without the variable nothing is read back.
void dump_level(const char* dir, int level, const DeviceBuffer& dc, int64_t n, const DeviceBuffer* h, int c,
                hipStream_t s) {
    hip_check(hipStreamSynchronize(s), "decoder dump");
    std::vector<int32_t> co((size_t)n * 3);
    if (n) hip_check(hipMemcpy(co.data(), dc.get(), (size_t)n * 12, hipMemcpyDeviceToHost), "decoder dump");
    const std::string base = std::string(dir) + "/level" + std::to_string(level);
    npyio::save(base + "_coords.npy", "<i4", {n, 3}, co.data(), co.size() * 4);
    if (h) {
        std::vector<float> f((size_t)n * c);
        if (n) hip_check(hipMemcpy(f.data(), h->get(), f.size() * 4, hipMemcpyDeviceToHost), "decoder dump");
        npyio::save(base + "_in.npy", "<f4", {n, (int64_t)c}, f.data(), f.size() * 4);
    }
}

// One decoder pass; coords is updated to the final voxel set.
std::vector<float> decode(const Model& m, const std::vector<float>& latent, int out_ch,
                          std::vector<std::array<int, 3>>& coords,
                          const std::vector<std::vector<uint8_t>>* guide,
                          std::vector<std::vector<uint8_t>>* subs_out, bool coords_only,
                          bool want_coords = true) {
    const std::vector<Stage> stages = stages_of(m);
    if (guide && guide->size() < stages.size()) fail("tex_decode: one subdivision mask per stage is needed");
    int64_t n = (int64_t)coords.size();
    const ggml_tensor* wl = m.get("from_latent.weight");
    const int in_ch = (int)wl->ne[0], c0 = (int)wl->ne[1];
    if ((int64_t)latent.size() != n * in_ch) fail("decoder: latent must hold " + std::to_string(in_ch) + "*N floats");
    hip_check(hipSetDevice(tgr::backend_device(m.backend)), "hipSetDevice");
    hipStream_t s = tgr::backend_stream(m.backend);

    // every device buffer below is stream-ordered on s: nothing waits for the GPU until the end
    DeviceBuffer dc((size_t)n * 12, s), dl((size_t)n * in_ch * 4, s);
    hip_check(hipMemcpyAsync(dc.get(), coords.data(), (size_t)n * 12, hipMemcpyHostToDevice, s), "decoder upload");
    hip_check(hipMemcpyAsync(dl.get(), latent.data(), latent.size() * 4, hipMemcpyHostToDevice, s),
              "decoder upload");
    DeviceBuffer h((size_t)n * c0 * 4, s);
    ops::run_linear(m, "from_latent", dl.as<float>(), n, in_ch, c0, false, 0.f, h.as<float>(), s);
    dl.reset();
    int c = c0;
    ops::Table table;
    // coordinate range checks of every table of the pass, read once at the end
    DeviceBuffer status(4, s);
    hip_check(hipMemsetAsync(status.get(), 0, 4, s), "decoder");
    // Morton-ordered plans: dc holds each level's coordinates until that level's plans are built
    ops::build_table(dc.as<int32_t>(), n, table, s, status.as<int32_t>(), /*morton_plan=*/true);
    DeviceBuffer scratch, h2;
    // h rounded to h16dt, the input type of the next ConvNeXt conv (-1: none): written by the
    // stores of the block or C2S that produced h, so that conv needs no rounding pass of its own
    DeviceBuffer h16, h16b;
    int h16dt = -1;
    auto conv_input16 = [&](const std::string& block) {
        const ops::Conv nc = ops::conv_of(m, block + ".conv");
        return nc.xdt != TSP_F32 ? nc.xdt : -1;
    };
    // The result's host memory is touched on threads of their own while the device works: from
    // the start when the masks fix the final voxel count, else once the last subdivision is known.
    tgr::HostVector<float> result;
    tgr::HostVector<std::array<int, 3>> result_coords;
    bool result_started = false;
    auto start_result = [&](int64_t m_final) {
        if (!coords_only) result.start((size_t)m_final * out_ch);
        if (want_coords) result_coords.start((size_t)m_final);
        result_started = true;
    };
    // with masks, every stage's child count is counted on a thread of its own, off the path that
    // keeps the device fed
    std::future<std::vector<int64_t>> guide_counts;
    std::vector<int64_t> counts;
    if (guide)
        guide_counts = std::async(std::launch::async, [guide, ns = stages.size()] {
            std::vector<int64_t> c(ns);
            for (size_t i = 0; i < ns; ++i) c[i] = ops::count_nonzero((*guide)[i].data(), (*guide)[i].size());
            return c;
        });
    const char* dump_dir = std::getenv("TRELLIS_DECODER_DUMP");
    DeviceBuffer last_x;
    std::function<void(int64_t, int64_t)> conv2_rows;
    for (size_t si = 0; si < stages.size(); ++si) {
        const Stage& g = stages[si];
        for (size_t j = 0; j < g.convnext.size(); ++j) {   // ConvNeXt stage, ping-pong buffers
            const std::string& p = g.convnext[j];
            ops::ConvNext a = ops::convnext_of(m, p, n);
            if (a.c != c) fail(p + ": expected " + std::to_string(c) + " channels");
            if (a.conv.mfma) table.ensure_plan(s);
            const size_t need = ops::convnext_scratch(a, TSP_F32);
            if (scratch.size() < need) scratch = DeviceBuffer(need, s);
            if (h2.size() < (size_t)n * c * 4) h2 = DeviceBuffer((size_t)n * c * 4, s);
            const int next16 = j + 1 < g.convnext.size() ? conv_input16(g.convnext[j + 1]) : -1;
            if (next16 >= 0 && h16b.size() < (size_t)n * c * 2) h16b = DeviceBuffer((size_t)n * c * 2, s);
            const void* x16 = h16dt >= 0 && h16dt == a.conv.xdt ? h16.get() : nullptr;
            ops::Carve sc(scratch.get());
            ops::run_convnext(a, h.get(), TSP_F32, table.nbr.as<int32_t>(), table.plan.get(), h2.as<float>(), sc, s,
                              x16, next16 >= 0 ? h16b.get() : nullptr, next16 >= 0 ? next16 : TSP_BF16);
            std::swap(h, h2);
            std::swap(h16, h16b);
            h16dt = next16;
        }
        if (g.cin != c) fail(g.c2s + ": expected " + std::to_string(c) + " input channels");
        if (dump_dir) dump_level(dump_dir, (int)si, dc, n, si + 1 == stages.size() ? &h : nullptr, c, s);
        const std::vector<uint8_t>* ext = guide ? &(*guide)[si] : nullptr;
        if (guide && counts.empty()) {
            counts = guide_counts.get();
            start_result(counts.back());
        }
        const int c2s16 = si + 1 < stages.size() && !stages[si + 1].convnext.empty()
                              ? conv_input16(stages[si + 1].convnext[0]) : -1;
        // the last block's conv2 runs by ranges of rows as the output layer and the readback take
        // them (below), so that the copy to the host overlaps it
        const bool defer = si + 1 == stages.size() && !dump_dir;
        ops::C2SOut o = ops::run_c2s(m, g.c2s, h.as<float>(), dc.as<int32_t>(), table, g.cin, g.cout, ext, s,
                                     status.as<int32_t>(), subs_out != nullptr, guide ? counts[si] : -1, c2s16,
                                     defer);
        if (subs_out) subs_out->push_back(std::move(o.mask));
        if (defer) {
            last_x = std::move(h);   // the deferred conv2's skip reads the block's input
            conv2_rows = std::move(o.conv2_rows);
        }
        h = std::move(o.feats);
        h16 = std::move(o.feats16);
        h16dt = c2s16;
        dc = std::move(o.coords);
        table = std::move(o.table);
        if (table.n != o.m) ops::build_table(dc.as<int32_t>(), o.m, table, s, status.as<int32_t>(), true);
        n = o.m;
        c = g.cout;
        if (!result_started && si + 1 == stages.size()) start_result(n);
    }
    if (!result_started) start_result(n);
    if (dump_dir) dump_level(dump_dir, (int)stages.size(), dc, n, nullptr, c, s);
    int32_t st = 0;
    hip_check(hipMemcpyAsync(&st, status.get(), 4, hipMemcpyDeviceToHost, s), "decoder");
    hip_check(hipStreamSynchronize(s), "decoder");
    if (st) fail("decoder: a voxel coordinate lies outside [0, 2^21-3]");
    if (want_coords) {
        coords = result_coords.take();
        if (coords.size() != (size_t)n) fail("decoder: the masks' final voxel count is not the decoded one");
        tgr::download_into(coords.data(), dc.get(), (size_t)n * 12, s);
    }
    if (coords_only) return {};
    const ggml_tensor* wo = m.get("output_layer.weight");
    if (wo->ne[0] != c || wo->ne[1] != out_ch)
        fail("output_layer.weight: expected ggml shape [" + std::to_string(c) + ", " + std::to_string(out_ch) + "]");
    DeviceBuffer out((size_t)n * out_ch * 4, s);
    std::vector<float> feats = result.take();
    if (feats.size() != (size_t)n * out_ch) fail("decoder: the masks' final voxel count is not the decoded one");
    // the last block's conv2 (when deferred) and the output layer (a row-wise LayerNorm + linear) in
    // chunks of whole 512-row tiles, each chunk's rows copied to the host while the next chunk's are
    // computed
    const size_t row_bytes = (size_t)out_ch * 4;
    tgr::download_produced(feats.data(), out.get(), feats.size() * 4, 512 * row_bytes, s, [&](size_t off, size_t len) {
        const int64_t r0 = (int64_t)(off / row_bytes), nr = (int64_t)(len / row_bytes);
        if (conv2_rows) conv2_rows(r0, r0 + nr);
        ops::run_linear(m, "output_layer", h.as<float>() + r0 * c, nr, c, out_ch, true, 1e-5f,
                        out.as<float>() + r0 * out_ch, s);
    });
    return feats;
}

}  // namespace

ShapeOut shape_decode(const Model& m, const std::vector<float>& latent,
                      const std::vector<std::array<int, 3>>& coords0, int resolution) {
    ShapeOut so;
    so.coords = coords0;
    so.res = resolution;
    so.feats7 = decode(m, latent, 7, so.coords, nullptr, &so.subs, false);
    return so;
}

std::vector<std::array<int, 3>> shape_upsample(const Model& m, const std::vector<float>& latent,
                                               const std::vector<std::array<int, 3>>& coords0) {
    std::vector<std::array<int, 3>> coords = coords0;
    decode(m, latent, 7, coords, nullptr, nullptr, true);
    return coords;
}

std::vector<float> tex_decode(const Model& m, const std::vector<float>& tex_latent,
                              const std::vector<std::array<int, 3>>& coords0,
                              const std::vector<std::vector<uint8_t>>& subs) {
    std::vector<std::array<int, 3>> coords = coords0;
    // the caller has the final voxel set from shape_decode: only the features come back
    return decode(m, tex_latent, 6, coords, &subs, nullptr, false, false);
}

}  // namespace trellis
