// The ConvNeXt block and the feature half of the C2S block as single C-ABI calls, composed from
// the library's own entry points on caller-owned buffers (no allocation: temporaries come from
// the caller's workspace, carved by the same walk that sizes it).
//
// Every matrix product takes its input rounded as ggml's mul_mat rounds it (sparse.cpp:74, 126,
// 128): to the weights' type for F16 and BF16 weights, unrounded for F32 weights and for F16
// conv weights under TSP_BLOCK_CAST_F32 (the reference's g_sparse_cast_f32 casts them, w32,
// sparse.cpp:16-19).
#include <algorithm>

#include "blocks_internal.hpp"
#include "common.hpp"
#include "conv_internal.hpp"

namespace tsp {
namespace {

// Workspace carving: a null base only sizes (take() returns null), a real one hands out pieces.
struct Carve {
    char* base;
    size_t off = 0;
    explicit Carve(void* b) : base(static_cast<char*>(b)) {}
    void* take(size_t bytes) {
        void* p = base ? base + off : nullptr;
        off += (bytes + 255) / 256 * 256;
        return p;
    }
};

int act_dtype(int wdt, bool conv_weight, int flags) {
    if (wdt == TSP_F16) return conv_weight && (flags & TSP_BLOCK_CAST_F32) ? TSP_F32 : TSP_F16;
    return wdt;
}

bool is16(int dt) { return dt == TSP_F16 || dt == TSP_BF16; }

// One conv of the blocks: out f32 [n][co] = conv(x) with x of dtype xdt (already rounded to
// act_dtype; row0, when given, the f32 row it was rounded from); the planned matrix-core kernel
// when a plan is given and the shapes fit it (packed weights from `packed` or packed into the
// workspace), otherwise tsp_subm_conv3x3_ex's kernels.
struct ConvPlan {
    bool planned;
    bool pack_here;
};

ConvPlan conv_plan(int xdt, int ci, int co, const void* plan, const void* packed) {
    ConvPlan p;
    p.planned = plan && is16(xdt) && ci % 16 == 0 && co % 64 == 0;
    p.pack_here = p.planned && !packed;
    return p;
}

int run_conv(const void* x, int xdt, int64_t n, int ci, const int32_t* nbr, const void* plan,
             const void* w, int wdt, const void* packed, const float* bias, int co, float* out, int flags,
             const float* row0, Carve& ws, hipStream_t s) {
    const ConvPlan cp = conv_plan(xdt, ci, co, plan, packed);
    void* pk = cp.pack_here ? ws.take(tsp_conv_weight_packed_bytes(ci, co)) : nullptr;
    if (!ws.base) return TSP_OK;
    if (cp.planned) {
        if (cp.pack_here) {
            if (int st = tsp_conv_weight_pack(w, wdt, ci, co, pk, s)) return st;
            packed = pk;
        }
        return tsp_subm_conv3x3_planned_ex(x, xdt, n, ci, nbr, plan, packed, bias, co, out, TSP_F32, flags, row0, s);
    }
    return tsp_subm_conv3x3_ex(x, xdt, n, ci, nbr, w, wdt, bias, co, out, TSP_F32,
                               TSP_ALGO_AUTO, flags, row0, s);
}

// The ConvNeXt conv and the LayerNorm after it in one kernel (the planned kernel's row-norm
// stores, straight into the norm's 16-bit output) when a plan is given, the conv's rows fit one
// workgroup (C = 64 or 128) and the norm's output type is the conv input's; the f32 conv output
// and the separate norm pass are then never needed.
bool ln_fused(int cdt, int adt0, int c, const void* plan) {
    return plan && is16(cdt) && adt0 == cdt && (c == 64 || c == 128);
}

int run_conv_ln(const void* x, int xdt, int64_t n, int c, const int32_t* nbr, const void* plan, const void* w,
                int wdt, const void* packed, const float* bias, const float* norm_w, const float* norm_b,
                const float* row0, void* hn, Carve& ws, hipStream_t s) {
    void* pk = packed ? nullptr : ws.take(tsp_conv_weight_packed_bytes(c, c));
    if (!ws.base) return TSP_OK;
    if (n == 0) return TSP_OK;
    if (!packed) {
        if (int st = tsp_conv_weight_pack(w, wdt, c, c, pk, s)) return st;
        packed = pk;
    }
    TSP_REQUIRE(reinterpret_cast<uintptr_t>(x) % 16 == 0 && reinterpret_cast<uintptr_t>(packed) % 16 == 0 &&
                    reinterpret_cast<uintptr_t>(hn) % 16 == 0,
                TSP_ERR_INVALID, "tsp_convnext: conv buffers must be 16-byte aligned");
    TSP_REQUIRE(halo_fits(n, c), TSP_ERR_UNSUPPORTED, "tsp_convnext: %lld rows of %d channels exceed the "
                "planned conv's 4 GiB of features", (long long)n, c);
    PadRow pad;
    pad.row0 = row0;
    RowNorm ln;
    ln.w = norm_w;
    ln.b = norm_b;
    ln.eps = 1e-6f;
    return halo_conv_launch(xdt, xdt, x, n, c, nbr, plan, packed, bias, c, hn, s, OctantScatter{}, SkipAdd{},
                            pad, ln);
}

// the rows of one MLP chunk: its f32 hidden layer [chunk][4C] stays within 1 GiB
int64_t mlp_chunk(int64_t n, int c) {
    return std::max<int64_t>(1, std::min<int64_t>(n, (int64_t(1) << 30) / (16 * (int64_t)c)));
}

// x16 (optional): x already rounded to the conv input's 16-bit type; out16 (optional): out rounded
// to out16dt, written by the MLP kernel's stores where it runs, else by a rounding pass.
int convnext_walk(const void* x, int xdt, const void* x16, int64_t n, int c, const int32_t* nbr, const void* plan,
                  const tsp_convnext_weights& w, float* out, void* out16, int out16dt, int flags, Carve& ws,
                  hipStream_t s) {
    const int cdt = act_dtype(w.conv_dtype, true, flags);
    const int adt0 = act_dtype(w.mlp0_dtype, false, flags), adt2 = act_dtype(w.mlp2_dtype, false, flags);
    const int64_t chunk = mlp_chunk(n, c);
    // conv input rounded (when x is f32 and the conv takes 16-bit input; x is f32 there, the entry
    // point rejects other mixes)
    void* xr16 = xdt != cdt && !x16 ? ws.take((size_t)n * c * dtype_size(cdt)) : nullptr;
    const void* xc = x16 ? x16 : xr16 ? xr16 : x;
    const bool fuse = ln_fused(cdt, adt0, c, plan);
    // the MLP in one kernel, its 16-bit hidden layer never stored (C = 128, one 16-bit dtype)
    const bool mlp1 = is16(adt0) && adt2 == adt0 && w.mlp0_dtype == adt0 && w.mlp2_dtype == adt0 &&
                      xdt == TSP_F32 && c == 128;
    float* h = fuse ? nullptr : static_cast<float*>(ws.take((size_t)n * c * 4));
    void* hn = ws.take((size_t)n * c * dtype_size(adt0));
    void* mlp_packed = mlp1 && !w.mlp_packed ? ws.take(mlp_packed_bytes(c)) : nullptr;
    float* hid = mlp1 ? nullptr : static_cast<float*>(ws.take((size_t)chunk * 4 * c * 4));
    void* hid_in = mlp1 || adt2 == TSP_F32 ? hid : ws.take((size_t)chunk * 4 * c * 2);
    const float* row0 = xdt == TSP_F32 && cdt != TSP_F32 ? static_cast<const float*>(x) : nullptr;
    if (!ws.base) {
        // the conv's own pieces (packed weights) are sized by the same walk
        if (fuse) return run_conv_ln(xc, cdt, n, c, nbr, plan, w.conv_weight, w.conv_dtype, w.conv_packed,
                                     w.conv_bias, w.norm_weight, w.norm_bias, row0, hn, ws, s);
        return run_conv(xc, cdt, n, c, nbr, plan, w.conv_weight, w.conv_dtype, w.conv_packed, w.conv_bias, c, h, 0,
                        row0, ws, s);
    }
    // every check before the first launch, so that an error leaves no work behind
    if (mlp1) {
        auto al = [](const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; };
        TSP_REQUIRE(w.mlp_packed ? al(w.mlp_packed) : al(w.mlp0_weight) && al(w.mlp2_weight), TSP_ERR_INVALID,
                    "tsp_convnext: the MLP weights (or mlp_packed) must be 16-byte aligned");
        TSP_REQUIRE(mlp_fused_eligible(adt0, c, hn, w.mlp_packed ? w.mlp_packed : mlp_packed,
                                       static_cast<const float*>(x), out),
                    TSP_ERR_INVALID, "tsp_convnext: the workspace must be 16-byte aligned");
    }
    if (xr16)
        if (int st = f32_to(static_cast<const float*>(x), n * c, xr16, cdt, false, s)) return st;
    if (fuse) {
        if (int st = run_conv_ln(xc, cdt, n, c, nbr, plan, w.conv_weight, w.conv_dtype, w.conv_packed, w.conv_bias,
                                 w.norm_weight, w.norm_bias, row0, hn, ws, s))
            return st;
        if (!ws.base) return TSP_OK;
    } else {
        if (int st = run_conv(xc, cdt, n, c, nbr, plan, w.conv_weight, w.conv_dtype, w.conv_packed, w.conv_bias,
                              c, h, 0, row0, ws, s))
            return st;
        if (!ws.base) return TSP_OK;
        if (int st = tsp_layer_norm(h, TSP_F32, n, c, w.norm_weight, w.norm_bias, 1e-6f, 0, hn, adt0, s)) return st;
    }
    if (mlp1) {
        const void* mp = w.mlp_packed;
        if (!mp) {
            if (int st = mlp_pack(w.mlp0_weight, w.mlp2_weight, c, mlp_packed, s)) return st;
            mp = mlp_packed;
        }
        return mlp_fused(hn, adt0, n, c, mp, w.mlp0_bias, w.mlp2_bias, static_cast<const float*>(x), out, s, out16,
                         out16dt);
    }
    const size_t aes = dtype_size(adt0), xes = dtype_size(xdt);
    for (int64_t r0 = 0; r0 < n; r0 += chunk) {
        const int64_t nr = std::min(chunk, n - r0);
        const void* hin = static_cast<const char*>(hn) + (size_t)r0 * c * aes;
        const void* xr = static_cast<const char*>(x) + (size_t)r0 * c * xes;
        float* yr = out + r0 * c;
        // mlp.0 + bias + SiLU, stored in mlp.2's input type: one library GEMM where it runs the
        // shape, else the GEMM then the SiLU pass
        int st = TSP_ERR_UNSUPPORTED;
        if (is16(adt0) && is16(adt2))
            st = tsp_linear_ex(hin, adt0, nr, c, w.mlp0_weight, w.mlp0_dtype, w.mlp0_bias, 4 * c, TSP_ACT_SILU,
                               nullptr, hid_in, adt2, s);
        if (st == TSP_ERR_UNSUPPORTED) {
            if ((st = tsp_linear(hin, adt0, nr, c, w.mlp0_weight, w.mlp0_dtype, w.mlp0_bias, 4 * c, hid, TSP_F32, s)))
                return st;
            st = f32_to(hid, nr * 4 * c, hid_in, adt2, true, s);
        }
        if (st) return st;
        // mlp.2 + bias + the block input
        st = TSP_ERR_UNSUPPORTED;
        if (is16(adt2) && xdt == TSP_F32)
            st = tsp_linear_ex(hid_in, adt2, nr, 4 * c, w.mlp2_weight, w.mlp2_dtype, w.mlp2_bias, c, TSP_ACT_NONE,
                               static_cast<const float*>(xr), yr, TSP_F32, s);
        if (st == TSP_ERR_UNSUPPORTED) {
            if ((st = tsp_linear(hid_in, adt2, nr, 4 * c, w.mlp2_weight, w.mlp2_dtype, w.mlp2_bias, c, yr, TSP_F32, s)))
                return st;
            st = add_to(yr, xr, xdt, nr * c, s);
        }
        if (st) return st;
    }
    return out16 ? f32_to(out, n * c, out16, out16dt, false, s) : TSP_OK;
}

// The C2S block after its subdivision (sparse.cpp:256-336): norm1 + SiLU -> conv1 (Cin -> 8 Cout)
// -> octant gather -> norm2 (no affine) + SiLU -> conv2 (exact zero padding row) -> + skip.
// part: TSP_C2S_PART_FRONT runs everything before conv2 (its input stays in the workspace),
// TSP_C2S_PART_CONV2 conv2 and the skip, over the child plan's tiles `tiles` (all by default).
int c2s_walk(const float* x, int64_t n, int cin, const int32_t* nbr, const void* plan, const uint8_t* mask,
             const int32_t* mstart, const int32_t* gidx, int64_t m, int cout, const int32_t* cnbr,
             const void* cplan, const tsp_c2s_weights& w, float* out, void* out16, int out16dt, int flags,
             Carve& ws, hipStream_t s, int part = TSP_C2S_PART_FRONT | TSP_C2S_PART_CONV2, TileRange tiles = {}) {
    const int in1 = act_dtype(w.conv1_dtype, true, flags), in2 = act_dtype(w.conv2_dtype, true, flags);
    const ConvPlan cp1 = conv_plan(in1, cin, 8 * cout, plan, w.conv1_packed);
    const ConvPlan cp2 = conv_plan(in2, cout, cout, cplan, w.conv2_packed);
    // conv1's stores do the octant gather on the planned matrix-core kernel (Cout % 64 == 0),
    // otherwise its [N][8 Cout] output goes through the gather pass; conv2's stores add the skip
    // when each skip element spans a multiple of 4 channels, otherwise the skip pass does
    const bool octants = cp1.planned && cout % 64 == 0;
    const bool skip_in_stores = cp2.planned && (cout / (cin / 8)) % 4 == 0;
    // at Cout = 64 / 128 (a wave's / a workgroup's channels: whole child rows) conv1's stores also
    // do norm2 + SiLU and write conv2's 16-bit input directly
    const bool norm_in_stores = octants && (cout == 64 || cout == 128) && is16(in1) && in2 == in1;
    void* h0 = ws.take((size_t)n * cin * dtype_size(in1));
    float* h1 = octants ? nullptr : static_cast<float*>(ws.take((size_t)n * 8 * cout * 4));
    float* g = norm_in_stores ? nullptr : static_cast<float*>(ws.take((size_t)m * cout * 4));
    void* h2 = ws.take((size_t)m * cout * dtype_size(in2));
    void* pk1 = cp1.pack_here ? ws.take(tsp_conv_weight_packed_bytes(cin, 8 * cout)) : nullptr;
    void* pk2 = cp2.pack_here ? ws.take(tsp_conv_weight_packed_bytes(cout, cout)) : nullptr;
    // with octant stores: which of conv1's row blocks hold a parent keeping each octant (the
    // others' MFMAs for that octant's channels are skipped; their outputs are never stored)
    auto* blocks = octants ? static_cast<uint32_t*>(ws.take((size_t)ceil_div(n, HB_M) * 4 * 4)) : nullptr;
    if (!ws.base) return TSP_OK;
    int st;
    const void* p2 = pk2 ? pk2 : w.conv2_packed;
    if (part & TSP_C2S_PART_FRONT) {
        if ((st = tsp_layer_norm(x, TSP_F32, n, cin, w.norm1_weight, w.norm1_bias, 1e-6f, 1, h0, in1, s))) return st;
        const void* p1 = w.conv1_packed;
        if (pk1) {
            if ((st = tsp_conv_weight_pack(w.conv1_weight, w.conv1_dtype, cin, 8 * cout, pk1, s))) return st;
            p1 = pk1;
        }
        if (octants && (st = octant_blocks(plan, n, mask, blocks, s))) return st;
        if (norm_in_stores) {
            TSP_REQUIRE((reinterpret_cast<uintptr_t>(p1) & 15) == 0 &&
                            (reinterpret_cast<uintptr_t>(mask) & 7) == 0,
                        TSP_ERR_INVALID, "tsp_c2s: packed conv1 weights must be 16-byte aligned, the mask 8-byte");
            OctantScatter osc;
            osc.mask = mask;
            osc.mstart = mstart;
            osc.cout = cout;
            osc.norm_silu = true;
            osc.norm_eps = 1e-6f;
            osc.blocks = blocks;
            st = halo_conv_launch(in1, in2, h0, n, cin, nbr, plan, p1, w.conv1_bias, 8 * cout, h2, s, osc);
        } else if (octants) {
            st = planned_octants(h0, in1, n, cin, nbr, plan, p1, w.conv1_bias, cout, mask, mstart, g, blocks, s);
        } else {
            if (cp1.planned)
                st = tsp_subm_conv3x3_planned_ex(h0, in1, n, cin, nbr, plan, p1, w.conv1_bias, 8 * cout, h1,
                                                 TSP_F32, 0, nullptr, s);
            else
                st = tsp_subm_conv3x3_ex(h0, in1, n, cin, nbr, w.conv1_weight, w.conv1_dtype, w.conv1_bias,
                                         8 * cout, h1, TSP_F32, TSP_ALGO_AUTO, 0, nullptr, s);
            if (!st) st = tsp_c2s_gather(h1, TSP_F32, gidx, m, cout, g, s);
        }
        if (st) return st;
        if (!norm_in_stores && (st = tsp_layer_norm(g, TSP_F32, m, cout, nullptr, nullptr, 1e-6f, 1, h2, in2, s)))
            return st;
        if (pk2 && (st = tsp_conv_weight_pack(w.conv2_weight, w.conv2_dtype, cout, cout, pk2, s))) return st;
    }
    if (!(part & TSP_C2S_PART_CONV2)) return TSP_OK;
    if (skip_in_stores)
        return planned_skip(h2, in2, m, cout, cnbr, cplan, p2, w.conv2_bias, cout, x, cin, gidx, out, out16, out16dt, s,
                            tiles);
    TSP_REQUIRE(tiles.t0 == 0 && tiles.nt < 0, TSP_ERR_UNSUPPORTED,
                "tsp_c2s_part: conv2 over a range of tiles needs it on the matrix cores with the skip in its "
                "stores (a child plan, 16-bit weights, Cout %% 64 == 0, Cout / (Cin / 8) %% 4 == 0)");
    if (cp2.planned)
        st = tsp_subm_conv3x3_planned_ex(h2, in2, m, cout, cnbr, cplan, p2, w.conv2_bias, cout, out, TSP_F32,
                                         TSP_CONV_ZERO_PAD, nullptr, s);
    else
        st = tsp_subm_conv3x3_ex(h2, in2, m, cout, cnbr, w.conv2_weight, w.conv2_dtype, w.conv2_bias, cout, out,
                                 TSP_F32, TSP_ALGO_AUTO,
                                 TSP_CONV_ZERO_PAD, nullptr, s);
    if (st) return st;
    if ((st = tsp_c2s_skip_add(x, TSP_F32, gidx, m, cin, cout, out, TSP_F32, s))) return st;
    return out16 ? f32_to(out, m * cout, out16, out16dt, false, s) : TSP_OK;
}

// a non-null stand-in for the plan when sizing (sizing never dereferences it)
const void* plan_flag(int has_plan) { return has_plan ? reinterpret_cast<const void*>(uintptr_t(1)) : nullptr; }

}  // namespace
}  // namespace tsp

using namespace tsp;

extern "C" size_t tsp_convnext_workspace_bytes(int64_t n, int c, int x_dtype, const tsp_convnext_weights* w,
                                               int has_plan, int flags) {
    if (n <= 0 || c <= 0 || !w) return 0;
    Carve ws(nullptr);
    convnext_walk(nullptr, x_dtype, nullptr, n, c, nullptr, plan_flag(has_plan), *w, nullptr, nullptr, TSP_BF16, flags, ws,
                  nullptr);
    return ws.off;
}

extern "C" int tsp_convnext_ex(const void* d_x, int x_dtype, const void* d_x16, int64_t n, int c,
                               const int32_t* d_nbr, const void* d_plan, const tsp_convnext_weights* w,
                               float* d_out, void* d_out16, int out16_dtype, void* d_workspace,
                               size_t workspace_bytes, int flags, void* stream) {
    clear_error();
    TSP_REQUIRE(w, TSP_ERR_INVALID, "tsp_convnext: null weights");
    TSP_REQUIRE(n >= 0 && n < (int64_t)INT32_MAX && c > 0, TSP_ERR_INVALID, "tsp_convnext: n=%lld c=%d",
                (long long)n, c);
    TSP_REQUIRE((flags & ~TSP_BLOCK_CAST_F32) == 0, TSP_ERR_INVALID, "tsp_convnext: bad flags %d", flags);
    TSP_REQUIRE(dtype_valid(x_dtype) && dtype_valid(w->conv_dtype) && dtype_valid(w->mlp0_dtype) && dtype_valid(w->mlp2_dtype),
                TSP_ERR_INVALID, "tsp_convnext: bad dtype");
    const int cdt = act_dtype(w->conv_dtype, true, flags);
    TSP_REQUIRE(x_dtype == TSP_F32 || x_dtype == cdt, TSP_ERR_UNSUPPORTED,
                "tsp_convnext: 16-bit x must have the conv input's type (%d), got %d", cdt, x_dtype);
    TSP_REQUIRE(!d_x16 || (x_dtype == TSP_F32 && is16(cdt)), TSP_ERR_INVALID,
                "tsp_convnext: a rounded copy of x goes with f32 x and a 16-bit conv input");
    TSP_REQUIRE(!d_out16 || out16_dtype == TSP_BF16 || out16_dtype == TSP_F16, TSP_ERR_INVALID,
                "tsp_convnext: the rounded copy of out is bf16 or f16, not dtype %d", out16_dtype);
    if (n == 0) return TSP_OK;
    TSP_REQUIRE(d_x && d_nbr && d_out && w->conv_weight && w->conv_bias && w->norm_weight && w->norm_bias &&
                    w->mlp0_weight && w->mlp0_bias && w->mlp2_weight && w->mlp2_bias,
                TSP_ERR_INVALID, "tsp_convnext: null pointer");
    TSP_REQUIRE(static_cast<const void*>(d_out) != d_x, TSP_ERR_INVALID, "tsp_convnext: out aliases x");
    TSP_REQUIRE(!d_out16 || (d_out16 != d_x && d_out16 != d_out && d_out16 != d_x16), TSP_ERR_INVALID,
                "tsp_convnext: the rounded copy of out aliases another buffer");
    auto al16 = [](const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; };
    TSP_REQUIRE(al16(d_x16) && al16(d_out16), TSP_ERR_INVALID, "tsp_convnext: the rounded copies must be 16-byte aligned");
    const size_t need = tsp_convnext_workspace_bytes(n, c, x_dtype, w, d_plan != nullptr, flags);
    TSP_REQUIRE(d_workspace && workspace_bytes >= need, TSP_ERR_WORKSPACE,
                "tsp_convnext: workspace %zu < %zu bytes", workspace_bytes, need);
    Carve ws(d_workspace);
    return convnext_walk(d_x, x_dtype, d_x16, n, c, d_nbr, d_plan, *w, d_out, d_out16, out16_dtype, flags, ws,
                         as_stream(stream));
}

extern "C" int tsp_convnext(const void* d_x, int x_dtype, int64_t n, int c, const int32_t* d_nbr,
                            const void* d_plan, const tsp_convnext_weights* w, float* d_out,
                            void* d_workspace, size_t workspace_bytes, int flags, void* stream) {
    return tsp_convnext_ex(d_x, x_dtype, nullptr, n, c, d_nbr, d_plan, w, d_out, nullptr, TSP_BF16, d_workspace,
                           workspace_bytes, flags, stream);
}

extern "C" size_t tsp_c2s_workspace_bytes(int64_t n, int64_t m, int cin, int cout, const tsp_c2s_weights* w,
                                          int has_plan, int has_child_plan, int flags) {
    if (n <= 0 || m < 0 || cin <= 0 || cout <= 0 || !w) return 0;
    Carve ws(nullptr);
    c2s_walk(nullptr, n, cin, nullptr, plan_flag(has_plan), nullptr, nullptr, nullptr, m, cout, nullptr,
             plan_flag(has_child_plan), *w, nullptr, nullptr, TSP_BF16, flags, ws, nullptr);
    return ws.off;
}

extern "C" int tsp_c2s_part(const float* d_x, int64_t n, int cin, const int32_t* d_nbr, const void* d_plan,
                            const uint8_t* d_mask, const int32_t* d_mstart, const int32_t* d_gidx, int64_t m,
                            int cout, const int32_t* d_child_nbr, const void* d_child_plan,
                            const tsp_c2s_weights* w, float* d_out, void* d_out16, int out16_dtype,
                            void* d_workspace, size_t workspace_bytes, int flags, int part, int64_t t0, int64_t nt,
                            void* stream) {
    clear_error();
    TSP_REQUIRE(part >= TSP_C2S_PART_FRONT && part <= (TSP_C2S_PART_FRONT | TSP_C2S_PART_CONV2), TSP_ERR_INVALID,
                "tsp_c2s_part: bad part %d", part);
    TSP_REQUIRE(t0 >= 0 && (nt >= 0 || nt == -1), TSP_ERR_INVALID, "tsp_c2s_part: bad tiles t0=%lld nt=%lld",
                (long long)t0, (long long)nt);
    TSP_REQUIRE((part & TSP_C2S_PART_CONV2) || (t0 == 0 && nt == -1), TSP_ERR_INVALID,
                "tsp_c2s_part: a tile range is for the conv2 part");
    TSP_REQUIRE(w, TSP_ERR_INVALID, "tsp_c2s: null weights");
    TSP_REQUIRE(n >= 0 && 8 * n < (int64_t)INT32_MAX && m >= 0 && m <= 8 * n, TSP_ERR_INVALID,
                "tsp_c2s: n=%lld m=%lld out of range", (long long)n, (long long)m);
    TSP_REQUIRE(cin > 0 && cin % 8 == 0 && cout > 0 && cout % (cin / 8) == 0, TSP_ERR_INVALID,
                "tsp_c2s: needs Cin %% 8 == 0 and Cout %% (Cin/8) == 0 (Cin=%d Cout=%d)", cin, cout);
    TSP_REQUIRE((flags & ~TSP_BLOCK_CAST_F32) == 0, TSP_ERR_INVALID, "tsp_c2s: bad flags %d", flags);
    TSP_REQUIRE(dtype_valid(w->conv1_dtype) && dtype_valid(w->conv2_dtype), TSP_ERR_INVALID, "tsp_c2s: bad dtype");
    TSP_REQUIRE(!d_out16 || out16_dtype == TSP_BF16 || out16_dtype == TSP_F16, TSP_ERR_INVALID,
                "tsp_c2s: the rounded copy of out is bf16 or f16, not dtype %d", out16_dtype);
    if (m == 0) return TSP_OK;
    TSP_REQUIRE(d_x && d_nbr && d_mask && d_mstart && d_gidx && d_child_nbr && d_out && w->norm1_weight &&
                    w->norm1_bias && w->conv1_weight && w->conv1_bias && w->conv2_weight && w->conv2_bias,
                TSP_ERR_INVALID, "tsp_c2s: null pointer");
    TSP_REQUIRE(d_out != d_x, TSP_ERR_INVALID, "tsp_c2s: out aliases x");
    TSP_REQUIRE(!d_out16 || (d_out16 != static_cast<const void*>(d_x) && d_out16 != static_cast<void*>(d_out)),
                TSP_ERR_INVALID, "tsp_c2s: the rounded copy of out aliases another buffer");
    TSP_REQUIRE((reinterpret_cast<uintptr_t>(d_out16) & 15) == 0, TSP_ERR_INVALID,
                "tsp_c2s: the rounded copy of out must be 16-byte aligned");
    const size_t need = tsp_c2s_workspace_bytes(n, m, cin, cout, w, d_plan != nullptr, d_child_plan != nullptr, flags);
    TSP_REQUIRE(d_workspace && workspace_bytes >= need, TSP_ERR_WORKSPACE, "tsp_c2s: workspace %zu < %zu bytes",
                workspace_bytes, need);
    Carve ws(d_workspace);
    return c2s_walk(d_x, n, cin, d_nbr, d_plan, d_mask, d_mstart, d_gidx, m, cout, d_child_nbr, d_child_plan, *w,
                    d_out, d_out16, out16_dtype, flags, ws, as_stream(stream), part, TileRange{t0, nt});
}

extern "C" int tsp_c2s_ex(const float* d_x, int64_t n, int cin, const int32_t* d_nbr, const void* d_plan,
                          const uint8_t* d_mask, const int32_t* d_mstart, const int32_t* d_gidx, int64_t m, int cout,
                          const int32_t* d_child_nbr, const void* d_child_plan, const tsp_c2s_weights* w,
                          float* d_out, void* d_out16, int out16_dtype, void* d_workspace, size_t workspace_bytes,
                          int flags, void* stream) {
    return tsp_c2s_part(d_x, n, cin, d_nbr, d_plan, d_mask, d_mstart, d_gidx, m, cout, d_child_nbr, d_child_plan, w,
                        d_out, d_out16, out16_dtype, d_workspace, workspace_bytes, flags,
                        TSP_C2S_PART_FRONT | TSP_C2S_PART_CONV2, 0, -1, stream);
}

extern "C" int tsp_c2s(const float* d_x, int64_t n, int cin, const int32_t* d_nbr, const void* d_plan,
                       const uint8_t* d_mask, const int32_t* d_mstart, const int32_t* d_gidx, int64_t m, int cout,
                       const int32_t* d_child_nbr, const void* d_child_plan, const tsp_c2s_weights* w,
                       float* d_out, void* d_workspace, size_t workspace_bytes, int flags, void* stream) {
    return tsp_c2s_ex(d_x, n, cin, d_nbr, d_plan, d_mask, d_mstart, d_gidx, m, cout, d_child_nbr, d_child_plan, w,
                      d_out, nullptr, TSP_BF16, d_workspace, workspace_bytes, flags, stream);
}
