// Pieces shared by the conv translation units (conv.hip, conv_halo.hip).
#pragma once
#include "common.hpp"

namespace tsp {

// Operand layout of v_mfma_f32_32x32x16_{bf16,f16} (64 lanes, l = lane):
//   A (32 x 16): lane l holds A[l % 32][8*(l/32) .. 8*(l/32)+7]
//   B (16 x 32): lane l holds B[8*(l/32) .. 8*(l/32)+7][l % 32]
//   D (32 x 32): lane l, element j holds D[8*(j/4) + 4*(l/32) + (j%4)][l % 32]
// A 16-channel k-step uses channels 8*(l/32) .. +7 of lane l for both A and B, so every lane's
// operand is one contiguous 16-byte load.
template <bool BF16>
__device__ __forceinline__ f32x16_t mfma32x32x16(const u32x4_t& a, const u32x4_t& b,
                                                 const f32x16_t& c) {
    if constexpr (BF16) {
        return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8_t, a),
                                                       __builtin_bit_cast(bf16x8_t, b), c, 0, 0, 0);
    } else {
        return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8_t, a),
                                                      __builtin_bit_cast(f16x8_t, b), c, 0, 0, 0);
    }
}

template <int ODT>
__device__ __forceinline__ void store_out(void* out, int64_t idx, float v) {
    Elem<ODT>::store(reinterpret_cast<typename Elem<ODT>::storage*>(out), idx, v);
}

// ---- LDS-staged ("halo") MFMA conv, conv_halo.hip --------------------------------------------
constexpr int HB_M = 512;   // output voxels per workgroup (and per plan tile)

// Bytes of a conv plan for n voxels (see tsp_conv_plan_bytes), with the scratch its build sorts in.
size_t halo_plan_bytes(int64_t n);
// whether the LDS-staged kernel can address n rows of ci channels (32-bit byte offsets)
bool halo_fits(int64_t n, int ci);

// Dense linear layers on hipBLASLt (linear_blaslt.cpp): 16-bit x and weights of one dtype, out f32
// or that dtype, ci % 8 == 0, co % 8 == 0, 16-byte aligned. blaslt_linear returns
// TSP_ERR_UNSUPPORTED when the library has no algorithm for the shape.
bool blaslt_eligible(int x_dtype, int weight_dtype, int out_dtype, int ci, int co, const void* x,
                     const void* w, const void* out);
int blaslt_linear(const void* x, int xdt, int64_t n, int ci, const void* w, const float* bias,
                  int co, int act, const float* residual, void* out, int odt, hipStream_t s);
// The ConvNeXt MLP in one kernel (mlp.hip): y = x + b2 + W2 . silu(W0 . xn + b0) for 16-bit xn and
// weights of one dtype dt, C = 128, the weights packed by mlp_pack (mlp_packed_bytes(c) bytes: W0
// then W2 in MFMA operand order), 16-byte aligned xn and packed (mlp_fused_eligible). With y16
// set, y is also stored rounded to y16_dtype (TSP_BF16 or TSP_F16) in y16 [n][c].
size_t mlp_packed_bytes(int c);
int mlp_pack(const void* w0, const void* w2, int c, void* packed, hipStream_t s);
bool mlp_fused_eligible(int dt, int c, const void* xn, const void* packed, const float* x, const float* y);
int mlp_fused(const void* xn, int dt, int64_t n, int c, const void* packed, const float* b0, const float* b2,
              const float* x, float* y, hipStream_t s, void* y16 = nullptr, int y16_dtype = TSP_BF16);
// Builds the plan of neighbour table `nbr` into `plan`: tiles in the Morton order of the voxels'
// 8^3 cells when `coords` is given, else tiles of consecutive rows.
int halo_plan_build(const int32_t* nbr, const int32_t* coords, int64_t n, void* plan, hipStream_t s);
// The same Morton-ordered plan on a cell grid already built from `coords` (region and tail of
// grid_build, with cell_of = plan_cell_of(plan, n)), e.g. the neighbour table's.
int32_t* plan_cell_of(void* plan, int64_t n);
// The most grid blocks the plan's per-block scratch holds (grid_build's block_cap for a grid whose
// blocks the plan walks).
int64_t plan_block_cap(int64_t n);
// With probe, the same launches also write the neighbour table nbr from that grid (probe->nbr,
// the grid's brick hash for the fallback), which the plan then reads only after those launches.
struct ProbeJob;
int halo_plan_build_on_grid(const int32_t* nbr, const int32_t* coords, int64_t n, void* plan,
                            const void* region, void* tail, hipStream_t s, const ProbeJob* probe = nullptr);
// Packed weights: the [co][27][ci] 16-bit values in the MFMA operand order, then a trailer of
// HB_PACK_TRAILER bytes whose first word is nonzero when some weight is an Inf or a NaN. With
// finite weights the planned conv skips the MFMAs of taps absent from a whole 32-row block (their
// products with the zero padding row are exact zeros); otherwise it computes them, as 0 * W is NaN.
constexpr int HB_PACK_TRAILER = 256;
inline size_t packed_weight_bytes(int ci, int co) { return (size_t)kTaps * ci * co * 2 + HB_PACK_TRAILER; }
// Packs [co][27][ci] 16-bit weights of dtype wdt (ci % 16 == 0, co % 32 == 0) and writes the trailer.
int halo_weight_pack(const void* w, int wdt, int ci, int co, void* packed, hipStream_t s);
// Output rows scattered to the children of a 2x subdivision: with cout > 0, the conv's output
// channel c = o * cout + k of row i goes to row mstart[i] + (octants of parent i kept before o)
// of an [M][cout] output when mask[8 i + o] != 0, and nowhere otherwise (the octant gather of
// sparse.cpp:263-291 done by the conv's stores). mask must be 8-byte aligned. With norm_silu
// set (cout == 64 or 128: the channels of a wave or of a workgroup; 16-bit output of the feature
// type) each child row
// is stored as silu((y - mean(y)) / sqrt(var(y) + norm_eps)) instead: the C2S block's norm2 + SiLU
// (no affine, sparse.cpp:293) done by the stores, its f32 input never written.
struct OctantScatter {
    const uint8_t* mask = nullptr;
    const int32_t* mstart = nullptr;
    int cout = 0;
    bool norm_silu = false;
    float norm_eps = 0.f;
    // Optional, from octant_blocks: word (tile * 4 + row group) has bit 4 o + b set when some
    // parent of 32-row block b of that row group keeps octant o. The MFMAs of a block whose
    // parents keep none of a wave's octant are skipped: those outputs are never stored.
    const uint32_t* blocks = nullptr;
};

// The words OctantScatter::blocks reads, for a stored plan of n parents and their mask [8 n]:
// out [n_tiles * 4].
int octant_blocks(const void* plan, int64_t n, const uint8_t* mask, uint32_t* out, hipStream_t s);

// The C2S skip added by the conv's stores (sparse.cpp:302-323): with cin > 0, output row m
// channel c gets x[gidx[m] / 8][(gidx[m] % 8) * K + c / R] added, K = cin / 8, R = co / K
// (R % 4 == 0), x f32 [N][cin]. With out16 set, the stores also write each output value rounded
// to bf16 (out16_bf16) or f16 into out16 [M][co]: the next conv's 16-bit input, without a
// rounding pass over the output.
struct SkipAdd {
    const float* x = nullptr;
    const int32_t* gidx = nullptr;
    int cin = 0;
    void* out16 = nullptr;
    bool out16_bf16 = true;
};

// The padding row that absent taps read. The reference's is 0 * feats[0] (submconv_pad,
// sparse.cpp:81-85): zeros, or NaN in the channels where row 0 holds an Inf or a NaN. With
// `zero` set it is an exact zero row instead (the C2S block's conv2, whose padding column is
// silu(norm(0)) = 0, sparse.cpp:289-306). `row0`, when not null, is the f32 row 0 that the
// 16-bit features were rounded from; the NaN test then reads it instead of the rounded row.
struct PadRow {
    const float* row0 = nullptr;
    bool zero = false;
};

// A LayerNorm over each output row done by the conv's stores (the ConvNeXt block's norm after
// its conv, sparse.cpp:121-135): with w set, row i of the output is
// (y - mean(y)) / sqrt(var(y) + eps) * w + b for y = conv row i (f32, bias added), the mean and
// the biased variance over its co channels, stored in the 16-bit feature type.
struct RowNorm {
    const float* w = nullptr;
    const float* b = nullptr;
    float eps = 0.f;
};

// The conv. With plan == nullptr the tile plan is built inside the kernel and `weight` is in
// the [co][27][ci] layout; with a plan, `weight` must be packed by halo_weight_pack. An
// OctantScatter or a SkipAdd needs a plan and f32 output; an OctantScatter needs cout a multiple
// of the channels one wave owns (64 when co % 128 == 0, else 32). A RowNorm needs a plan,
// co == 64 or 128 (one workgroup holds whole rows) and odt == fdt.
// Tiles [t0, t0 + nt) of a stored plan (nt < 0: every tile from t0): the planned launches run
// the persistent grid over those tiles' units only.
struct TileRange {
    int64_t t0 = 0;
    int64_t nt = -1;
};

// The planned convs at co % 128 == 0 (nct = co / 128 column tiles) run tiles [0, t) as 128-channel
// units and the rest as 64-channel units when the 128-channel units leave a last round that the
// 64-channel grid takes in one: returns that t, or 0 for one launch (cus: compute units).
int64_t column_split_tiles(int64_t n_tiles, int nct, int cus);

// tr (planned only): the plan's tiles to run, all of them by default; a narrower range runs in one
// launch of its units.
int halo_conv_launch(int fdt, int odt, const void* feats, int64_t n, int ci, const int32_t* nbr,
                     const void* plan, const void* weight, const float* bias, int co, void* out,
                     hipStream_t s, OctantScatter osc = {}, SkipAdd skip = {}, PadRow pad = {},
                     RowNorm ln = {}, TileRange tr = {});

// tsp_subm_conv3x3_planned_octants with, when blocks is not null, the MFMAs of row blocks whose
// parents keep none of a wave's octant skipped (blocks from octant_blocks).
int planned_octants(const void* feats, int dtype, int64_t n, int ci, const int32_t* nbr, const void* plan,
                    const void* packed, const float* bias, int cout, const uint8_t* mask, const int32_t* mstart,
                    float* out, const uint32_t* blocks, hipStream_t s);

// tsp_subm_conv3x3_planned_skip with, when out16 is not null, out also rounded to out16_dtype
// (TSP_BF16 or TSP_F16) in out16 [n][co] by the same stores.
// tr: the plan's tiles whose rows are computed (all by default).
int planned_skip(const void* feats, int dtype, int64_t n, int ci, const int32_t* nbr, const void* plan,
                 const void* packed, const float* bias, int co, const float* x, int cin, const int32_t* gidx,
                 float* out, void* out16, int out16_dtype, hipStream_t s, TileRange tr = {});

// The thin-channel matrix-core conv (conv_thin_mfma.hip): f16/bf16 features and weights of one
// dtype, Ci in {8, 16, 32}, Co in {4, 8, 16, 32}, Ci * Co <= 512, a neighbour table, 16-byte
// aligned features and weights (output 8-byte, f32 output 16-byte). Returns TSP_ERR_UNSUPPORTED
// (with no message) for anything else.
bool thin_mfma_fits(int fdt, int wdt, int ci, int co);
int thin_mfma_launch(int fdt, int wdt, int odt, const void* feats, int64_t n, int ci, const int32_t* nbr,
                     const void* weight, const float* bias, int co, void* out, hipStream_t s, PadRow pad);

// The fp32 matrix-core conv (conv_f32_mfma.hip): f32 features and weights, Ci % 16 == 0,
// Co % 32 == 0, a neighbour table, 16-byte aligned features and weights. Returns
// TSP_ERR_UNSUPPORTED (with no message) for anything else.
bool f32_mfma_fits(int fdt, int wdt, int ci, int co, const void* feats, const void* weight);
int f32_mfma_launch(int fdt, int wdt, int odt, const void* feats, int64_t n, int ci, const int32_t* nbr,
                    const void* weight, const float* bias, int co, void* out, hipStream_t s, PadRow pad);

// The thin-channel VALU conv (conv_thin.hip): Co in {4, 8, 16, 32}, Ci % 4 == 0, Ci * Co <= 512,
// a neighbour table, 16-byte aligned features. Returns TSP_ERR_UNSUPPORTED (with no message) for
// anything else.
bool thin_fits(int ci, int co);
int thin_conv_launch(int fdt, int wdt, int odt, const void* feats, int64_t n, int ci, const int32_t* nbr,
                     const void* weight, const float* bias, int co, void* out, hipStream_t s, PadRow pad);

}  // namespace tsp
