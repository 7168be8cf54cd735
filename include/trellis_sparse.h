/*
 * trellis_sparse.h -- C ABI of the MI355X (gfx950) sparse-voxel convolution library.
 *
 * This is the drop-in boundary for trellis.cpp's sparse path (include/sparse.h,
 * src/sparse.cpp). Every entry point takes plain device pointers, sizes and a HIP stream
 * passed as void* (a hipStream_t; NULL = the null stream), never allocates on the caller's
 * behalf unless its comment says so, and is stream-ordered: it enqueues work and returns.
 *
 * Memory layouts are the reference's own, so buffers interoperate without transposes:
 *   coords  int32 [N][3]        (x, y, z) as std::vector<std::array<int,3>> (sparse.h:17)
 *   feats   [N][C] row-major    = ggml [C, N] (sparse.h:19; test_sparse_conv.cpp:42-44)
 *   nbr     int32 [27][N]       tap-major neighbour table, sentinel N (sparse.h:14-16)
 *                               tap t = kd*9 + kh*3 + kw reads the voxel at
 *                               (x+kd-1, y+kh-1, z+kw-1)
 *   weight  [Co][27][Ci]        = ggml ne [Ci, 27, Co] (sparse.h:20; convert.py:143-146)
 *   bias    float [Co]
 *
 * Coordinates must lie in [0, 2^21 - 3] on every axis (the reference's own key is exact on
 * [0, 4094], sparse.cpp:25). Errors are reported as a tsp_status with a message readable
 * through tsp_last_error(); nothing throws across this boundary.
 */
#ifndef TRELLIS_SPARSE_ABI_H
#define TRELLIS_SPARSE_ABI_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef enum {
    TSP_OK = 0,
    TSP_ERR_INVALID = 1,      /* bad argument (null pointer, negative size, ...)          */
    TSP_ERR_HIP = 2,          /* a HIP runtime call failed                                  */
    TSP_ERR_RANGE = 3,        /* a coordinate outside [0, 2^21-3]                           */
    TSP_ERR_UNSUPPORTED = 4,  /* dtype / channel combination no kernel implements           */
    TSP_ERR_WORKSPACE = 5     /* workspace smaller than the matching *_workspace_bytes()    */
} tsp_status;

typedef enum { TSP_F32 = 0, TSP_F16 = 1, TSP_BF16 = 2 } tsp_dtype;

/* Conv kernel selection. AUTO picks MFMA for 16-bit features with Ci % 32 == 0 and
 * Co % 64 == 0, THIN_MFMA and then THIN where their shapes fit, F32_MFMA where its shapes fit,
 * and NARROW otherwise.
 *   MFMA         matrix-core kernel that stages each tile's distinct neighbour rows in LDS
 *   NARROW       VALU fp32-FMA kernel over 64 x 64 output tiles, any dtype mix and channel count
 *   MFMA_GATHER  matrix-core kernel that gathers neighbour rows straight from L2/HBM (no LDS
 *                staging; same eligibility as MFMA)
 *   THIN         VALU fp32-FMA kernel with one voxel's whole output row per thread, for thin
 *                layers: Co in {4, 8, 16, 32}, Ci % 4 == 0, Ci * Co <= 512
 *   THIN_MFMA    memory-bound kernel for thin 16-bit layers: the 27 taps folded into the
 *                contraction (K = 27 Ci) of 16 x 16 x 32 matrix-core steps, each lane gathering
 *                one 16-byte piece of a neighbour row per step straight into its operand; f16/bf16
 *                feats and weights of one dtype, Ci in {8, 16, 32}, Co in {4, 8, 16, 32},
 *                Ci * Co <= 512, out f32 or the feats' dtype, 16-byte aligned feats and weights
 *   F32_MFMA     fp32 matrix-core kernel (v_mfma_f32_32x32x2_f32) for f32 feats and weights (the
 *                reference's cast-to-f32 mode, sparse.cpp:16-19): Ci % 16 == 0, Co % 32 == 0,
 *                16-byte aligned feats and weights, any output dtype; operands gathered from L2,
 *                the taps of small convs split over up to 8 waves a tile */
typedef enum {
    TSP_ALGO_AUTO = 0, TSP_ALGO_MFMA = 1, TSP_ALGO_NARROW = 2, TSP_ALGO_MFMA_GATHER = 3,
    TSP_ALGO_THIN = 4, TSP_ALGO_THIN_MFMA = 5, TSP_ALGO_F32_MFMA = 6
} tsp_algo;

/* Thread-local message for the last failing call on this thread ("" if none). */
const char* tsp_last_error(void);

/* Library version: major*10000 + minor*100 + patch. */
int tsp_version(void);

/* ---------------------------------------------------------------------------------------
 * Coordinate hash and neighbour table.
 * Replaces trellis::build_neighbor_table (include/sparse.h:17, src/sparse.cpp:21-39),
 * which builds a std::unordered_map on the host; here the map lives in device memory -- a
 * Morton-ordered grid of 8^3-voxel cells when the voxels' bounding box is compact enough for
 * the workspace, otherwise an open-addressing hash of 2x2x2 bricks (chosen on the device) --
 * and the 27 probes per voxel run on the GPU. The table is bit-identical to
 * the reference's: row of the voxel at each offset, N when absent, and for duplicate
 * coordinates the largest row index (the reference's last insert wins, sparse.cpp:26).
 * ------------------------------------------------------------------------------------- */

/* Device workspace (bytes) tsp_rulebook_build needs for n voxels (64 bytes per bucket of a
 * 2x2x2-brick hash with 1.5 n + 1024 buckets, which the cell grid reuses, plus 32 KiB); the
 * workspace must be 64-byte aligned. */
size_t tsp_rulebook_workspace_bytes(int64_t n);

/* d_coords int32 [n][3] -> d_nbr int32 [27*n]. d_status, if not NULL, is a device int32 that
 * the kernels OR with 1 when a coordinate is out of range (the caller zeroes it and reads it
 * back when it wants to check). */
int tsp_rulebook_build(const int32_t* d_coords, int64_t n, int32_t* d_nbr,
                       void* d_workspace, size_t workspace_bytes, int32_t* d_status,
                       void* stream);

/* Adds the number of active (voxel, tap) pairs #{(t,i): nbr[t*n+i] != n} to *d_count
 * (device uint64). */
int tsp_rulebook_count_pairs(const int32_t* d_nbr, int64_t n, unsigned long long* d_count,
                             void* stream);

/* ---------------------------------------------------------------------------------------
 * Submanifold 3x3x3 convolution.
 * Replaces trellis::sparse_submconv (include/sparse.h:20-22, src/sparse.cpp:61-92):
 *   out[i] = bias + sum_t W_t . feats[nbr[t*n+i]]   (absent taps contribute nothing)
 * computed in one fused gather-GEMM kernel with fp32 accumulation. feats and weight share a
 * dtype (f32, f16 or bf16), except that f32 feats may be combined with f16/bf16 weights (the
 * reference's default of f32 activations and f16 weights, sparse.cpp:17-19). out may be f32
 * or the feature dtype. d_out must not alias d_feats.
 * ------------------------------------------------------------------------------------- */
int tsp_subm_conv3x3(const void* d_feats, int feat_dtype, int64_t n, int ci,
                     const int32_t* d_nbr, const void* d_weight, int weight_dtype,
                     const float* d_bias, int co, void* d_out, int out_dtype, int algo,
                     void* stream);

/* Flags of the *_ex convs. TSP_CONV_ZERO_PAD: absent taps read an exact zero row instead of
 * the reference's padding row 0 * feats[0] (whose NaN channels, where feats[0] holds an Inf or
 * a NaN, make every output row with an absent tap NaN). The C2S block's conv2 reads such a row:
 * its padding column is silu(norm(0)) = 0 (sparse.cpp:289-306). */
enum { TSP_CONV_ZERO_PAD = 1 };

/* tsp_subm_conv3x3 with flags and, optionally, d_row0: the f32 row 0 (ci floats) that a caller
 * rounded 16-bit d_feats from (ggml's F16/BF16 mul_mat rounds F32 activations, sparse.cpp:74,
 * while the padding row 0 * feats[0] is formed before that, in F32, sparse.cpp:81-85). Where
 * d_row0 is given, the padding row's NaN channels are those of 0 * d_row0; NULL tests feats row 0
 * itself. Same replaced function, sparse.cpp:61-92; flags 0 and d_row0 NULL = the same call. */
int tsp_subm_conv3x3_ex(const void* d_feats, int feat_dtype, int64_t n, int ci,
                        const int32_t* d_nbr, const void* d_weight, int weight_dtype,
                        const float* d_bias, int co, void* d_out, int out_dtype, int algo,
                        int flags, const float* d_row0, void* stream);

/* ---------------------------------------------------------------------------------------
 * Reusable conv plan and packed weights (no counterpart call in the reference: they split
 * the work sparse_submconv repeats on every call, sparse.cpp:61-92, into what depends only on
 * the neighbour table -- shared by every conv of a decoder stage, shape_decoder.cpp:93-103 --
 * and what depends only on the weights, loaded once per model, trellis_model.cpp:96-142).
 *
 * A plan splits the voxels into tiles of 512 and holds, for each tile, its voxels' rows (grouped
 * by which of the 8 corner taps they have inside the tile), which taps each 32-row block has, the
 * set of input rows their table entries reference and each entry's rank in that set (the
 * planned conv stages those rows in LDS once per tile).
 * Packed weights hold W [Co][27][Ci] in the order the matrix-core operands are read. Both are
 * plain device buffers owned by the caller. Every present tap of every voxel is computed, in the
 * same order, so the results of a planned conv do not depend on how the plan grouped the voxels
 * (a skipped absent tap only adds exact zeros, see tsp_conv_weight_pack).
 * ------------------------------------------------------------------------------------- */
size_t tsp_conv_plan_bytes(int64_t n);
/* Tiles of 512 consecutive rows. d_plan 16-byte aligned, plan_bytes >= tsp_conv_plan_bytes(n). */
int tsp_conv_plan_build(const int32_t* d_nbr, int64_t n, void* d_plan, size_t plan_bytes,
                        void* stream);
/* Tiles of 512 voxels in the Morton order of their 8^3 cells (d_coords int32 [n][3], the
 * coordinates d_nbr was built from): compact patches of a surface, whose 27-neighbourhoods
 * overlap, so a tile stages about half the rows of one made of consecutive rows. The plan's
 * buffer also holds the build's cell grid of the coordinates; where that grid does not fit
 * (scattered or far-flung voxels) the tiles are consecutive rows. The slot sets are in (x, y, z)
 * order of the referenced voxels -- row order for coordinate-sorted sets. */
int tsp_conv_plan_build_ordered(const int32_t* d_nbr, const int32_t* d_coords, int64_t n,
                                void* d_plan, size_t plan_bytes, void* stream);
/* tsp_rulebook_build and tsp_conv_plan_build_ordered in one call, on one cell grid of the
 * coordinates (the table's workspace holds it; no counterpart in the reference, whose decoder
 * builds a table per level, shape_decoder.cpp:93, that every conv of the level then uses). The
 * table and the plan are those of the two separate calls. */
int tsp_rulebook_build_planned(const int32_t* d_coords, int64_t n, int32_t* d_nbr, void* d_workspace,
                               size_t workspace_bytes, int32_t* d_status, void* d_plan, size_t plan_bytes,
                               void* stream);

/* W [co][27][ci] (f16 or bf16; ci % 16 == 0, co % 32 == 0) -> d_packed, which must hold
 * tsp_conv_weight_packed_bytes(ci, co) bytes: the 27*ci*co values in operand order, then a
 * 256-byte trailer that records whether some weight is an Inf or a NaN. With finite weights the
 * planned convs skip the matrix-core work of a tap that is absent from a whole 32-row block of a
 * tile (it would add exact zeros); with a non-finite weight they compute it, since the padding
 * row times an Inf or a NaN is NaN, as in the reference's mul_mat. */
int tsp_conv_weight_pack(const void* d_weight, int dtype, int ci, int co, void* d_packed,
                         void* stream);
/* Bytes of packed weights for ci input and co output channels (0 for non-positive sizes). */
size_t tsp_conv_weight_packed_bytes(int ci, int co);

/* The conv of tsp_subm_conv3x3 (MFMA kernel) with a plan of d_nbr and packed weights:
 * f16/bf16 features, ci % 16 == 0, co % 64 == 0, out f32 or the feature dtype. d_nbr is still
 * read for the tiles whose rows do not fit the LDS stage. */
int tsp_subm_conv3x3_planned(const void* d_feats, int dtype, int64_t n, int ci,
                             const int32_t* d_nbr, const void* d_plan,
                             const void* d_packed_weight, const float* d_bias, int co,
                             void* d_out, int out_dtype, void* stream);

/* tsp_subm_conv3x3_planned with flags (TSP_CONV_ZERO_PAD) and, optionally, d_row0 (as for
 * tsp_subm_conv3x3_ex). flags 0 and d_row0 NULL = the same call. */
int tsp_subm_conv3x3_planned_ex(const void* d_feats, int dtype, int64_t n, int ci,
                                const int32_t* d_nbr, const void* d_plan,
                                const void* d_packed_weight, const float* d_bias, int co,
                                void* d_out, int out_dtype, int flags, const float* d_row0,
                                void* stream);

/* The C2S block's conv1 with its octant gather fused into the stores (sparse.cpp:263-291: conv1
 * maps Cin -> 8*Cout, then child m takes channels [(gidx[m]%8)*Cout, +Cout) of parent
 * gidx[m]/8; the stores here put them there directly, and the [N][8*Cout] intermediate is never
 * written). The conv of tsp_subm_conv3x3_planned with co = 8*cout; channel o*cout + k of parent
 * row i goes to row mstart[i] + #{o' < o : mask[8i+o'] != 0} of d_out [M][cout] (f32) when
 * mask[8i+o] != 0, and nowhere otherwise: every child row is written once. d_mask [8N] and
 * d_mstart [N+1] are tsp_subdivide's input mask and output (M = d_mstart[N]). cout % 64 == 0;
 * d_mask 8-byte aligned. */
int tsp_subm_conv3x3_planned_octants(const void* d_feats, int dtype, int64_t n, int ci,
                                     const int32_t* d_nbr, const void* d_plan,
                                     const void* d_packed_weight, const float* d_bias, int cout,
                                     const uint8_t* d_mask, const int32_t* d_mstart, float* d_out,
                                     void* stream);

/* The C2S block's conv2 with its skip connection added by the stores (sparse.cpp:302-323: the
 * block input x, octant block K = cin/8 repeated R = co/K times, added to conv2's output): the
 * conv of tsp_subm_conv3x3_planned with f32 output over the M children, plus
 * x[gidx[m]/8][(gidx[m]%8)*K + c/R] in output channel c of row m -- the result of
 * tsp_subm_conv3x3_planned followed by tsp_c2s_skip_add, without the second pass over the
 * output. x f32 [N][cin]; gidx [M] from tsp_subdivide; cin % 8 == 0 and R % 4 == 0. Absent
 * taps read an exact zero row (TSP_CONV_ZERO_PAD), as the reference's conv2 does. */
int tsp_subm_conv3x3_planned_skip(const void* d_feats, int dtype, int64_t n, int ci,
                                  const int32_t* d_nbr, const void* d_plan,
                                  const void* d_packed_weight, const float* d_bias, int co,
                                  const float* d_x, int cin, const int32_t* d_gidx, float* d_out,
                                  void* stream);

/* The ConvNeXt block's conv and the LayerNorm after it in one kernel (sparse.cpp:121-128:
 * h = conv(x) + bias, then norm(h) * norm.weight + norm.bias, eps 1e-6 there): the conv of
 * tsp_subm_conv3x3_planned_ex (d_row0 as there, flags 0) whose stores normalise each output row
 * over its co channels -- mean, biased variance, (h - mean) / sqrt(var + eps) * w + b, in f32 --
 * and write it in the feature dtype (the ggml mul_mat after the norm rounds its input to that
 * type, sparse.cpp:128). The f32 conv output and the separate norm pass are never needed.
 * co = 64 or 128 (one workgroup holds a whole row); norm weight and bias f32 [co]. */
int tsp_subm_conv3x3_planned_ln(const void* d_feats, int dtype, int64_t n, int ci,
                                const int32_t* d_nbr, const void* d_plan,
                                const void* d_packed_weight, const float* d_bias, int co,
                                const float* d_norm_weight, const float* d_norm_bias, float eps,
                                void* d_out, const float* d_row0, void* stream);

/* ---------------------------------------------------------------------------------------
 * 2x subdivision (channel-to-spatial) index math.
 * Replaces the host loop of trellis::sparse_c2s (src/sparse.cpp:205-222): parent i keeps
 * octant o (0..7) when d_mask[o + 8i] != 0; children are emitted parent-major, octant
 * ascending, at (2x+(o&1), 2y+((o>>1)&1), 2z+((o>>2)&1)) with gidx = o + 8i, and
 * mstart[i] = index of parent i's first child, mstart[n] = M.
 * d_child_coords must hold 8*n*3 int32 and d_gidx 8*n int32 (the most M can be); *d_m
 * (device int64) receives M.
 * ------------------------------------------------------------------------------------- */
size_t tsp_subdivide_workspace_bytes(int64_t n);
int tsp_subdivide(const uint8_t* d_mask, const int32_t* d_coords, int64_t n,
                  int32_t* d_mstart, int32_t* d_child_coords, int32_t* d_gidx, int64_t* d_m,
                  void* d_workspace, size_t workspace_bytes, void* stream);
/* tsp_subdivide without a workspace argument and without allocating: no counterpart in the
 * reference; for callers that cannot allocate device memory (HIP graph capture, serving loops,
 * harnesses that forbid hipMalloc). Its block counts live in a 1 MiB array that the library
 * holds on each device it runs on until the process ends, which covers every n tsp_subdivide
 * accepts (8n < 2^31); larger n is rejected with TSP_ERR_INVALID. Calls on one device share
 * that array, so calls that overlap on one device (different streams, other threads) race;
 * calls in stream order do not. Results are identical to tsp_subdivide's. */
int tsp_subdivide_noalloc(const uint8_t* d_mask, const int32_t* d_coords, int64_t n,
                          int32_t* d_mstart, int32_t* d_child_coords, int32_t* d_gidx,
                          int64_t* d_m, void* stream);

/* ---------------------------------------------------------------------------------------
 * Per-voxel pieces of the ConvNeXt and C2S blocks (sparse_convnext, sparse.cpp:94-137;
 * sparse_c2s, sparse.cpp:172-336). Rows are voxels, row-major [N][C].
 * ------------------------------------------------------------------------------------- */

/* out[i] = x[i] . W^T + bias for W [co][ci] (ggml_mul_mat of ne [ci, co] plus ggml_add,
 * sparse.cpp:126-128, 188). Any dtype mix; fp32 accumulation; d_bias may be NULL. f16/bf16 x and
 * weights of one dtype with out f32 or that dtype, ci % 8 == 0, co % 8 == 0 and 16-byte aligned
 * buffers run as a hipBLASLt GEMM; otherwise (or when hipBLASLt has no algorithm for the shape)
 * f16/bf16 with ci % 32 == 0 and co % 64 == 0 run on this library's matrix-core kernel, the rest
 * on its VALU kernel. The first hipBLASLt call on a device creates a hipBLASLt handle, kept until
 * the process ends; the GEMMs use no workspace. */
int tsp_linear(const void* d_x, int x_dtype, int64_t n, int ci, const void* d_weight,
               int weight_dtype, const float* d_bias, int co, void* d_out, int out_dtype,
               void* stream);

/* Activations of tsp_linear_ex. */
enum { TSP_ACT_NONE = 0, TSP_ACT_SILU = 1 };

/* out[i] = act(x[i] . W^T + bias) + residual[i]: the ConvNeXt MLP's mlp.0 -> SiLU and
 * mlp.2 -> + x (sparse.cpp:126-134: ggml_mul_mat, ggml_add of the bias, ggml_silu; ggml_mul_mat,
 * ggml_add of the bias, ggml_add of the block input) as one GEMM each, with the bias, the SiLU
 * (fp32, before the output's rounding) and the residual in the GEMM's epilogue. d_bias and
 * d_residual (f32 [n][co], 16-byte aligned; needs f32 output) may be NULL. Needs 16-bit x and
 * weights of one dtype, out f32 or that dtype, ci % 8 == 0, co % 8 == 0, 16-byte aligned buffers;
 * returns TSP_ERR_UNSUPPORTED otherwise, or when hipBLASLt has no algorithm for the shape, and the
 * caller then runs tsp_linear and the elementwise steps. */
int tsp_linear_ex(const void* d_x, int x_dtype, int64_t n, int ci, const void* d_weight,
                  int weight_dtype, const float* d_bias, int co, int act, const float* d_residual,
                  void* d_out, int out_dtype, void* stream);

/* Rows of x that tsp_linear and tsp_linear_ex hand hipBLASLt per library call: they cut n into
 * chunks of this many rows so that no operand of one call (x, out, residual) spans 2^31 bytes or
 * more (the counterpart of the reference's mul_mat_rows, sparse.cpp:41-59, which cuts at
 * 1,000,000 rows for a Vulkan grid limit). A multiple of 256 where 256 rows fit; 0 for invalid
 * arguments or a row of 2 GiB. Host arithmetic only (no device call). */
int64_t tsp_linear_rows_per_call(int ci, int co, int x_dtype, int out_dtype, int has_residual);

/* Row LayerNorm over c channels with biased variance and eps (ggml_norm, sparse.cpp:124,
 * 259, 293), then * gamma + beta when those are not NULL, then x * sigmoid(x) when silu != 0.
 * d_out may equal d_x. */
int tsp_layer_norm(const void* d_x, int x_dtype, int64_t n, int c, const float* d_gamma,
                   const float* d_beta, float eps, int silu, void* d_out, int out_dtype,
                   void* stream);

/* Channel-to-spatial gather (sparse.cpp:263-291): out[m][k] = h[gidx[m]/8][(gidx[m]%8)*cout + k]
 * for h [N][8*cout]; gidx from tsp_subdivide. */
int tsp_c2s_gather(const void* d_h, int dtype, const int32_t* d_gidx, int64_t m, int cout,
                   void* d_out, void* stream);

/* C2S skip connection (sparse.cpp:302-323): with K = cin/8 and R = cout/K,
 * acc[m][k*R + r] += x[gidx[m]/8][(gidx[m]%8)*K + k] for every r < R. */
int tsp_c2s_skip_add(const void* d_x, int x_dtype, const int32_t* d_gidx, int64_t m, int cin,
                     int cout, void* d_acc, int acc_dtype, void* stream);

/* mask[e] = logits[e] > 0 (the predicted subdivision, sparse.cpp:215). */
int tsp_mask_positive(const float* d_logits, int64_t n, uint8_t* d_mask, void* stream);

/* ---------------------------------------------------------------------------------------
 * Composite blocks: one call each for the ConvNeXt block and the C2S block's features, over the
 * entry points above, on caller-owned buffers (temporaries in the caller's workspace; nothing is
 * allocated). Every matrix product takes its input rounded as ggml's mul_mat rounds it: to the
 * weights' type for F16 and BF16 weights, unrounded for F32 weights and, with
 * TSP_BLOCK_CAST_F32 (the reference's g_sparse_cast_f32, sparse.cpp:16-19), for F16 conv weights.
 * Matrices in the reference's layouts (ggml ne reversed), vectors f32, all device pointers.
 * A *_packed pointer, optional, holds its conv weight packed by tsp_conv_weight_pack; NULL packs
 * it into the workspace on each call that runs the planned kernel.
 * ------------------------------------------------------------------------------------- */
enum { TSP_BLOCK_CAST_F32 = 2 };

typedef struct {
    const void* conv_weight;   /* [C][27][C] */
    int conv_dtype;
    const float* conv_bias;    /* [C] */
    const void* conv_packed;
    const float* norm_weight;  /* [C] */
    const float* norm_bias;    /* [C] */
    const void* mlp0_weight;   /* [4C][C] */
    int mlp0_dtype;
    const float* mlp0_bias;    /* [4C] */
    const void* mlp2_weight;   /* [C][4C] */
    int mlp2_dtype;
    const float* mlp2_bias;    /* [C] */
    const void* mlp_packed;    /* optional: mlp.0 and mlp.2 packed by tsp_convnext_mlp_pack (used where
                                  the MLP is one kernel; NULL packs them into the workspace per call) */
} tsp_convnext_weights;

/* Workspace tsp_convnext needs (only the dtypes, conv_packed and mlp_packed of w are read). */
size_t tsp_convnext_workspace_bytes(int64_t n, int c, int x_dtype, const tsp_convnext_weights* w,
                                    int has_plan, int flags);
/* SparseConvNeXtBlock3d (replaces trellis::sparse_convnext, include/sparse.h:24-25,
 * src/sparse.cpp:94-137): out f32 [n][c] = x + mlp.2(SiLU(mlp.0(LN(conv(x)) * norm.weight +
 * norm.bias))), LN eps 1e-6. x f32, or 16-bit of the conv input's type; d_plan (of d_nbr) may be
 * NULL; out must not alias x. With f32 x, c = 128 and both MLP weights of the normalised input's
 * 16-bit type, the MLP is one kernel (tsp_convnext_mlp): its weights (or mlp_packed) and the
 * workspace must then be 16-byte aligned. Arguments are checked before any work is enqueued. */
int tsp_convnext(const void* d_x, int x_dtype, int64_t n, int c, const int32_t* d_nbr,
                 const void* d_plan, const tsp_convnext_weights* w, float* d_out,
                 void* d_workspace, size_t workspace_bytes, int flags, void* stream);
/* tsp_convnext with the 16-bit copies of a decoder's residual stream (no counterpart in the
 * reference, where each conv rounds its f32 input itself; for callers that chain blocks):
 * d_x16, optional with f32 x and a 16-bit conv input, is x already rounded to the conv input's
 * type (as tsp_convnext would round it), so the block skips that pass; d_out16, optional, receives
 * out rounded to out16_dtype (TSP_BF16 or TSP_F16, round to nearest even) -- written by the MLP
 * kernel's stores where the MLP is one kernel, by a rounding pass otherwise. Both 16-byte aligned;
 * d_out16 must not alias x, x16 or out. The workspace of tsp_convnext_workspace_bytes suffices. */
int tsp_convnext_ex(const void* d_x, int x_dtype, const void* d_x16, int64_t n, int c,
                    const int32_t* d_nbr, const void* d_plan, const tsp_convnext_weights* w,
                    float* d_out, void* d_out16, int out16_dtype, void* d_workspace,
                    size_t workspace_bytes, int flags, void* stream);

/* The ConvNeXt block's MLP in one kernel (sparse.cpp:126-134: mlp.0, SiLU, mlp.2, + x, in place of
 * two mul_mats): out f32 [n][c] = x + b2 + W2 . silu(W0 . xn + b0), with the hidden layer kept on
 * chip and rounded to xn's type as a stored hidden layer would be. The weights W0 [4c][c] and
 * W2 [c][4c] (xn's 16-bit dtype) are packed first by tsp_convnext_mlp_pack into
 * tsp_convnext_mlp_packed_bytes(c) bytes (at model load; no counterpart in the reference). xn
 * [n][c] and the packed weights 16-byte aligned; x, out f32 [n][c] (out may be x); b0 [4c], b2 [c]
 * f32 or NULL. c = 128 (else TSP_ERR_UNSUPPORTED: wider blocks keep the two library GEMMs, whose
 * hidden-layer traffic is small beside their arithmetic). */
size_t tsp_convnext_mlp_packed_bytes(int c);
int tsp_convnext_mlp_pack(const void* d_w0, const void* d_w2, int dtype, int c, void* d_packed, void* stream);
int tsp_convnext_mlp(const void* d_xn, int dtype, int64_t n, int c, const void* d_packed, const float* d_b0,
                     const float* d_b2, const float* d_x, float* d_out, void* stream);

typedef struct {
    const float* norm1_weight;  /* [Cin] */
    const float* norm1_bias;    /* [Cin] */
    const void* conv1_weight;   /* [8 Cout][27][Cin] */
    int conv1_dtype;
    const float* conv1_bias;    /* [8 Cout] */
    const void* conv1_packed;
    const void* conv2_weight;   /* [Cout][27][Cout] */
    int conv2_dtype;
    const float* conv2_bias;    /* [Cout] */
    const void* conv2_packed;
} tsp_c2s_weights;

/* Workspace tsp_c2s needs (only the dtypes and *_packed of w are read). */
size_t tsp_c2s_workspace_bytes(int64_t n, int64_t m, int cin, int cout, const tsp_c2s_weights* w,
                               int has_plan, int has_child_plan, int flags);
/* The features of SparseResBlockC2S3d (replaces the feature half of trellis::sparse_c2s,
 * include/sparse.h:27-35, src/sparse.cpp:256-336) once its subdivision is known: the caller has
 * the mask (its own, or tsp_linear of to_subdiv + tsp_mask_positive), ran tsp_subdivide (mstart,
 * gidx, M children) and tsp_rulebook_build on the children. out f32 [m][cout] =
 * conv2(SiLU(LN(gather(conv1(SiLU(LN(x) * norm1.weight + norm1.bias))))), absent taps of conv2
 * reading an exact zero row) + the repeat-interleaved skip of x. d_plan (of d_nbr, for conv1)
 * and d_child_plan (of d_child_nbr, for conv2) may each be NULL. out must not alias x. With
 * d_plan, cout = 64 or 128 and both convs' weights of one 16-bit type, conv1's stores also do the
 * children's LN + SiLU (the gathered f32 rows are never written; the packed conv1 weights must
 * then be 16-byte aligned and the mask 8-byte aligned). */
int tsp_c2s(const float* d_x, int64_t n, int cin, const int32_t* d_nbr, const void* d_plan,
            const uint8_t* d_mask, const int32_t* d_mstart, const int32_t* d_gidx, int64_t m,
            int cout, const int32_t* d_child_nbr, const void* d_child_plan,
            const tsp_c2s_weights* w, float* d_out, void* d_workspace, size_t workspace_bytes,
            int flags, void* stream);
/* tsp_c2s with d_out16 (optional, 16-byte aligned, not aliasing x or out) receiving out rounded to
 * out16_dtype (TSP_BF16 or TSP_F16): the next ConvNeXt conv's 16-bit input (tsp_convnext_ex's
 * d_x16), written by conv2's stores where they add the skip, by a rounding pass otherwise (no
 * counterpart in the reference). */
int tsp_c2s_ex(const float* d_x, int64_t n, int cin, const int32_t* d_nbr, const void* d_plan,
               const uint8_t* d_mask, const int32_t* d_mstart, const int32_t* d_gidx, int64_t m,
               int cout, const int32_t* d_child_nbr, const void* d_child_plan,
               const tsp_c2s_weights* w, float* d_out, void* d_out16, int out16_dtype,
               void* d_workspace, size_t workspace_bytes, int flags, void* stream);
/* tsp_c2s_ex in two parts, for a caller that takes the output rows while conv2 still runs (no
 * counterpart in the reference; the decoder's last block, whose rows go to the host): part
 * TSP_C2S_PART_FRONT runs everything before conv2 (norm1, conv1, the gather, norm2: conv2's input
 * stays in the workspace); then TSP_C2S_PART_CONV2, with the same arguments and workspace, runs
 * conv2 and the skip over the child plan's tiles [t0, t0 + nt) (nt = -1: to the last tile), so
 * that rows [512 t0, 512 (t0 + nt)) are final when the child plan was built without coordinates
 * (tiles of consecutive rows). Both parts at once (t0 = 0, nt = -1) are tsp_c2s_ex. A tile range
 * other than all tiles needs conv2 on the matrix cores with the skip in its stores (a child plan,
 * conv2's input 16-bit, Cout % 64 == 0, Cout / (Cin / 8) % 4 == 0), else TSP_ERR_UNSUPPORTED; a
 * range past the plan's tiles is TSP_ERR_INVALID. Conv2 parts over disjoint ranges write disjoint
 * rows of d_out (and d_out16). */
enum { TSP_C2S_PART_FRONT = 1, TSP_C2S_PART_CONV2 = 2 };
int tsp_c2s_part(const float* d_x, int64_t n, int cin, const int32_t* d_nbr, const void* d_plan,
                 const uint8_t* d_mask, const int32_t* d_mstart, const int32_t* d_gidx, int64_t m,
                 int cout, const int32_t* d_child_nbr, const void* d_child_plan,
                 const tsp_c2s_weights* w, float* d_out, void* d_out16, int out16_dtype,
                 void* d_workspace, size_t workspace_bytes, int flags, int part, int64_t t0, int64_t nt,
                 void* stream);

#ifdef __cplusplus
}
#endif
#endif /* TRELLIS_SPARSE_ABI_H */
