/*
 * CPU oracle for the sparse submanifold 3x3x3 conv path.
 *
 * TEST INFRASTRUCTURE ONLY. This library is the checker that the HIP library is
 * compared against. Only tests/, __graft_entry__.smoke() and bench.py's CPU
 * baseline leg may load it; the product path never does.
 *
 * Every function restates an algorithm of the reference (pwilkin/trellis.cpp);
 * the file:line it follows is given beside each declaration.
 *
 * Layouts (identical to the reference's memory layouts):
 *   coords   int32 [N][3]   (x, y, z)              -- std::vector<std::array<int,3>>
 *   feats    f32   [N][Ci]  row-major                -- ggml [Ci, N]
 *   nbr      int32 [27][N]  tap-major, sentinel N    -- sparse.h:14-16
 *   weight   f32   [Co][27][Ci]                      -- ggml [Ci, 27, Co]
 *   bias     f32   [Co]
 *   out      f32/f64 [N][Co]
 */
#ifndef TRELLIS_SPARSE_ORACLE_H
#define TRELLIS_SPARSE_ORACLE_H
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* build_neighbor_table restated with a hash map: insert rows 0..N-1 in order so a later
 * duplicate overwrites an earlier one, then probe the 27 offsets of every voxel
 * (sparse.cpp:21-39). Returns 0, or -1 if a coordinate lies outside [-2^20, 2^20). */
int orc_neighbor_table_hash(const int32_t* coords, int64_t n, int32_t* nbr);

/* The same table by brute force on a dense occupancy grid over the bounding box
 * (grid cell -> max row index). Independent of any hashing. Returns 0, or -1 when
 * the bounding box exceeds max_cells. */
int orc_neighbor_table_grid(const int32_t* coords, int64_t n, int32_t* nbr, int64_t max_cells);

/* Number of active (voxel, tap) pairs: #{(t,i): nbr[t*N+i] != N}. */
int64_t orc_count_pairs(const int32_t* nbr, int64_t n);

/* Submanifold conv in fp32, following submconv_range (sparse.cpp:64-79): for each tap t
 * the gathered row (the zero row when nbr == N, sparse.cpp:81-85) is multiplied by W_t,
 * the 27 per-tap products are accumulated in tap order, and the bias is added last.
 * All 27 taps are evaluated, absent ones against the zero row, exactly as the reference
 * does. Parallel over output rows with `threads` OpenMP threads (<=0: all). */
void orc_subm_conv_f32(const float* feats, int64_t n, int ci, const int32_t* nbr,
                       const float* weight, const float* bias, int co, float* out,
                       int threads);

/* The same sum evaluated in fp64 over only the active taps: the judge for tolerances. */
void orc_subm_conv_f64(const float* feats, int64_t n, int ci, const int32_t* nbr,
                       const float* weight, const float* bias, int co, double* out,
                       int threads, int zero_pad);

/* orc_subm_conv_f64 for the output rows listed in rows[0..nrows) only; out is [nrows][Co].
 * zero_pad (both forms): absent taps read an exact zero row, not 0 * feats[0]. */
void orc_subm_conv_f64_rows(const float* feats, int64_t n, int ci, const int32_t* nbr,
                            const float* weight, const float* bias, int co, double* out,
                            const int64_t* rows, int64_t nrows, int threads, int zero_pad);

/* Timed CPU baseline: orc_subm_conv_f32 over output rows [r0, r1) only. */
void orc_subm_conv_f32_rows(const float* feats, int64_t n, int ci, const int32_t* nbr,
                            const float* weight, const float* bias, int co, float* out,
                            int64_t r0, int64_t r1, int threads);

/* C2S subdivision index math (sparse.cpp:205-222): parent i, octant o = 0..7 ascending;
 * an octant is kept when mask[o+8i] != 0; child = (2x+(o&1), 2y+((o>>1)&1), 2z+((o>>2)&1));
 * gidx = o + 8i; mstart[i] = first child of parent i, mstart[N] = M.
 * child_coords must hold 8N*3 ints and gidx 8N ints. Returns M. */
int64_t orc_subdivide(const uint8_t* mask, const int32_t* coords, int64_t n,
                      int32_t* child_coords, int32_t* gidx, int32_t* mstart);

#ifdef __cplusplus
}
#endif
#endif
