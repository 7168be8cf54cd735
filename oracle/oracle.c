/*
 * CPU oracle for the sparse submanifold 3x3x3 conv path -- TEST INFRASTRUCTURE ONLY.
 * Declarations and layouts: oracle.h. Reference files are cited per function.
 */
#include "oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

/* ------------------------------------------------------------------------------------ */
/* Neighbour table via a hash map (sparse.cpp:21-39).                                    */
/* ------------------------------------------------------------------------------------ */

/* The reference packs (x,y,z) as ((u64)(u32)x<<40) | ((u64)(u32)y<<20) | (u32)z
 * (sparse.cpp:25). The same packing is used here so that the restatement keys exactly
 * what the reference keys. */
static uint64_t ref_key(int32_t x, int32_t y, int32_t z) {
    return ((uint64_t)(uint32_t)x << 40) | ((uint64_t)(uint32_t)y << 20) | (uint64_t)(uint32_t)z;
}

static uint64_t mix64(uint64_t k) {  /* splitmix64 finaliser */
    k ^= k >> 30; k *= 0xbf58476d1ce4e5b9ULL;
    k ^= k >> 27; k *= 0x94d049bb133111ebULL;
    k ^= k >> 31;
    return k;
}

typedef struct { uint64_t* keys; int32_t* vals; uint8_t* used; uint64_t mask; } omap;

static int omap_init(omap* m, int64_t n) {
    uint64_t cap = 16;
    while (cap < (uint64_t)(2 * n + 1)) cap <<= 1;           /* reserve(2N), sparse.cpp:24 */
    m->keys = (uint64_t*)malloc(cap * sizeof(uint64_t));
    m->vals = (int32_t*)malloc(cap * sizeof(int32_t));
    m->used = (uint8_t*)calloc(cap, 1);
    m->mask = cap - 1;
    return (m->keys && m->vals && m->used) ? 0 : -1;
}
static void omap_free(omap* m) { free(m->keys); free(m->vals); free(m->used); }

/* cmap[key] = i : insert or overwrite (sparse.cpp:26) */
static void omap_set(omap* m, uint64_t key, int32_t v) {
    uint64_t h = mix64(key) & m->mask;
    while (m->used[h] && m->keys[h] != key) h = (h + 1) & m->mask;
    m->used[h] = 1; m->keys[h] = key; m->vals[h] = v;
}
static int omap_find(const omap* m, uint64_t key, int32_t* v) {
    uint64_t h = mix64(key) & m->mask;
    while (m->used[h]) {
        if (m->keys[h] == key) { *v = m->vals[h]; return 1; }
        h = (h + 1) & m->mask;
    }
    return 0;
}

int orc_neighbor_table_hash(const int32_t* coords, int64_t n, int32_t* nbr) {
    const int32_t lim = 1 << 20;
    for (int64_t i = 0; i < 3 * n; ++i)
        if (coords[i] < -lim || coords[i] >= lim) return -1;
    omap m;
    if (omap_init(&m, n) != 0) { omap_free(&m); return -1; }
    for (int64_t i = 0; i < n; ++i)                             /* later rows overwrite */
        omap_set(&m, ref_key(coords[3 * i], coords[3 * i + 1], coords[3 * i + 2]), (int32_t)i);
    for (int64_t i = 0; i < n; ++i) {
        const int32_t x = coords[3 * i], y = coords[3 * i + 1], z = coords[3 * i + 2];
        for (int kd = 0; kd < 3; ++kd)
            for (int kh = 0; kh < 3; ++kh)
                for (int kw = 0; kw < 3; ++kw) {
                    const int t = kd * 9 + kh * 3 + kw;              /* sparse.cpp:33 */
                    int32_t v;
                    const int hit = omap_find(&m, ref_key(x + kd - 1, y + kh - 1, z + kw - 1), &v);
                    nbr[(int64_t)t * n + i] = hit ? v : (int32_t)n;  /* sentinel N, :35 */
                }
    }
    omap_free(&m);
    return 0;
}

/* ------------------------------------------------------------------------------------ */
/* Neighbour table by brute force on a dense grid (independent check).                   */
/* ------------------------------------------------------------------------------------ */
int orc_neighbor_table_grid(const int32_t* coords, int64_t n, int32_t* nbr, int64_t max_cells) {
    if (n == 0) return 0;
    int32_t lo[3], hi[3];
    for (int a = 0; a < 3; ++a) { lo[a] = coords[a]; hi[a] = coords[a]; }
    for (int64_t i = 0; i < n; ++i)
        for (int a = 0; a < 3; ++a) {
            if (coords[3 * i + a] < lo[a]) lo[a] = coords[3 * i + a];
            if (coords[3 * i + a] > hi[a]) hi[a] = coords[3 * i + a];
        }
    /* one cell of margin on each side so every probe lands inside the grid */
    const int64_t dx = (int64_t)hi[0] - lo[0] + 3, dy = (int64_t)hi[1] - lo[1] + 3,
                  dz = (int64_t)hi[2] - lo[2] + 3;
    if (dx * dy * dz > max_cells) return -1;
    int32_t* grid = (int32_t*)malloc((size_t)(dx * dy * dz) * sizeof(int32_t));
    if (!grid) return -1;
    for (int64_t c = 0; c < dx * dy * dz; ++c) grid[c] = -1;
#define CELL(x, y, z) ((((int64_t)(x) - lo[0] + 1) * dy + ((int64_t)(y) - lo[1] + 1)) * dz + ((int64_t)(z) - lo[2] + 1))
    for (int64_t i = 0; i < n; ++i) {
        int64_t c = CELL(coords[3 * i], coords[3 * i + 1], coords[3 * i + 2]);
        if ((int32_t)i > grid[c]) grid[c] = (int32_t)i;   /* duplicate coords: max row wins */
    }
    for (int t = 0; t < 27; ++t) {
        const int ox = t / 9 - 1, oy = (t / 3) % 3 - 1, oz = t % 3 - 1;
        for (int64_t i = 0; i < n; ++i) {
            int32_t v = grid[CELL(coords[3 * i] + ox, coords[3 * i + 1] + oy, coords[3 * i + 2] + oz)];
            nbr[(int64_t)t * n + i] = v < 0 ? (int32_t)n : v;
        }
    }
#undef CELL
    free(grid);
    return 0;
}

int64_t orc_count_pairs(const int32_t* nbr, int64_t n) {
    int64_t p = 0;
    for (int64_t j = 0; j < 27 * n; ++j) p += nbr[j] != (int32_t)n;
    return p;
}

/* ------------------------------------------------------------------------------------ */
/* Submanifold conv (sparse.cpp:61-92).                                                  */
/* ------------------------------------------------------------------------------------ */
static void set_threads(int threads) {
#ifdef _OPENMP
    if (threads > 0) omp_set_num_threads(threads);
    else omp_set_num_threads(omp_get_num_procs());
#else
    (void)threads;
#endif
}

void orc_subm_conv_f32_rows(const float* feats, int64_t n, int ci, const int32_t* nbr,
                            const float* weight, const float* bias, int co, float* out,
                            int64_t r0, int64_t r1, int threads) {
    set_threads(threads);
    /* the sentinel row N = 0 * feats[0] (submconv_pad, sparse.cpp:81-85): +-0 for finite
       values, NaN where feats[0] holds an Inf or a NaN */
    const float* zero_row = NULL;
    float* zbuf = (float*)calloc((size_t)ci, sizeof(float));
    if (n > 0)
        for (int k = 0; k < ci; ++k) zbuf[k] = 0.0f * feats[k];
    zero_row = zbuf;
#pragma omp parallel
    {
        float* acc = (float*)malloc((size_t)co * sizeof(float));
#pragma omp for schedule(static)
        for (int64_t i = r0; i < r1; ++i) {
            for (int t = 0; t < 27; ++t) {
                const int32_t r = nbr[(int64_t)t * n + i];
                const float* g = (r == (int32_t)n) ? zero_row : feats + (int64_t)r * ci;   /* get_rows */
                for (int o = 0; o < co; ++o) {                                              /* mul_mat  */
                    const float* w = weight + ((int64_t)o * 27 + t) * ci;
                    float s = 0.0f;
#pragma omp simd reduction(+ : s)
                    for (int k = 0; k < ci; ++k) s += w[k] * g[k];
                    acc[o] = (t == 0) ? s : acc[o] + s;                                     /* add, tap order */
                }
            }
            float* dst = out + i * co;
            for (int o = 0; o < co; ++o) dst[o] = acc[o] + bias[o];                      /* + bias last */
        }
        free(acc);
    }
    free(zbuf);
}

void orc_subm_conv_f32(const float* feats, int64_t n, int ci, const int32_t* nbr,
                       const float* weight, const float* bias, int co, float* out,
                       int threads) {
    orc_subm_conv_f32_rows(feats, n, ci, nbr, weight, bias, co, out, 0, n, threads);
}

/* Whether the sentinel row 0 * feats[0] holds a NaN (feats[0] has an Inf or a NaN): then every
   absent tap makes the whole output row NaN, as in the reference. */
static int sentinel_nan(const float* feats, int64_t n, int ci) {
    if (n <= 0) return 0;
    for (int k = 0; k < ci; ++k)
        if (!isfinite(feats[k])) return 1;
    return 0;
}

void orc_subm_conv_f64_rows(const float* feats, int64_t n, int ci, const int32_t* nbr,
                            const float* weight, const float* bias, int co, double* out,
                            const int64_t* rows, int64_t nrows, int threads, int zero_pad) {
    set_threads(threads);
    /* zero_pad: the padding row is an exact zero column (the C2S conv2 reads hn, whose column M
       is silu(norm(0)) = 0, sparse.cpp:289-306) instead of 0 * feats[0] */
    const int snan = zero_pad ? 0 : sentinel_nan(feats, n, ci);
#pragma omp parallel for schedule(static)
    for (int64_t j = 0; j < nrows; ++j) {
        const int64_t i = rows[j];
        double* dst = out + j * co;
        for (int o = 0; o < co; ++o) dst[o] = (double)bias[o];
        for (int t = 0; t < 27; ++t) {
            const int32_t r = nbr[(int64_t)t * n + i];
            if (r == (int32_t)n) {   /* 0 * feats[0]: contributes +-0, or NaN */
                if (snan)
                    for (int o = 0; o < co; ++o) dst[o] = NAN;
                continue;
            }
            const float* g = feats + (int64_t)r * ci;
            for (int o = 0; o < co; ++o) {
                const float* w = weight + ((int64_t)o * 27 + t) * ci;
                double s = 0.0;
                for (int k = 0; k < ci; ++k) s += (double)w[k] * (double)g[k];
                dst[o] += s;
            }
        }
    }
}

void orc_subm_conv_f64(const float* feats, int64_t n, int ci, const int32_t* nbr,
                       const float* weight, const float* bias, int co, double* out,
                       int threads, int zero_pad) {
    set_threads(threads);
    const int snan = zero_pad ? 0 : sentinel_nan(feats, n, ci);   /* as in the _rows form */
#pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < n; ++i) {
        double* dst = out + i * co;
        for (int o = 0; o < co; ++o) dst[o] = (double)bias[o];
        for (int t = 0; t < 27; ++t) {
            const int32_t r = nbr[(int64_t)t * n + i];
            if (r == (int32_t)n) {   /* 0 * feats[0]: contributes +-0, or NaN */
                if (snan)
                    for (int o = 0; o < co; ++o) dst[o] = NAN;
                continue;
            }
            const float* g = feats + (int64_t)r * ci;
            for (int o = 0; o < co; ++o) {
                const float* w = weight + ((int64_t)o * 27 + t) * ci;
                double s = 0.0;
                for (int k = 0; k < ci; ++k) s += (double)w[k] * (double)g[k];
                dst[o] += s;
            }
        }
    }
}

/* ------------------------------------------------------------------------------------ */
/* C2S subdivision index math (sparse.cpp:205-222).                                      */
/* ------------------------------------------------------------------------------------ */
int64_t orc_subdivide(const uint8_t* mask, const int32_t* coords, int64_t n,
                      int32_t* child_coords, int32_t* gidx, int32_t* mstart) {
    int64_t m = 0;
    for (int64_t i = 0; i < n; ++i) {
        mstart[i] = (int32_t)m;
        const int32_t x = coords[3 * i], y = coords[3 * i + 1], z = coords[3 * i + 2];
        for (int o = 0; o < 8; ++o) {
            if (mask[o + 8 * i] == 0) continue;
            child_coords[3 * m + 0] = 2 * x + (o & 1);
            child_coords[3 * m + 1] = 2 * y + ((o >> 1) & 1);
            child_coords[3 * m + 2] = 2 * z + ((o >> 2) & 1);
            gidx[m] = (int32_t)(o + 8 * i);
            ++m;
        }
    }
    mstart[n] = (int32_t)m;
    return m;
}
