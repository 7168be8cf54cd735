/* Runs every oracle function on small inputs, for a build with AddressSanitizer and
 * UndefinedBehaviorSanitizer (test infrastructure, like the oracle): the hash table against the
 * grid brute force, the conv in its four forms, the pair count and the subdivision, including
 * the empty set, a lone voxel, duplicates and coordinates at the ends of the range.
 * Exit 0 when every cross-check holds (and nothing was reported by the sanitizers). */
#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "oracle.h"

static unsigned long long g_rng = 88172645463325252ull;
static unsigned rnd(void) {
    g_rng ^= g_rng << 13;
    g_rng ^= g_rng >> 7;
    g_rng ^= g_rng << 17;
    return (unsigned)(g_rng >> 11);
}
static float frnd(void) { return (float)(rnd() % 2001) / 1000.0f - 1.0f; }

static int check_set(const int32_t* coords, int64_t n, int ci, int co) {
    int32_t* a = malloc(sizeof(int32_t) * (size_t)(27 * n + 1));
    int32_t* b = malloc(sizeof(int32_t) * (size_t)(27 * n + 1));
    if (orc_neighbor_table_hash(coords, n, a) != 0) return 1;
    if (orc_neighbor_table_grid(coords, n, b, (int64_t)1 << 24) == 0 && memcmp(a, b, sizeof(int32_t) * 27 * n) != 0)
        return 2;
    const int64_t pairs = orc_count_pairs(a, n);
    if (pairs < n || pairs > 27 * n) return 3;
    float* f = malloc(sizeof(float) * (size_t)(n * ci + 1));
    float* w = malloc(sizeof(float) * (size_t)(co * 27 * ci));
    float* bias = malloc(sizeof(float) * (size_t)co);
    for (int64_t i = 0; i < n * ci; ++i) f[i] = frnd();
    for (int64_t i = 0; i < (int64_t)co * 27 * ci; ++i) w[i] = frnd() / 8;
    for (int i = 0; i < co; ++i) bias[i] = frnd();
    float* o32 = malloc(sizeof(float) * (size_t)(n * co + 1));
    float* r32 = malloc(sizeof(float) * (size_t)(n * co + 1));
    double* o64 = malloc(sizeof(double) * (size_t)(n * co + 1));
    double* r64 = malloc(sizeof(double) * (size_t)(n * co + 1));
    int64_t* rows = malloc(sizeof(int64_t) * (size_t)(n + 1));
    for (int64_t i = 0; i < n; ++i) rows[i] = n - 1 - i;
    int bad = 0;
    for (int zp = 0; zp < 2; ++zp) {
        orc_subm_conv_f32(f, n, ci, a, w, bias, co, o32, 1);
        orc_subm_conv_f32_rows(f, n, ci, a, w, bias, co, r32, 0, n, 1);
        orc_subm_conv_f64(f, n, ci, a, w, bias, co, o64, 1, zp);
        orc_subm_conv_f64_rows(f, n, ci, a, w, bias, co, r64, rows, n, 1, zp);
        for (int64_t i = 0; i < n; ++i)
            for (int c = 0; c < co; ++c) {
                const double x = o64[i * co + c];
                if (r64[(n - 1 - i) * co + c] != x) bad = 4;
                if (o32[i * co + c] != r32[i * co + c]) bad = 5;
                if (fabs(o32[i * co + c] - x) > 1e-4 * (1 + fabs(x))) bad = 6;
            }
    }
    uint8_t* mask = malloc((size_t)(8 * n + 1));
    for (int64_t i = 0; i < 8 * n; ++i) mask[i] = (uint8_t)(rnd() % 3 == 0);
    int32_t* child = malloc(sizeof(int32_t) * (size_t)(24 * n + 1));
    int32_t* gidx = malloc(sizeof(int32_t) * (size_t)(8 * n + 1));
    int32_t* mstart = malloc(sizeof(int32_t) * (size_t)(n + 1));
    const int64_t m = orc_subdivide(mask, coords, n, child, gidx, mstart);
    int64_t want = 0;
    for (int64_t i = 0; i < 8 * n; ++i) want += mask[i];
    if (m != want || mstart[n] != m) bad = 7;
    free(a); free(b); free(f); free(w); free(bias); free(o32); free(r32); free(o64); free(r64); free(rows);
    free(mask); free(child); free(gidx); free(mstart);
    return bad;
}

int main(void) {
    int st = 0;
    /* empty set */
    st |= check_set(NULL, 0, 8, 4) << 0;
    /* a lone voxel at the top of the range, and at the origin */
    const int32_t lone[6] = {(1 << 20) - 3, 5, 0, 0, 0, 0};
    st |= check_set(lone, 1, 8, 4);
    st |= check_set(lone + 3, 1, 4, 8);
    /* random voxels in a 6^3 box with duplicates */
    for (int rep = 0; rep < 3; ++rep) {
        const int64_t n = 300;
        int32_t* c = malloc(sizeof(int32_t) * 3 * n);
        for (int64_t i = 0; i < 3 * n; ++i) c[i] = (int32_t)(rnd() % 6);
        st |= check_set(c, n, 16, 8 + 8 * rep);
        free(c);
    }
    printf(st ? "san_check: FAILED (%d)\n" : "san_check: ok\n", st);
    return st;
}
