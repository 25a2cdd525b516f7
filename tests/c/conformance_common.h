/*
 * conformance_common.h - helpers shared by the compiled C callers of
 * include/trellis_sparse_hip.h (decoder_conformance.c, encoder_conformance.c):
 * status checks, seeded weights, the ConvNeXt block through backend->ops and
 * on the CPU oracle (the same slot order in both U-Nets:
 * sparse_unet_decoder/executor.c:176-255, sparse_unet_encoder/executor.c:27-134),
 * the storage rounding the oracle mirrors, and the tolerance comparison.
 * Test code only: every function is static inline so each caller takes what
 * it needs.
 */
#ifndef TSH_CONFORMANCE_COMMON_H
#define TSH_CONFORMANCE_COMMON_H

#include "trellis_sparse_hip.h"
#include "trellis_oracle.h"

#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#define CHECK(expr)                                                                      \
    do {                                                                                 \
        if (!(expr)) {                                                                   \
            fprintf(stderr, "CHECK failed at %s:%d: %s\n", __FILE__, __LINE__, #expr); \
            return 0;                                                                    \
        }                                                                                \
    } while (0)
#define CHECK_OK(be, expr)                                                                         \
    do {                                                                                           \
        const trellis_status st_ = (expr);                                                         \
        if (st_ != TRELLIS_STATUS_OK) {                                                            \
            fprintf(stderr, "%s:%d: %s -> status %d (%s)\n", __FILE__, __LINE__, #expr, (int) st_, \
                    trellis_sparse_hip_last_error(be));                                            \
            return 0;                                                                              \
        }                                                                                          \
    } while (0)

static inline float * fvec(size_t n) {
    float * p = (float *) calloc(n ? n : 1, sizeof(float));
    if (p == NULL) {
        fprintf(stderr, "out of host memory\n");
        exit(1);
    }
    return p;
}

static inline int32_t * ivec(size_t n) {
    int32_t * p = (int32_t *) calloc(n ? n : 1, sizeof(int32_t));
    if (p == NULL) {
        fprintf(stderr, "out of host memory\n");
        exit(1);
    }
    return p;
}

/* Seeded uniform draws in [-a, a] (xorshift64*). */
static uint64_t g_rng = 0x9e3779b97f4a7c15ull;
static inline float urand(float a) {
    g_rng ^= g_rng >> 12;
    g_rng ^= g_rng << 25;
    g_rng ^= g_rng >> 27;
    const uint64_t r = g_rng * 0x2545f4914f6cdd1dull;
    return a * ((float) (r >> 40) / (float) (1u << 23) - 1.0f);
}
static inline void fill_rand(float * w, size_t n, float a) {
    for (size_t i = 0; i < n; ++i) w[i] = urand(a);
}

/* Storage type of the backend under test (TRELLIS_SPARSE_HIP_F32 / _BF16). */
static int g_dtype = TRELLIS_SPARSE_HIP_F32;

/* Storage rounding of the backend's buffers: bf16 round-to-nearest-even,
 * with a positive value that would round to +0 kept as the smallest positive
 * bf16 (the backend's sign-preserving store on uploads and linear outputs;
 * the other slots' outputs never hit that case in these models). */
static inline void round_store(float * v, size_t n) {
    if (g_dtype != TRELLIS_SPARSE_HIP_BF16) return;
    for (size_t i = 0; i < n; ++i) {
        uint32_t u;
        memcpy(&u, &v[i], 4);
        const int pos = v[i] > 0.0f;
        u += 0x7fffu + ((u >> 16) & 1u);
        u &= 0xffff0000u;
        if (pos && u == 0) u = 0x10000u;
        memcpy(&v[i], &u, 4);
    }
}

/* ------------------------------------------------------ ConvNeXt block */

typedef struct block_w {
    int c;
    float *conv_w, *conv_b, *norm_g, *norm_b, *mlp0_w, *mlp0_b, *mlp2_w, *mlp2_b;
} block_w;

static inline void block_alloc(block_w * b, int c) {
    b->c = c;
    b->conv_w = fvec((size_t) c * 27 * c);
    b->conv_b = fvec(c);
    b->norm_g = fvec(c);
    b->norm_b = fvec(c);
    b->mlp0_w = fvec((size_t) 4 * c * c);
    b->mlp0_b = fvec(4 * c);
    b->mlp2_w = fvec((size_t) c * 4 * c);
    b->mlp2_b = fvec(c);
}

static inline void block_rand(block_w * b, int c) {
    block_alloc(b, c);
    fill_rand(b->conv_w, (size_t) c * 27 * c, 1.7f / sqrtf(27.0f * c));
    fill_rand(b->conv_b, c, 0.05f);
    for (int i = 0; i < c; ++i) b->norm_g[i] = 1.0f + urand(0.1f), b->norm_b[i] = urand(0.1f);
    fill_rand(b->mlp0_w, (size_t) 4 * c * c, 1.7f / sqrtf((float) c));
    fill_rand(b->mlp0_b, 4 * c, 0.05f);
    fill_rand(b->mlp2_w, (size_t) c * 4 * c, 1.7f / sqrtf(4.0f * c));
    fill_rand(b->mlp2_b, c, 0.05f);
}

/* h <- h + mlp2(silu(mlp0(LN(conv(h))))) through the vtable; frees the old h. */
static inline int convnext_dev(trellis_sparse_backend * be, const block_w * b, const trellis_sparse_rulebook * rb,
                               trellis_sparse_buffer ** h, int64_t n) {
    const trellis_sparse_backend_ops * ops = be->ops;
    const int c = b->c;
    trellis_sparse_buffer *conv = NULL, *norm = NULL, *mlp1 = NULL, *mlp2 = NULL, *out = NULL;
    CHECK_OK(be, ops->alloc_f32(be, (size_t) n * c, &conv));
    CHECK_OK(be, ops->sparse_conv3d(be, rb, *h, b->conv_w, b->conv_b, conv, n, c, c));
    CHECK_OK(be, ops->alloc_f32(be, (size_t) n * c, &norm));
    CHECK_OK(be, ops->row_norm(be, conv, b->norm_g, b->norm_b, norm, n, c, 1e-6f));
    ops->free_buffer(be, conv);
    CHECK_OK(be, ops->alloc_f32(be, (size_t) n * c * 4, &mlp1));
    CHECK_OK(be, ops->linear_silu(be, norm, b->mlp0_w, b->mlp0_b, mlp1, n, c, 4 * c));
    ops->free_buffer(be, norm);
    CHECK_OK(be, ops->alloc_f32(be, (size_t) n * c, &mlp2));
    CHECK_OK(be, ops->linear(be, mlp1, b->mlp2_w, b->mlp2_b, mlp2, n, 4 * c, c));
    ops->free_buffer(be, mlp1);
    CHECK_OK(be, ops->alloc_f32(be, (size_t) n * c, &out));
    CHECK_OK(be, ops->add(be, *h, mlp2, out, (size_t) n * c));
    ops->free_buffer(be, mlp2);
    ops->free_buffer(be, *h);
    *h = out;
    return 1;
}

/* The oracle's submanifold conv on its own rulebook of coords, rounded. */
static inline int conv_orc(const int32_t * coords, int64_t n, const float * x, const float * w, const float * b,
                           float * y, int ci, int co) {
    orc_rulebook rb;
    CHECK(orc_rulebook_build(coords, n, &rb) == 0);
    CHECK(orc_conv3d_rows(&rb, x, w, b, y, ci, co, 0, n, 1) == 0);
    orc_rulebook_free(&rb);
    round_store(y, (size_t) n * co);
    return 1;
}

static inline int convnext_orc(const block_w * b, const int32_t * coords, int64_t n, float ** hp) {
    const int c = b->c;
    float * h = *hp;
    float * conv = fvec((size_t) n * c);
    CHECK(conv_orc(coords, n, h, b->conv_w, b->conv_b, conv, c, c));
    float * norm = fvec((size_t) n * c);
    orc_row_norm(conv, b->norm_g, b->norm_b, norm, n, c, 1e-6f, 0);
    round_store(norm, (size_t) n * c);
    float * mlp1 = fvec((size_t) n * c * 4);
    orc_linear(norm, b->mlp0_w, b->mlp0_b, mlp1, n, c, 4 * c, 1);
    round_store(mlp1, (size_t) n * c * 4);
    float * mlp2 = fvec((size_t) n * c);
    orc_linear(mlp1, b->mlp2_w, b->mlp2_b, mlp2, n, 4 * c, c, 0);
    round_store(mlp2, (size_t) n * c);
    float * out = fvec((size_t) n * c);
    orc_add(h, mlp2, out, (size_t) n * c);
    round_store(out, (size_t) n * c);
    free(conv), free(norm), free(mlp1), free(mlp2), free(h);
    *hp = out;
    return 1;
}

/* ------------------------------------------------------------ comparison */

/* |got - exp| <= tol * max(1, |got|, |exp|) for every value. */
static inline int close_all(const char * what, const float * got, const float * exp, size_t n, float tol) {
    double worst = 0.0;
    size_t bad = 0;
    for (size_t i = 0; i < n; ++i) {
        const double d = fabs((double) got[i] - (double) exp[i]);
        const double s = fmax(1.0, fmax(fabs((double) got[i]), fabs((double) exp[i])));
        const double r = d / s;
        if (!(r <= tol)) {
            if (bad < 5) fprintf(stderr, "%s[%zu]: got %g expected %g\n", what, i, got[i], exp[i]);
            ++bad;
        }
        if (r > worst) worst = r;
    }
    printf("%s: %zu values, max rel err %.3e (tol %.1e)\n", what, n, worst, tol);
    return bad == 0;
}

/* Cells of a grid^3 box whose centre lies within 0.75 of a sphere of the
 * given radius about the box centre, batch 0, in (x, y, z) order. */
static inline int32_t * shell_coords(int grid, double radius, int64_t * n_out) {
    int32_t * c = ivec((size_t) grid * grid * grid * 4);
    int64_t n = 0;
    const double mid = 0.5 * grid;
    for (int x = 0; x < grid; ++x)
        for (int y = 0; y < grid; ++y)
            for (int z = 0; z < grid; ++z) {
                const double dx = x + 0.5 - mid, dy = y + 0.5 - mid, dz = z + 0.5 - mid;
                if (fabs(sqrt(dx * dx + dy * dy + dz * dz) - radius) <= 0.75) {
                    c[4 * n] = 0, c[4 * n + 1] = x, c[4 * n + 2] = y, c[4 * n + 3] = z;
                    ++n;
                }
            }
    *n_out = n;
    return c;
}

#endif
