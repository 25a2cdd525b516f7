/*
 * trellis_synth.c - seeded synthetic workloads (see trellis_synth.h).
 */
#include "trellis_synth.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

static uint64_t ts_mix(uint64_t v) {
    v = (v ^ (v >> 30)) * 0xbf58476d1ce4e5b9ull;
    v = (v ^ (v >> 27)) * 0x94d049bb133111ebull;
    return v ^ (v >> 31);
}

static uint64_t ts_bits(uint64_t seed, uint64_t stream, uint64_t i) {
    return ts_mix(ts_mix(seed * 0x9e3779b97f4a7c15ull + 0x632be59bd9b4e019ull) ^
                  ts_mix(stream * 0xd1b54a32d192ed03ull + 0x8cb92ba72f3d8dd7ull) ^ (i * 0xa0761d6478bd642full));
}

double ts_uniform(uint64_t seed, uint64_t stream, uint64_t i) {
    return (double) (ts_bits(seed, stream, i) >> 11) * (1.0 / 9007199254740992.0);
}

void ts_normal(uint64_t seed, uint64_t stream, float std, float * out, int64_t count) {
    /* Box-Muller on pair j = i/2: u1 in (0,1], u2 in [0,1). */
#pragma omp parallel for schedule(static)
    for (int64_t j = 0; j < (count + 1) / 2; ++j) {
        const double u1 = 1.0 - ts_uniform(seed, stream, 2 * (uint64_t) j);
        const double u2 = ts_uniform(seed, stream, 2 * (uint64_t) j + 1);
        const double r = sqrt(-2.0 * log(u1));
        const double a = 6.283185307179586 * u2;
        out[2 * j] = (float) (std * r * cos(a));
        if (2 * j + 1 < count) {
            out[2 * j + 1] = (float) (std * r * sin(a));
        }
    }
}

void ts_pm1(uint64_t seed, uint64_t stream, double p, float * out, int64_t count) {
#pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < count; ++i) {
        out[i] = ts_uniform(seed, stream, (uint64_t) i) < p ? 1.0f : -1.0f;
    }
}

void ts_free(void * p) { free(p); }

typedef struct ts_grid {
    int R;
    uint64_t * bits; /* R^3 bits, raster index (x*R + y)*R + z */
} ts_grid;

static int ts_grid_init(ts_grid * g, int R) {
    g->R = R;
    const uint64_t cells = (uint64_t) R * R * R;
    g->bits = (uint64_t *) calloc((size_t) ((cells + 63) / 64), sizeof(uint64_t));
    return g->bits == NULL ? 5 : 0;
}

static void ts_grid_set(ts_grid * g, int x, int y, int z) {
    const uint64_t idx = ((uint64_t) x * g->R + (uint64_t) y) * g->R + (uint64_t) z;
    g->bits[idx >> 6] |= 1ull << (idx & 63);
}

/* Appends the set cells of g in raster order with batch index b. */
static int ts_grid_emit(const ts_grid * g, int32_t b, int32_t ** coords, int64_t * n) {
    const uint64_t cells = (uint64_t) g->R * g->R * g->R;
    const uint64_t words = (cells + 63) / 64;
    int64_t add = 0;
    for (uint64_t w = 0; w < words; ++w) {
        add += __builtin_popcountll(g->bits[w]);
    }
    int32_t * grown = (int32_t *) realloc(*coords, (size_t) (*n + add) * 4u * sizeof(int32_t) + 16u);
    if (grown == NULL) {
        return 5;
    }
    *coords = grown;
    int64_t at = *n;
    const uint64_t R = (uint64_t) g->R;
    for (uint64_t w = 0; w < words; ++w) {
        uint64_t v = g->bits[w];
        while (v != 0) {
            const uint64_t idx = w * 64 + (uint64_t) __builtin_ctzll(v);
            v &= v - 1;
            grown[4 * at + 0] = b;
            grown[4 * at + 1] = (int32_t) (idx / (R * R));
            grown[4 * at + 2] = (int32_t) ((idx / R) % R);
            grown[4 * at + 3] = (int32_t) (idx % R);
            ++at;
        }
    }
    *n = at;
    return 0;
}

/* Marks the cells of one ellipsoid shell. */
static void ts_mark_shell(ts_grid * g, const double c[3], const double a[3], double t) {
    const int R = g->R;
    const double amin = fmin(a[0], fmin(a[1], a[2]));
    /* On the shell |grad rho| >= 1/amax... use the safe radial bound
     * |rho-1| <= (t/2)*|grad rho| <= (t/2)*(rho/amin) to bracket candidates. */
    const double slack = 0.5 * t / amin * 1.5 + 1e-9;
    const double lo = fmax(0.0, 1.0 - slack), hi = 1.0 + slack;
    const int x0 = (int) fmax(0.0, floor(c[0] - a[0] * hi - 1.0));
    const int x1 = (int) fmin((double) (R - 1), ceil(c[0] + a[0] * hi + 1.0));
    const int y0 = (int) fmax(0.0, floor(c[1] - a[1] * hi - 1.0));
    const int y1 = (int) fmin((double) (R - 1), ceil(c[1] + a[1] * hi + 1.0));
    for (int x = x0; x <= x1; ++x) {
        const double qx = (x + 0.5 - c[0]) / a[0];
        for (int y = y0; y <= y1; ++y) {
            const double qy = (y + 0.5 - c[1]) / a[1];
            const double q = qx * qx + qy * qy;
            if (q > hi * hi) {
                continue;
            }
            const double s_hi = sqrt(hi * hi - q);
            const double s_lo = q < lo * lo ? sqrt(lo * lo - q) : 0.0;
            /* z candidates: c_z +- a_z * [s_lo, s_hi], widened by one cell. */
            for (int side = 0; side < 2; ++side) {
                const double zlo = side == 0 ? c[2] - a[2] * s_hi - 1.0 : c[2] + a[2] * s_lo - 1.0;
                const double zhi = side == 0 ? c[2] - a[2] * s_lo + 1.0 : c[2] + a[2] * s_hi + 1.0;
                const int za = (int) fmax(0.0, floor(zlo));
                const int zb = (int) fmin((double) (R - 1), ceil(zhi));
                for (int z = za; z <= zb; ++z) {
                    const double d[3] = {x + 0.5 - c[0], y + 0.5 - c[1], z + 0.5 - c[2]};
                    const double u[3] = {d[0] / a[0], d[1] / a[1], d[2] / a[2]};
                    const double rho = sqrt(u[0] * u[0] + u[1] * u[1] + u[2] * u[2]);
                    if (rho <= 0.0) {
                        continue;
                    }
                    const double gx = u[0] / a[0], gy = u[1] / a[1], gz = u[2] / a[2];
                    const double grad = sqrt(gx * gx + gy * gy + gz * gz) / rho;
                    if (fabs(rho - 1.0) <= 0.5 * t * grad) {
                        ts_grid_set(g, x, y, z);
                    }
                }
            }
        }
    }
}

int ts_shells(int R, int n_shells, double c_lo, double c_hi, double a_lo, double a_hi, double t,
              uint64_t seed, int32_t batch, int32_t ** coords_out, int64_t * n_out) {
    if (coords_out == NULL || n_out == NULL || R <= 0 || n_shells <= 0) {
        return 2;
    }
    ts_grid g;
    if (ts_grid_init(&g, R) != 0) {
        return 5;
    }
    uint64_t draw = 0;
    for (int s = 0; s < n_shells; ++s) {
        double c[3], a[3];
        for (int i = 0; i < 3; ++i) c[i] = c_lo + (c_hi - c_lo) * ts_uniform(seed, 0, draw++);
        for (int i = 0; i < 3; ++i) a[i] = a_lo + (a_hi - a_lo) * ts_uniform(seed, 0, draw++);
        ts_mark_shell(&g, c, a, t);
    }
    *coords_out = NULL;
    *n_out = 0;
    const int rc = ts_grid_emit(&g, batch, coords_out, n_out);
    free(g.bits);
    return rc;
}

static int ts_sphere_config1(int32_t ** coords, int64_t * n) {
    /* R=64, cells whose centre lies within 1.0 of the sphere |p-32| = 24. */
    ts_grid g;
    if (ts_grid_init(&g, 64) != 0) {
        return 5;
    }
    for (int x = 0; x < 64; ++x)
        for (int y = 0; y < 64; ++y)
            for (int z = 0; z < 64; ++z) {
                const double dx = x + 0.5 - 32.0, dy = y + 0.5 - 32.0, dz = z + 0.5 - 32.0;
                if (fabs(sqrt(dx * dx + dy * dy + dz * dz) - 24.0) <= 1.0) {
                    ts_grid_set(&g, x, y, z);
                }
            }
    *coords = NULL;
    *n = 0;
    const int rc = ts_grid_emit(&g, 0, coords, n);
    free(g.bits);
    return rc;
}

static int ts_blocks_config5(int32_t ** coords, int64_t * n) {
    /* b=0,1: dense 32^3; b=2,3: 64^3 cells kept with probability 0.5. */
    *coords = NULL;
    *n = 0;
    for (int b = 0; b < 4; ++b) {
        const int R = b < 2 ? 32 : 64;
        ts_grid g;
        if (ts_grid_init(&g, R) != 0) {
            return 5;
        }
        uint64_t i = 0;
        for (int x = 0; x < R; ++x)
            for (int y = 0; y < R; ++y)
                for (int z = 0; z < R; ++z, ++i) {
                    if (b < 2 || ts_uniform(5, 10 + (uint64_t) b, i) < 0.5) {
                        ts_grid_set(&g, x, y, z);
                    }
                }
        const int rc = ts_grid_emit(&g, b, coords, n);
        free(g.bits);
        if (rc != 0) {
            return rc;
        }
    }
    return 0;
}

int ts_make_coords(int cfg, int32_t ** coords_out, int64_t * n_out) {
    if (coords_out == NULL || n_out == NULL) {
        return 2;
    }
    switch (cfg) {
        case 1:
            return ts_sphere_config1(coords_out, n_out);
        case 2:
            /* 12 shells from seed 2 put N at ~0.42M (stated size ~0.4M). */
            return ts_shells(256, 12, 48.0, 208.0, 16.0, 64.0, 1.5, 2, 0, coords_out, n_out);
        case 3:
            /* 13 shells from seed 3 put the parents at ~0.32M (stated ~0.3M, ~1.2M children). */
            return ts_shells(256, 13, 48.0, 208.0, 16.0, 64.0, 1.5, 3, 0, coords_out, n_out);
        case 4:
            return ts_shells(1024, 4, 400.0, 623.0, 128.0, 400.0, 1.0, 4, 0, coords_out, n_out);
        case 5:
            return ts_blocks_config5(coords_out, n_out);
        default:
            return 2;
    }
}
