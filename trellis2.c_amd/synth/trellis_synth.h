/*
 * trellis_synth.h - seeded synthetic workloads for the sparse-voxel path.
 *
 * Deterministic, thread-count independent generators for the benchmark
 * configurations: voxel coordinate sets (sphere / ellipsoid shells / dense and
 * Bernoulli grids) and counter-based N(0, std) and +-1 fills.  Used by the
 * benchmark and the tests to build identical inputs for the GPU path and the
 * CPU oracle.  Not part of the product library.
 */
#ifndef TRELLIS_SYNTH_H
#define TRELLIS_SYNTH_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Coordinates [n][4] (b,x,y,z), raster order (b, then x, y, z ascending), for
 * workload cfg in 1..5 (config 3 returns the R=256 parent shells).  The array
 * is malloc'd; release with ts_free.  Returns 0 on success. */
int ts_make_coords(int cfg, int32_t ** coords_out, int64_t * n_out);

/* Union of ellipsoid shells on an R^3 grid with cell centres at integer+0.5:
 * a cell is in a shell when |rho-1| / |grad rho| <= t/2 with
 * rho = |(p-c)/a|.  Centres ~ U[c_lo,c_hi]^3, semi-axes ~ U[a_lo,a_hi]. */
int ts_shells(int R, int n_shells, double c_lo, double c_hi, double a_lo, double a_hi, double t,
              uint64_t seed, int32_t batch, int32_t ** coords_out, int64_t * n_out);

/* out[i] = std * N(0,1), value i drawn from (seed, stream, i) only. */
void ts_normal(uint64_t seed, uint64_t stream, float std, float * out, int64_t count);
/* out[i] = +1 with probability p, else -1. */
void ts_pm1(uint64_t seed, uint64_t stream, double p, float * out, int64_t count);
/* Uniform [0,1) value i of (seed, stream). */
double ts_uniform(uint64_t seed, uint64_t stream, uint64_t i);

void ts_free(void * p);

#ifdef __cplusplus
}
#endif

#endif
