/*
 * trellis_oracle.h - CPU oracle for the sparse-voxel convolution path.
 *
 * TEST INFRASTRUCTURE ONLY.  This is a plain-C restatement of the reference
 * CPU backend's algorithm (src/ops/sparse/trellis_sparse_cpu.c) and of the
 * decoder's host subdivide (src/architectures/sparse_unet_decoder/
 * executor.c:108-154).  It is the checker that GPU results are compared
 * against.  Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline
 * leg may load it; the product library never links or calls it.
 *
 * Pinning (what checks each function against something other than itself):
 *   orc_pack_coord4 / orc_hash_u64 / table  - neighbour results are compared
 *       with an O(n^2) brute-force search (orc_neighbors_bruteforce) and with a
 *       numpy sort + searchsorted join; the symmetry nbr[i][k]=j <=> nbr[j][26-k]=i
 *       is checked; the 16-bit wrap is checked on hand-made coordinates.
 *   orc_conv3d_rows - reference test inputs (test_sparse_decoder_backend.c:366-459,
 *       test_trellis.c:1374-1420) against the brute-force conv restated from
 *       test_trellis.c:1051-1093; centre-only weights vs numpy matmul; a dense
 *       block vs torch.nn.functional.conv3d (float64); linearity.
 *   orc_c2s_map - the reference's known-answer vector (test_trellis.c:1325-1374).
 *   orc_c2s_gather - the host channel2spatial known answer (test_trellis.c:1521-1533)
 *       and closed-form numpy indexing.
 *   orc_skip_repeat - closed-form numpy indexing with the ceil-div repeat.
 *   orc_s2c_map / orc_s2c_skip_mean - the reference encoder's known-answer
 *       vector (test_sparse_encoder_backend.c:84-110: coarse coords, parent,
 *       subidx and the skip means it produces with zero conv weights); the map
 *       against numpy unique(axis=0) on random sets; S2C of a C2S map
 *       returns the parents.
 *   orc_fdg_mesh - the reference's known answer (test_trellis.c:581-627:
 *       vertices, face order, the five rejected inputs); quads against a
 *       Python set-based corner search on random voxel sets; vertices
 *       against numpy float64 sigmoid.
 *   orc_s2c_pack - c2s_gather (the reference's inverse index map) of the
 *       packed rows returns the input rows; all other slots are zero.
 *   orc_row_norm / orc_silu / orc_add / orc_linear - torch.nn.functional in float64.
 * Each pin is exercised with a planted mistake (orc_set_mutation) to show the
 * check would fail on a plausible error.
 */
#ifndef TRELLIS_ORACLE_H
#define TRELLIS_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Planted-mistake switch for the oracle self-tests (0 = exact restatement). */
enum {
    ORC_MUT_NONE = 0,
    ORC_MUT_SWAP_KD_KW = 1,      /* offset index k = kw*9 + kh*3 + kd instead of kd*9 + kh*3 + kw */
    ORC_MUT_DROP_BIAS = 2,       /* conv ignores bias */
    ORC_MUT_SUBIDX_BITS = 3,     /* subdivide takes x from bit 2 and z from bit 0 */
    ORC_MUT_REPEAT_FLOOR = 4,    /* skip_repeat uses floor(8*Co/Ci) instead of ceil */
    ORC_MUT_NORM_SAMPLE_VAR = 5, /* row_norm divides the variance by C-1 */
    ORC_MUT_NEIGHBOR_SIGN = 6,   /* neighbour offset uses (1 - kd) instead of (kd - 1) on x */
    ORC_MUT_CROSS_BATCH = 7,     /* neighbour lookup ignores the batch index */
    ORC_MUT_SUBDIV_GE = 8,       /* subdivide keeps logits >= 0 instead of > 0 */
    ORC_MUT_S2C_ORDER = 9,       /* S2C orders coarse voxels z-major (z, y, x, b) instead of (b, x, y, z) */
    ORC_MUT_S2C_CHANNEL = 10,    /* S2C skip mean groups channel-major ((c*8 + s) / g instead of (s*ci + c) / g) */
    ORC_MUT_FDG_SPLIT = 11,      /* mesh quads split on w02 >= w13 instead of w02 > w13 */
    ORC_MUT_FDG_QUAD = 12        /* mesh quad of axis 2 takes corners (0,0,0),(1,0,0),(1,1,0),(0,1,0) */
};
void orc_set_mutation(int mutation);
int orc_get_mutation(void);

/* trellis_sparse_cpu.c:24-31 - key = (b|x|y|z as 16-bit fields) + 1, 0 = empty. */
uint64_t orc_pack_coord4(int32_t b, int32_t x, int32_t y, int32_t z);
/* trellis_sparse_cpu.c:33-40 - splitmix64 finaliser. */
uint64_t orc_hash_u64(uint64_t x);
/* trellis_sparse_cpu.c:42-48 and :297 - table size nextpow2(2n). */
int64_t orc_table_size(int64_t n);

typedef struct orc_rulebook {
    int32_t * coords;  /* copy of [n][4] */
    int64_t n;
    uint64_t * keys;
    int32_t * vals;
    int64_t mask;
} orc_rulebook;

/* trellis_sparse_cpu.c:282-322.  Returns 0 on success, 2 on bad argument, 5 on OOM. */
int orc_rulebook_build(const int32_t * coords, int64_t n, orc_rulebook * rb);
void orc_rulebook_free(orc_rulebook * rb);
/* trellis_sparse_cpu.c:266-280 - row for a coordinate or -1. */
int32_t orc_rulebook_find(const orc_rulebook * rb, int32_t b, int32_t x, int32_t y, int32_t z);

/* The 27 probes of trellis_sparse_cpu.c:346-358 written out as a table:
 * nbr[i*27 + k], k = kd*9 + kh*3 + kw, neighbour (b, x+kd-1, y+kh-1, z+kw-1). */
void orc_neighbors(const orc_rulebook * rb, int32_t * nbr);
/* O(n^2) linear search, the lookup of test_trellis.c:1041-1049 (no hashing, no wrap). */
void orc_neighbors_bruteforce(const int32_t * coords, int64_t n, int32_t * nbr);

/* Canonical pair lists from a neighbour table: offset-major, dst ascending.
 * counts[27] out; src/dst hold sum(counts) entries.  Returns the total. */
int64_t orc_pairs(const int32_t * nbr, int64_t n, int64_t * counts, int32_t * src, int32_t * dst);

/* trellis_sparse_cpu.c:324-373 with the same fp32 operation order (bias first,
 * then per offset in k order a sequential fp32 dot product added to the row).
 * Only rows row_begin, row_begin+row_step, ... < row_end are computed; row j of
 * that sequence is written to out[j*co .. j*co+co). bias may be NULL. */
int orc_conv3d_rows(const orc_rulebook * rb, const float * feats, const float * weight, const float * bias,
                    float * out, int ci, int co, int64_t row_begin, int64_t row_end, int64_t row_step);

/* test_trellis.c:1051-1093 - brute-force submanifold conv, generic kernel and
 * dilation, one accumulator per output starting at the bias. */
void orc_conv3d_bruteforce(const int32_t * coords, const float * feats, const float * weight, const float * bias,
                           float * out, int64_t n, int ci, int co, int kd, int kh, int kw, int dd, int dh, int dw);

/* sparse_unet_decoder/executor.c:108-154 - child s of parent p exists iff
 * logits[p*8+s] > 0; child coord (b, 2x+(s&1), 2y+((s>>1)&1), 2z+((s>>2)&1));
 * parent-major, s ascending.  Arrays are malloc'd; returns 0, 1 (no child),
 * 2 (bad argument) or 5 (OOM). */
int orc_c2s_map(const int32_t * coords, const float * logits, int64_t n, int32_t ** coords_out,
                int32_t ** parent_out, int32_t ** subidx_out, int64_t * m_out);
void orc_free(void * p);

/* sparse_unet_encoder/s2c_host.c:33-120 - coarse voxel (b, x/2, y/2, z/2) of
 * every fine voxel, the distinct coarse voxels in ascending (b, x, y, z)
 * order, parent[f] = coarse row, subidx[f] = (x&1) | (y&1)<<1 | (z&1)<<2.
 * Returns 0, 2 (bad argument or a negative coordinate), 4 (two fine voxels
 * with the same coarse voxel and subidx) or 5 (OOM); arrays are malloc'd. */
int orc_s2c_map(const int32_t * fine_coords, int64_t n, int32_t ** coarse_out, int32_t ** parent_out,
                int32_t ** subidx_out, int64_t * coarse_n_out);
/* sparse_unet_encoder/executor.c:279-286 - packed[parent[f]][subidx[f]*pc + c]
 * = x[f][c] (pc = co/8), zero where a coarse voxel lacks that child. */
void orc_s2c_pack(const float * x, const int32_t * parent, const int32_t * subidx, float * y, int64_t n_fine,
                  int64_t n_coarse, int co);
/* sparse_unet_encoder/executor.c:287-292 - skip[parent[f]][(subidx[f]*ci + c)/g]
 * += x[f][c] / g, g = 8*ci/co, fp32 in fine-row then channel order from 0. */
void orc_s2c_skip_mean(const float * x, const int32_t * parent, const int32_t * subidx, float * y, int64_t n_fine,
                       int64_t n_coarse, int ci, int co);

/* src/ops/mesh/flex_dual_grid.c:166-313 - mesh from FlexiDualGrid decoder
 * logits (channels >= 7).  Vertex i = ((coord + 2 sigmoid(f[a]) - 0.5) / res
 * - 0.5) per axis a; weight softplus(f[6]); for voxel i in row order and axis
 * a = 0, 1, 2 in order, when f[3+a] > 0 and the voxels at the quad's corners
 * base + Q[a][0..3] all exist, two triangles split along the diagonal with
 * the larger weight product ((q0,q1,q2),(q0,q2,q3) if w02 > w13, else
 * (q0,q1,q3),(q3,q1,q2)).  Returns 0, 2 (bad argument) or 4 (batch != 0, a
 * coordinate outside [0, res), a non-finite logit in channels 0..6, or a
 * repeated coordinate); vertices [n][3] and faces [n_faces][3] are malloc'd
 * (faces NULL when there are none). */
int orc_fdg_mesh(const int32_t * coords, const float * feats, int64_t n, int channels, int resolution,
                 float ** vertices_out, int32_t ** faces_out, int64_t * n_faces_out);

/* trellis_sparse_cpu.c:385-409. */
void orc_c2s_gather(const float * x, const int32_t * parent, const int32_t * subidx, float * y, int64_t n_out,
                    int co);
/* trellis_sparse_cpu.c:411-440. */
void orc_skip_repeat(const float * x, const int32_t * parent, const int32_t * subidx, float * y, int64_t n_out,
                     int ci, int co);
/* trellis_sparse_cpu.c:173-232 (silu != 0 applies :226-230 afterwards). */
void orc_row_norm(const float * x, const float * gamma, const float * beta, float * y, int64_t n, int c,
                  float eps, int silu);
/* trellis_sparse_cpu.c:234-244. */
void orc_silu(float * x, size_t count);
/* trellis_sparse_cpu.c:246-264. */
void orc_add(const float * a, const float * b, float * y, size_t count);
/* trellis_sparse_cpu.c:122-171 (silu != 0 applies :165-169 afterwards). */
void orc_linear(const float * x, const float * w, const float * bias, float * y, int64_t n, int ci, int co,
                int silu);

#ifdef __cplusplus
}
#endif

#endif
