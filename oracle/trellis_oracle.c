/*
 * trellis_oracle.c - CPU oracle (test infrastructure only; see trellis_oracle.h).
 *
 * Every function restates the reference algorithm named in its comment.  It
 * is compiled with -ffp-contract=off so that fp32 expressions round exactly as
 * written, in the reference's operation order.
 */
#include "trellis_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

static int g_mutation = ORC_MUT_NONE;

void orc_set_mutation(int mutation) { g_mutation = mutation; }
int orc_get_mutation(void) { return g_mutation; }

uint64_t orc_pack_coord4(int32_t b, int32_t x, int32_t y, int32_t z) {
    /* Four 16-bit fields, batch highest; +1 keeps 0 free as the empty marker. */
    const uint64_t fb = (uint64_t) ((uint32_t) b & 0xffffu);
    const uint64_t fx = (uint64_t) ((uint32_t) x & 0xffffu);
    const uint64_t fy = (uint64_t) ((uint32_t) y & 0xffffu);
    const uint64_t fz = (uint64_t) ((uint32_t) z & 0xffffu);
    return ((fb << 48) | (fx << 32) | (fy << 16) | fz) + 1ull;
}

uint64_t orc_hash_u64(uint64_t v) {
    v = (v ^ (v >> 30)) * 0xbf58476d1ce4e5b9ull;
    v = (v ^ (v >> 27)) * 0x94d049bb133111ebull;
    return v ^ (v >> 31);
}

int64_t orc_table_size(int64_t n) {
    const int64_t want = 2 * n;
    int64_t size = 1;
    while (size < want && size < INT64_MAX / 2) {
        size *= 2;
    }
    return size;
}

int orc_rulebook_build(const int32_t * coords, int64_t n, orc_rulebook * rb) {
    if (coords == NULL || n <= 0 || rb == NULL) {
        return 2;
    }
    memset(rb, 0, sizeof(*rb));
    const int64_t slots = orc_table_size(n);
    rb->coords = (int32_t *) malloc((size_t) n * 4u * sizeof(int32_t));
    rb->keys = (uint64_t *) calloc((size_t) slots, sizeof(uint64_t));
    rb->vals = (int32_t *) malloc((size_t) slots * sizeof(int32_t));
    if (rb->coords == NULL || rb->keys == NULL || rb->vals == NULL) {
        orc_rulebook_free(rb);
        return 5;
    }
    memcpy(rb->coords, coords, (size_t) n * 4u * sizeof(int32_t));
    rb->n = n;
    rb->mask = slots - 1;
    for (int64_t i = 0; i < n; ++i) {
        const int32_t * c = coords + 4 * i;
        const uint64_t key = orc_pack_coord4(c[0], c[1], c[2], c[3]);
        uint64_t s = orc_hash_u64(key) & (uint64_t) rb->mask;
        /* Linear probe to the key's slot or the first empty one; a repeated
         * key overwrites the row, so the last duplicate wins. */
        for (;;) {
            const uint64_t here = rb->keys[s];
            if (here == 0 || here == key) {
                break;
            }
            s = (s + 1u) & (uint64_t) rb->mask;
        }
        rb->keys[s] = key;
        rb->vals[s] = (int32_t) i;
    }
    return 0;
}

void orc_rulebook_free(orc_rulebook * rb) {
    if (rb == NULL) {
        return;
    }
    free(rb->coords);
    free(rb->keys);
    free(rb->vals);
    memset(rb, 0, sizeof(*rb));
}

int32_t orc_rulebook_find(const orc_rulebook * rb, int32_t b, int32_t x, int32_t y, int32_t z) {
    const uint64_t key = orc_pack_coord4(b, x, y, z);
    uint64_t s = orc_hash_u64(key) & (uint64_t) rb->mask;
    for (int64_t step = 0; step <= rb->mask; ++step) {
        const uint64_t here = rb->keys[s];
        if (here == key) {
            return rb->vals[s];
        }
        if (here == 0) {
            return -1;
        }
        s = (s + 1u) & (uint64_t) rb->mask;
    }
    return -1;
}

/* Offset index of (kd, kh, kw) with the planted axis swap available. */
static int orc_offset_index(int kd, int kh, int kw) {
    if (g_mutation == ORC_MUT_SWAP_KD_KW) {
        return kw * 9 + kh * 3 + kd;
    }
    return kd * 9 + kh * 3 + kw;
}

static int32_t orc_probe_neighbor(const orc_rulebook * rb, const int32_t * c, int kd, int kh, int kw) {
    const int dx = g_mutation == ORC_MUT_NEIGHBOR_SIGN ? 1 - kd : kd - 1;
    const int32_t b = g_mutation == ORC_MUT_CROSS_BATCH ? 0 : c[0];
    if (g_mutation == ORC_MUT_CROSS_BATCH) {
        /* Planted mistake: look the neighbour up in every batch, take the first hit. */
        for (int32_t bb = 0; bb < 4; ++bb) {
            const int32_t r = orc_rulebook_find(rb, bb, c[1] + dx, c[2] + kh - 1, c[3] + kw - 1);
            if (r >= 0) {
                return r;
            }
        }
        return -1;
    }
    return orc_rulebook_find(rb, b, c[1] + dx, c[2] + kh - 1, c[3] + kw - 1);
}

void orc_neighbors(const orc_rulebook * rb, int32_t * nbr) {
    for (int64_t i = 0; i < rb->n; ++i) {
        const int32_t * c = rb->coords + 4 * i;
        for (int kd = 0; kd < 3; ++kd) {
            for (int kh = 0; kh < 3; ++kh) {
                for (int kw = 0; kw < 3; ++kw) {
                    nbr[i * 27 + orc_offset_index(kd, kh, kw)] = orc_probe_neighbor(rb, c, kd, kh, kw);
                }
            }
        }
    }
}

void orc_neighbors_bruteforce(const int32_t * coords, int64_t n, int32_t * nbr) {
    /* Last match wins, matching the table's duplicate rule. */
    for (int64_t i = 0; i < n; ++i) {
        const int32_t * c = coords + 4 * i;
        for (int k = 0; k < 27; ++k) {
            const int32_t tx = c[1] + k / 9 - 1;
            const int32_t ty = c[2] + (k / 3) % 3 - 1;
            const int32_t tz = c[3] + k % 3 - 1;
            int32_t found = -1;
            for (int64_t j = 0; j < n; ++j) {
                const int32_t * d = coords + 4 * j;
                if (d[0] == c[0] && d[1] == tx && d[2] == ty && d[3] == tz) {
                    found = (int32_t) j;
                }
            }
            nbr[i * 27 + k] = found;
        }
    }
}

int64_t orc_pairs(const int32_t * nbr, int64_t n, int64_t * counts, int32_t * src, int32_t * dst) {
    int64_t total = 0;
    for (int k = 0; k < 27; ++k) {
        int64_t c = 0;
        for (int64_t i = 0; i < n; ++i) {
            const int32_t s = nbr[i * 27 + k];
            if (s >= 0) {
                if (src != NULL) src[total + c] = s;
                if (dst != NULL) dst[total + c] = (int32_t) i;
                ++c;
            }
        }
        counts[k] = c;
        total += c;
    }
    return total;
}

int orc_conv3d_rows(const orc_rulebook * rb, const float * feats, const float * weight, const float * bias,
                    float * out, int ci, int co, int64_t row_begin, int64_t row_end, int64_t row_step) {
    if (rb == NULL || feats == NULL || weight == NULL || out == NULL || ci <= 0 || co <= 0 || row_step <= 0 ||
        row_begin < 0 || row_end > rb->n) {
        return 2;
    }
    const int use_bias = bias != NULL && g_mutation != ORC_MUT_DROP_BIAS;
    int64_t j = 0;
    for (int64_t row = row_begin; row < row_end; row += row_step, ++j) {
        float * y = out + j * (int64_t) co;
        for (int o = 0; o < co; ++o) {
            y[o] = use_bias ? bias[o] : 0.0f;
        }
        const int32_t * c = rb->coords + 4 * row;
        for (int kd = 0; kd < 3; ++kd) {
            for (int kh = 0; kh < 3; ++kh) {
                for (int kw = 0; kw < 3; ++kw) {
                    const int32_t s = orc_probe_neighbor(rb, c, kd, kh, kw);
                    if (s < 0) {
                        continue;
                    }
                    const int k = orc_offset_index(kd, kh, kw);
                    const float * xr = feats + (int64_t) s * ci;
                    for (int o = 0; o < co; ++o) {
                        const float * wr = weight + ((int64_t) o * 27 + k) * ci;
                        float part = 0.0f;
                        for (int i = 0; i < ci; ++i) {
                            part += xr[i] * wr[i];
                        }
                        y[o] += part;
                    }
                }
            }
        }
    }
    return 0;
}

void orc_conv3d_bruteforce(const int32_t * coords, const float * feats, const float * weight, const float * bias,
                           float * out, int64_t n, int ci, int co, int kd, int kh, int kw, int dd, int dh, int dw) {
    const int hd = kd / 2, hh = kh / 2, hw = kw / 2;
    for (int64_t row = 0; row < n; ++row) {
        const int32_t * c = coords + 4 * row;
        for (int o = 0; o < co; ++o) {
            float acc = bias == NULL ? 0.0f : bias[o];
            for (int a = 0; a < kd; ++a) {
                for (int b = 0; b < kh; ++b) {
                    for (int d = 0; d < kw; ++d) {
                        const int32_t tx = c[1] + (a - hd) * dd;
                        const int32_t ty = c[2] + (b - hh) * dh;
                        const int32_t tz = c[3] + (d - hw) * dw;
                        int64_t src = -1;
                        for (int64_t j = 0; j < n && src < 0; ++j) {
                            const int32_t * e = coords + 4 * j;
                            if (e[0] == c[0] && e[1] == tx && e[2] == ty && e[3] == tz) {
                                src = j;
                            }
                        }
                        if (src < 0) {
                            continue;
                        }
                        const float * wr = weight + ((((int64_t) o * kd + a) * kh + b) * kw + d) * ci;
                        const float * xr = feats + src * ci;
                        for (int i = 0; i < ci; ++i) {
                            acc += xr[i] * wr[i];
                        }
                    }
                }
            }
            out[row * co + o] = acc;
        }
    }
}

int orc_c2s_map(const int32_t * coords, const float * logits, int64_t n, int32_t ** coords_out,
                int32_t ** parent_out, int32_t ** subidx_out, int64_t * m_out) {
    if (coords == NULL || logits == NULL || n <= 0 || coords_out == NULL || parent_out == NULL ||
        subidx_out == NULL || m_out == NULL) {
        return 2;
    }
    *coords_out = NULL;
    *parent_out = NULL;
    *subidx_out = NULL;
    *m_out = 0;
    const int keep_ge = g_mutation == ORC_MUT_SUBDIV_GE;
    int64_t m = 0;
    for (int64_t i = 0; i < n * 8; ++i) {
        if (keep_ge ? logits[i] >= 0.0f : logits[i] > 0.0f) {
            ++m;
        }
    }
    if (m == 0) {
        return 1;
    }
    int32_t * oc = (int32_t *) malloc((size_t) m * 4u * sizeof(int32_t));
    int32_t * op = (int32_t *) malloc((size_t) m * sizeof(int32_t));
    int32_t * os = (int32_t *) malloc((size_t) m * sizeof(int32_t));
    if (oc == NULL || op == NULL || os == NULL) {
        free(oc);
        free(op);
        free(os);
        return 5;
    }
    int64_t w = 0;
    for (int64_t p = 0; p < n; ++p) {
        const int32_t * c = coords + 4 * p;
        for (int s = 0; s < 8; ++s) {
            const float v = logits[p * 8 + s];
            if (!(keep_ge ? v >= 0.0f : v > 0.0f)) {
                continue;
            }
            int bx = s & 1, bz = (s >> 2) & 1;
            if (g_mutation == ORC_MUT_SUBIDX_BITS) {
                bx = (s >> 2) & 1;
                bz = s & 1;
            }
            oc[4 * w + 0] = c[0];
            oc[4 * w + 1] = 2 * c[1] + bx;
            oc[4 * w + 2] = 2 * c[2] + ((s >> 1) & 1);
            oc[4 * w + 3] = 2 * c[3] + bz;
            op[w] = (int32_t) p;
            os[w] = s;
            ++w;
        }
    }
    *coords_out = oc;
    *parent_out = op;
    *subidx_out = os;
    *m_out = m;
    return 0;
}

void orc_free(void * p) { free(p); }

/* Sort record: the coarse voxel as four non-negative int32 fields, then the
 * fine row (which makes the order total, so qsort's instability is moot). */
typedef struct orc_s2c_rec {
    int32_t key[4];
    int32_t row;
    int32_t sub;
} orc_s2c_rec;

static int orc_s2c_cmp(const void * pa, const void * pb) {
    const orc_s2c_rec * a = (const orc_s2c_rec *) pa;
    const orc_s2c_rec * b = (const orc_s2c_rec *) pb;
    static const int lex[4] = {0, 1, 2, 3};
    static const int zyxb[4] = {3, 2, 1, 0};
    const int * ord = g_mutation == ORC_MUT_S2C_ORDER ? zyxb : lex;
    for (int i = 0; i < 4; ++i) {
        const int32_t u = a->key[ord[i]], v = b->key[ord[i]];
        if (u != v) return u < v ? -1 : 1;
    }
    return a->row < b->row ? -1 : (a->row > b->row ? 1 : 0);
}

static int orc_s2c_same(const orc_s2c_rec * a, const orc_s2c_rec * b) {
    return memcmp(a->key, b->key, sizeof(a->key)) == 0;
}

int orc_s2c_map(const int32_t * fine_coords, int64_t n, int32_t ** coarse_out, int32_t ** parent_out,
                int32_t ** subidx_out, int64_t * coarse_n_out) {
    if (fine_coords == NULL || coarse_out == NULL || parent_out == NULL || subidx_out == NULL ||
        coarse_n_out == NULL || n <= 0 || n > INT32_MAX) {
        return 2;
    }
    *coarse_out = NULL;
    *parent_out = NULL;
    *subidx_out = NULL;
    *coarse_n_out = 0;
    orc_s2c_rec * rec = (orc_s2c_rec *) malloc((size_t) n * sizeof(orc_s2c_rec));
    int32_t * parent = (int32_t *) malloc((size_t) n * sizeof(int32_t));
    int32_t * subidx = (int32_t *) malloc((size_t) n * sizeof(int32_t));
    int32_t * coarse = NULL;
    int rc = 0;
    if (rec == NULL || parent == NULL || subidx == NULL) {
        rc = 5;
    }
    for (int64_t f = 0; rc == 0 && f < n; ++f) {
        const int32_t * c = fine_coords + 4 * f;
        if (c[0] < 0 || c[1] < 0 || c[2] < 0 || c[3] < 0) {
            rc = 2;
            break;
        }
        rec[f].key[0] = c[0];
        for (int a = 1; a < 4; ++a) rec[f].key[a] = c[a] / 2;
        rec[f].row = (int32_t) f;
        rec[f].sub = (c[1] & 1) | ((c[2] & 1) << 1) | ((c[3] & 1) << 2);
    }
    int64_t m = 0;
    if (rc == 0) {
        qsort(rec, (size_t) n, sizeof(orc_s2c_rec), orc_s2c_cmp);
        for (int64_t i = 0; i < n; ++i) {
            const int head = i == 0 || !orc_s2c_same(&rec[i - 1], &rec[i]);
            if (!head && rec[i - 1].sub == rec[i].sub) {
                rc = 4;  /* the same fine voxel twice */
                break;
            }
            m += head;
        }
    }
    if (rc == 0) {
        coarse = (int32_t *) malloc((size_t) m * 4u * sizeof(int32_t));
        if (coarse == NULL) rc = 5;
    }
    if (rc == 0) {
        int64_t row = -1;
        for (int64_t i = 0; i < n; ++i) {
            if (i == 0 || !orc_s2c_same(&rec[i - 1], &rec[i])) {
                ++row;
                memcpy(coarse + 4 * row, rec[i].key, 4 * sizeof(int32_t));
            }
            parent[rec[i].row] = (int32_t) row;
            subidx[rec[i].row] = rec[i].sub;
        }
    }
    free(rec);
    if (rc != 0) {
        free(parent);
        free(subidx);
        free(coarse);
        return rc;
    }
    *coarse_out = coarse;
    *parent_out = parent;
    *subidx_out = subidx;
    *coarse_n_out = m;
    return 0;
}

/* ---- FlexiDualGrid mesh (flex_dual_grid.c:166-313) ---------------------- */
static float orc_fdg_sigmoid(float v) {
    /* Split at 0 so that exp never overflows (flex_dual_grid.c:112-119). */
    if (v >= 0.0f) return 1.0f / (1.0f + expf(-v));
    const float e = expf(v);
    return e / (1.0f + e);
}

static float orc_fdg_softplus(float v) {
    if (v > 20.0f) return v;
    if (v < -20.0f) return expf(v);
    return log1pf(expf(v));
}

/* Voxel lookup by binary search over (x, y, z) keys sorted with their rows. */
typedef struct orc_fdg_key {
    int64_t key;
    int32_t row;
} orc_fdg_key;

static int orc_fdg_key_cmp(const void * a, const void * b) {
    const int64_t u = ((const orc_fdg_key *) a)->key, v = ((const orc_fdg_key *) b)->key;
    return u < v ? -1 : (u > v ? 1 : 0);
}

static int32_t orc_fdg_find(const orc_fdg_key * keys, int64_t n, int64_t res, int64_t x, int64_t y, int64_t z) {
    if (x < 0 || y < 0 || z < 0 || x >= res || y >= res || z >= res) return -1;
    const int64_t want = (x * res + y) * res + z;
    int64_t lo = 0, hi = n;
    while (lo < hi) {
        const int64_t mid = lo + (hi - lo) / 2;
        if (keys[mid].key < want) lo = mid + 1; else hi = mid;
    }
    return lo < n && keys[lo].key == want ? keys[lo].row : -1;
}

int orc_fdg_mesh(const int32_t * coords, const float * feats, int64_t n, int channels, int resolution,
                 float ** vertices_out, int32_t ** faces_out, int64_t * n_faces_out) {
    if (coords == NULL || feats == NULL || vertices_out == NULL || faces_out == NULL || n_faces_out == NULL ||
        n < 0 || n > INT32_MAX || channels < 7 || resolution <= 0) {
        return 2;
    }
    *vertices_out = NULL;
    *faces_out = NULL;
    *n_faces_out = 0;
    if (n == 0) return 0;
    for (int64_t i = 0; i < n; ++i) {
        const int32_t * c = coords + 4 * i;
        if (c[0] != 0) return 4;
        for (int a = 1; a < 4; ++a)
            if (c[a] < 0 || c[a] >= resolution) return 4;
        for (int ch = 0; ch < 7; ++ch)
            if (!isfinite(feats[i * channels + ch])) return 4;
    }
    const int64_t res = resolution;
    orc_fdg_key * keys = (orc_fdg_key *) malloc((size_t) n * sizeof(orc_fdg_key));
    float * vert = (float *) malloc((size_t) n * 3 * sizeof(float));
    float * wgt = (float *) malloc((size_t) n * sizeof(float));
    if (keys == NULL || vert == NULL || wgt == NULL) {
        free(keys);
        free(vert);
        free(wgt);
        return 5;
    }
    for (int64_t i = 0; i < n; ++i) {
        const int32_t * c = coords + 4 * i;
        keys[i].key = ((int64_t) c[1] * res + c[2]) * res + c[3];
        keys[i].row = (int32_t) i;
    }
    qsort(keys, (size_t) n, sizeof(orc_fdg_key), orc_fdg_key_cmp);
    for (int64_t i = 1; i < n; ++i) {
        if (keys[i].key == keys[i - 1].key) {  /* flex_dual_grid.c:236-246 */
            free(keys);
            free(vert);
            free(wgt);
            return 4;
        }
    }
    const float inv_res = 1.0f / (float) resolution;
    for (int64_t i = 0; i < n; ++i) {
        const float * f = feats + i * channels;
        for (int a = 0; a < 3; ++a) {
            const float local = 2.0f * orc_fdg_sigmoid(f[a]) - 0.5f;
            vert[i * 3 + a] = ((float) coords[4 * i + 1 + a] + local) * inv_res - 0.5f;
        }
        wgt[i] = orc_fdg_softplus(f[6]);
    }
    /* Quad corners per axis, as (dx, dy, dz) from the voxel. */
    static const int quad[3][4][3] = {
        {{0, 0, 0}, {0, 0, 1}, {0, 1, 1}, {0, 1, 0}},
        {{0, 0, 0}, {1, 0, 0}, {1, 0, 1}, {0, 0, 1}},
        {{0, 0, 0}, {0, 1, 0}, {1, 1, 0}, {1, 0, 0}},
    };
    static const int quad_mut[4][3] = {{0, 0, 0}, {1, 0, 0}, {1, 1, 0}, {0, 1, 0}};
    int32_t * faces = (int32_t *) malloc((size_t) n * 3 * 2 * 3 * sizeof(int32_t));  /* at most 3 quads per voxel */
    if (faces == NULL) {
        free(keys);
        free(vert);
        free(wgt);
        return 5;
    }
    int64_t nf = 0;
    for (int64_t i = 0; i < n; ++i) {
        const int32_t * c = coords + 4 * i;
        const float * f = feats + i * channels;
        for (int a = 0; a < 3; ++a) {
            if (!(f[3 + a] > 0.0f)) continue;
            int32_t q[4];
            int ok = 1;
            for (int j = 0; j < 4 && ok; ++j) {
                const int * d = (g_mutation == ORC_MUT_FDG_QUAD && a == 2) ? quad_mut[j] : quad[a][j];
                q[j] = orc_fdg_find(keys, n, res, c[1] + d[0], c[2] + d[1], c[3] + d[2]);
                ok = q[j] >= 0;
            }
            if (!ok) continue;
            const float w02 = wgt[q[0]] * wgt[q[2]], w13 = wgt[q[1]] * wgt[q[3]];
            const int first = g_mutation == ORC_MUT_FDG_SPLIT ? w02 >= w13 : w02 > w13;
            const int32_t t[6] = {q[0], q[1], first ? q[2] : q[3], first ? q[0] : q[3], first ? q[2] : q[1],
                                  first ? q[3] : q[2]};
            memcpy(faces + nf * 3, t, sizeof(t));
            nf += 2;
        }
    }
    free(keys);
    free(wgt);
    if (nf == 0) {
        free(faces);
        faces = NULL;
    }
    *vertices_out = vert;
    *faces_out = faces;
    *n_faces_out = nf;
    return 0;
}

void orc_s2c_pack(const float * x, const int32_t * parent, const int32_t * subidx, float * y, int64_t n_fine,
                  int64_t n_coarse, int co) {
    const int pc = co / 8;
    memset(y, 0, (size_t) n_coarse * (size_t) co * sizeof(float));
    for (int64_t f = 0; f < n_fine; ++f) {
        memcpy(y + (int64_t) parent[f] * co + subidx[f] * pc, x + f * pc, (size_t) pc * sizeof(float));
    }
}

void orc_s2c_skip_mean(const float * x, const int32_t * parent, const int32_t * subidx, float * y, int64_t n_fine,
                       int64_t n_coarse, int ci, int co) {
    const int g = 8 * ci / co;
    memset(y, 0, (size_t) n_coarse * (size_t) co * sizeof(float));
    for (int64_t f = 0; f < n_fine; ++f) {
        float * yr = y + (int64_t) parent[f] * co;
        for (int c = 0; c < ci; ++c) {
            const int flat = g_mutation == ORC_MUT_S2C_CHANNEL ? c * 8 + subidx[f] : subidx[f] * ci + c;
            yr[flat / g] += x[f * ci + c] / (float) g;
        }
    }
}

void orc_c2s_gather(const float * x, const int32_t * parent, const int32_t * subidx, float * y, int64_t n_out,
                    int co) {
    for (int64_t r = 0; r < n_out; ++r) {
        const float * from = x + ((int64_t) parent[r] * 8 + subidx[r]) * co;
        memcpy(y + r * co, from, (size_t) co * sizeof(float));
    }
}

void orc_skip_repeat(const float * x, const int32_t * parent, const int32_t * subidx, float * y, int64_t n_out,
                     int ci, int co) {
    /* Repeat-interleave of the parent row over 8 children: child s, channel c
     * reads parent channel (s*co + c) / repeat, clamped to the last channel. */
    const int repeat = g_mutation == ORC_MUT_REPEAT_FLOOR ? (8 * co) / ci : (8 * co + ci - 1) / ci;
    for (int64_t r = 0; r < n_out; ++r) {
        const float * xr = x + (int64_t) parent[r] * ci;
        for (int c = 0; c < co; ++c) {
            int from = (subidx[r] * co + c) / (repeat > 0 ? repeat : 1);
            if (from > ci - 1) {
                from = ci - 1;
            }
            y[r * co + c] = xr[from];
        }
    }
}

static float orc_silu1(float v) { return v / (1.0f + expf(-v)); }

void orc_row_norm(const float * x, const float * gamma, const float * beta, float * y, int64_t n, int c,
                  float eps, int silu) {
    const float var_div = g_mutation == ORC_MUT_NORM_SAMPLE_VAR ? (float) (c - 1) : (float) c;
    for (int64_t r = 0; r < n; ++r) {
        const float * xr = x + r * c;
        float * yr = y + r * c;
        float sum = 0.0f;
        for (int i = 0; i < c; ++i) {
            sum += xr[i];
        }
        const float mean = sum / (float) c;
        float sq = 0.0f;
        for (int i = 0; i < c; ++i) {
            const float d = xr[i] - mean;
            sq += d * d;
        }
        const float inv = 1.0f / sqrtf(sq / var_div + eps);
        for (int i = 0; i < c; ++i) {
            float v = (xr[i] - mean) * inv;
            if (gamma != NULL) v *= gamma[i];
            if (beta != NULL) v += beta[i];
            yr[i] = v;
        }
    }
    if (silu) {
        orc_silu(y, (size_t) n * (size_t) c);
    }
}

void orc_silu(float * x, size_t count) {
    for (size_t i = 0; i < count; ++i) {
        x[i] = orc_silu1(x[i]);
    }
}

void orc_add(const float * a, const float * b, float * y, size_t count) {
    for (size_t i = 0; i < count; ++i) {
        y[i] = a[i] + b[i];
    }
}

void orc_linear(const float * x, const float * w, const float * bias, float * y, int64_t n, int ci, int co,
                int silu) {
    for (int64_t r = 0; r < n; ++r) {
        const float * xr = x + r * ci;
        for (int o = 0; o < co; ++o) {
            const float * wr = w + (int64_t) o * ci;
            float acc = bias == NULL ? 0.0f : bias[o];
            for (int i = 0; i < ci; ++i) {
                acc += xr[i] * wr[i];
            }
            y[r * co + o] = acc;
        }
    }
    if (silu) {
        orc_silu(y, (size_t) n * (size_t) co);
    }
}
