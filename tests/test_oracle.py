"""Pins the CPU oracle (oracle/trellis_oracle.c) before it is trusted as the checker.

Each oracle function is checked against something other than its own formula:
the reference's known-answer vectors and test inputs, brute force, a library
routine (torch conv3d / layer_norm in float64), closed forms or invariants.
Every pin is also run with a planted mistake in the oracle to show it would
catch that error.
"""
import math

import numpy as np
import pytest

import oracle_lib as orc
import workloads as wl


def close(got, exp, tol):
    """check_close of tests/test_sparse_decoder_backend.c:16-24: |a-b| <= tol*max(1,|a|,|b|)."""
    got = np.asarray(got, dtype=np.float64)
    exp = np.asarray(exp, dtype=np.float64)
    scale = np.maximum(1.0, np.maximum(np.abs(got), np.abs(exp)))
    return bool(np.all(np.abs(got - exp) <= tol * scale))


def np_join_neighbors(coords):
    """Independent neighbour table: sorted 16-bit-field keys + searchsorted."""
    c = np.asarray(coords, dtype=np.int64)

    def key(a):
        return ((a[:, 0] & 0xFFFF) << 48) | ((a[:, 1] & 0xFFFF) << 32) | ((a[:, 2] & 0xFFFF) << 16) | (a[:, 3] & 0xFFFF)

    keys = key(c)
    order = np.argsort(keys, kind="stable")
    sk = keys[order]
    out = np.full((c.shape[0], 27), -1, dtype=np.int32)
    for k in range(27):
        q = c.copy()
        q[:, 1] += k // 9 - 1
        q[:, 2] += (k // 3) % 3 - 1
        q[:, 3] += k % 3 - 1
        kq = key(q)
        # last duplicate wins: take the rightmost equal key (stable sort keeps row order)
        pos = np.searchsorted(sk, kq, side="right") - 1
        ok = (pos >= 0) & (sk[np.clip(pos, 0, None)] == kq)
        out[ok, k] = order[pos[ok]]
    return out


# --------------------------------------------------------------------------- keys

def test_pack_coord4_fields_and_sentinel():
    # trellis_sparse_cpu.c:24-31: 16-bit fields b|x|y|z, +1.
    assert orc.pack_coord4(0, 0, 0, 0) == 1
    assert orc.pack_coord4(1, 2, 3, 4) == ((1 << 48) | (2 << 32) | (3 << 16) | 4) + 1
    assert orc.pack_coord4(0, -1, 0, 0) == (0xFFFF << 32) + 1  # wraps modulo 2^16
    assert orc.pack_coord4(0, 65536 + 7, 0, 0) == orc.pack_coord4(0, 7, 0, 0)


def test_hash_is_splitmix64_finaliser():
    # Published splitmix64 (Steele, Lea, Flood 2014): state += golden gamma, output = mix(state);
    # the first two outputs from seed 0 are known values.
    gamma = 0x9E3779B97F4A7C15
    assert orc.hash_u64(gamma) == 0xE220A8397B1DCDAF
    assert orc.hash_u64((2 * gamma) & (2**64 - 1)) == 0x6E789E6AA1B965F4


def test_table_size_is_next_pow2_of_2n():
    assert [orc.table_size(n) for n in (1, 2, 3, 4, 5, 1000)] == [2, 4, 8, 8, 16, 2048]


# ---------------------------------------------------------------------- neighbours

def small_coords(seed=0, n=300, box=7, batches=2, dup=True):
    rng = np.random.default_rng(seed)
    c = np.stack([rng.integers(0, batches, n), rng.integers(-2, box, n), rng.integers(-2, box, n),
                  rng.integers(-2, box, n)], axis=1).astype(np.int32)
    if dup:
        c[-5:] = c[:5]  # duplicates: the later rows must win
    return c


def test_neighbors_match_bruteforce_with_duplicates_and_negatives():
    c = small_coords()
    assert np.array_equal(orc.Rulebook(c).neighbors(), orc.neighbors_bruteforce(c))


def test_neighbors_wrap_like_reference_keys():
    # x = -1 packs to 0xffff, so a voxel at x = 65535 is the -x neighbour of x = 0.
    c = np.array([[0, 0, 5, 5], [0, 65535, 5, 5], [0, 1, 5, 5]], dtype=np.int32)
    nbr = orc.Rulebook(c).neighbors()
    assert nbr[0, 0 * 9 + 1 * 3 + 1] == 1   # kd=0 -> x-1 wraps onto row 1
    assert nbr[0, 2 * 9 + 1 * 3 + 1] == 2   # kd=2 -> x+1
    assert nbr[1, 2 * 9 + 1 * 3 + 1] == 0   # 65535 + 1 wraps onto x = 0
    assert nbr[0, 13] == 0 and nbr[1, 13] == 1


def test_config1_pairs_match_reference_calibration():
    # The compiled reference's CPU path (trellis_sparse_cpu.c), run on this set: N=14,648, P=261,416.
    c = wl.make_coords(1)
    assert c.shape[0] == 14648
    nbr = orc.Rulebook(c).neighbors()
    assert int((nbr >= 0).sum()) == 261416
    assert np.array_equal(nbr, np_join_neighbors(c))


def test_neighbor_symmetry_invariant():
    c = wl.make_coords(1)
    nbr = orc.Rulebook(c).neighbors()
    i, k = np.nonzero(nbr >= 0)
    j = nbr[i, k]
    assert np.array_equal(nbr[j, 26 - k], i.astype(np.int32))


@pytest.mark.parametrize("mut", [1, 6, 7])  # axis swap, sign flip, batch crossing
def test_neighbor_pins_catch_planted_mistakes(mut):
    c = small_coords(seed=3, n=400, box=6, batches=3, dup=False)
    with orc.mutation(mut):
        bad = orc.Rulebook(c).neighbors()
    assert not np.array_equal(bad, np_join_neighbors(c))


def test_pairs_canonical_order():
    c = small_coords(seed=1)
    nbr = orc.Rulebook(c).neighbors()
    counts, src, dst = orc.pairs(nbr)
    assert counts.sum() == (nbr >= 0).sum() == src.size
    at = 0
    for k in range(27):
        d = dst[at:at + counts[k]]
        assert np.all(np.diff(d) > 0)  # destination ascending within an offset
        assert np.array_equal(src[at:at + counts[k]], nbr[d, k])
        at += counts[k]


# ------------------------------------------------------------------------- conv

def reference_direct_case():
    """tests/test_sparse_decoder_backend.c:366-394 inputs (8 voxels, 3 -> 2)."""
    coords = np.array([[0, 1, 1, 1], [0, 0, 1, 1], [0, 2, 1, 1], [0, 1, 0, 1], [0, 1, 2, 1], [0, 1, 1, 0],
                       [0, 1, 1, 2], [0, 0, 0, 0]], dtype=np.int32)
    n, ci, co = 8, 3, 2
    feats = np.array([[math.sin(r * 0.31 + c * 0.17) + 0.05 * (r - c) for c in range(ci)] for r in range(n)],
                     dtype=np.float32)
    w = np.zeros((co, 27, ci), dtype=np.float32)
    for o in range(co):
        for v in range(27):
            for i in range(ci):
                w[o, v, i] = 0.01 * ((o + 1) * (i + 2)) + 0.0025 * (v - 13)
    bias = np.array([0.125, -0.075], dtype=np.float32)
    return coords, feats, w, bias, ci, co


def reference_trellis_case():
    """tests/test_trellis.c:1376-1396 inputs (6 voxels, 3 -> 2)."""
    coords = np.array([[0, 0, 0, 0], [0, 1, 0, 0], [0, 0, 1, 0], [0, 0, 0, 1], [0, 1, 1, 0], [0, 3, 0, 0]],
                      dtype=np.int32)
    ci, co = 3, 2
    feats = np.array([0.2 * math.sin(0.31 * (i + 1)) + 0.03 * (i % 4) for i in range(6 * ci)],
                     dtype=np.float32).reshape(6, ci)
    w = np.array([0.1 * math.cos(0.07 * (i - 5)) for i in range(co * 27 * ci)], dtype=np.float32).reshape(co, 27, ci)
    bias = np.array([0.15, -0.2], dtype=np.float32)
    return coords, feats, w, bias, ci, co


@pytest.mark.parametrize("case,tol", [(reference_direct_case, 2e-4), (reference_trellis_case, 2e-5)])
def test_conv_matches_bruteforce_on_reference_inputs(case, tol):
    coords, feats, w, bias, ci, co = case()
    got = orc.Rulebook(coords).conv(feats, w, bias, ci, co)
    exp = orc.conv_bruteforce(coords, feats, w, bias, ci, co)
    assert close(got, exp, tol)
    with orc.mutation(2):  # drop bias
        bad = orc.Rulebook(coords).conv(feats, w, bias, ci, co)
    assert not close(bad, exp, tol)


def test_conv_centre_only_is_linear_layer():
    c = wl.make_coords(1)[:3000]
    rng = np.random.default_rng(5)
    ci, co = 16, 8
    x = rng.standard_normal((c.shape[0], ci)).astype(np.float32)
    w = np.zeros((co, 27, ci), dtype=np.float32)
    w[:, 13, :] = rng.standard_normal((co, ci)).astype(np.float32)
    b = rng.standard_normal(co).astype(np.float32)
    got = orc.Rulebook(c).conv(x, w, b, ci, co)
    exp = x.astype(np.float64) @ w[:, 13, :].T.astype(np.float64) + b
    assert close(got, exp, 1e-5)


def dense_block(side=8, ci=4, co=3, seed=7):
    g = np.arange(side)
    xs, ys, zs = np.meshgrid(g, g, g, indexing="ij")
    coords = np.stack([np.zeros(side**3, np.int32), xs.ravel(), ys.ravel(), zs.ravel()], axis=1).astype(np.int32)
    rng = np.random.default_rng(seed)
    feats = rng.standard_normal((side**3, ci)).astype(np.float32)
    w = rng.standard_normal((co, 27, ci)).astype(np.float32) / math.sqrt(27 * ci)
    bias = rng.standard_normal(co).astype(np.float32)
    return coords, feats, w, bias, side


def torch_dense_conv(feats, w, bias, side):
    torch = pytest.importorskip("torch")
    ci = feats.shape[1]
    co = w.shape[0]
    inp = torch.from_numpy(feats.astype(np.float64).reshape(side, side, side, ci)).permute(3, 0, 1, 2)[None]
    wt = torch.from_numpy(w.astype(np.float64).reshape(co, 3, 3, 3, ci)).permute(0, 4, 1, 2, 3).contiguous()
    out = torch.nn.functional.conv3d(inp, wt, torch.from_numpy(bias.astype(np.float64)), padding=1)
    return out[0].permute(1, 2, 3, 0).reshape(-1, co).numpy()


def test_conv_dense_block_matches_torch_conv3d():
    coords, feats, w, bias, side = dense_block()
    got = orc.Rulebook(coords).conv(feats, w, bias, feats.shape[1], w.shape[0])
    exp = torch_dense_conv(feats, w, bias, side)
    assert close(got, exp, 1e-5)
    with orc.mutation(1):  # kd <-> kw swap
        bad = orc.Rulebook(coords).conv(feats, w, bias, feats.shape[1], w.shape[0])
    assert not close(bad, exp, 1e-5)


def test_conv_linearity_and_row_subset():
    c = wl.make_coords(1)[:2000]
    rng = np.random.default_rng(9)
    ci, co = 8, 8
    x1 = rng.standard_normal((c.shape[0], ci)).astype(np.float32)
    x2 = rng.standard_normal((c.shape[0], ci)).astype(np.float32)
    w = rng.standard_normal((co, 27, ci)).astype(np.float32) * 0.1
    rb = orc.Rulebook(c)
    y = rb.conv(2.0 * x1 + 3.0 * x2, w, None, ci, co)
    assert close(y, 2.0 * rb.conv(x1, w, None, ci, co) + 3.0 * rb.conv(x2, w, None, ci, co), 1e-5)
    sub = rb.conv(x1, w, None, ci, co, rows=(3, 2000, 7))
    assert np.array_equal(sub, rb.conv(x1, w, None, ci, co)[3:2000:7])


# -------------------------------------------------------------------- subdivide

def c2s_kat():
    """tests/test_trellis.c:1325-1347 known answer: 4 parents -> 6 children."""
    coords = np.array([[0, 1, 2, 3], [0, 4, 5, 6], [1, 0, 0, 0], [1, 2, 1, 0]], dtype=np.int32)
    subdiv = np.array([[0.5, -1.0, -1.0, 0.25, -1.0, -1.0, -1.0, -1.0], [-1.0] * 8,
                       [-1.0, -1.0, -1.0, -1.0, -1.0, -1.0, -1.0, 0.1],
                       [-1.0, 0.2, 0.3, -1.0, 0.4, -1.0, -1.0, -1.0]], dtype=np.float32)
    exp_coords = np.array([[0, 2, 4, 6], [0, 3, 5, 6], [1, 1, 1, 1], [1, 5, 2, 0], [1, 4, 3, 0], [1, 4, 2, 1]],
                          dtype=np.int32)
    return coords, subdiv, exp_coords, np.array([0, 0, 2, 3, 3, 3]), np.array([0, 3, 7, 1, 2, 4])


def test_c2s_map_known_answer():
    coords, subdiv, ec, ep, es = c2s_kat()
    rc, oc, op, os_ = orc.c2s_map(coords, subdiv)
    assert rc == 0
    assert np.array_equal(oc, ec) and np.array_equal(op, ep) and np.array_equal(os_, es)
    with orc.mutation(3):  # subidx bit order
        rc, oc, _, _ = orc.c2s_map(coords, subdiv)
    assert not np.array_equal(oc, ec)


def test_c2s_map_strict_positive_and_empty():
    coords = np.array([[0, 1, 1, 1]], dtype=np.int32)
    logits = np.array([[0.0, -0.0, 1e-30, -1.0, 0.0, 0.0, 0.0, 2.0]], dtype=np.float32)
    rc, oc, op, os_ = orc.c2s_map(coords, logits)
    assert rc == 0 and list(os_) == [2, 7]  # executor.c:119: only logits > 0 (strict)
    with orc.mutation(8):
        rc, _, _, os_bad = orc.c2s_map(coords, logits)
    assert list(os_bad) != [2, 7]
    rc, *_ = orc.c2s_map(coords, -np.ones((1, 8), np.float32))
    assert rc == 1  # executor.c:125-127: no child -> TRELLIS_STATUS_ERROR


def test_c2s_gather_known_answer_and_closed_form():
    # tests/test_trellis.c:1521-1533: coarse row [11,22,0,...] with children s=0,1 -> [11],[22].
    x = np.array([[11, 22, 0, 0, 0, 0, 0, 0]], dtype=np.float32)
    y = orc.c2s_gather(x, [0, 0], [0, 1], 1)
    assert y.ravel().tolist() == [11.0, 22.0]
    rng = np.random.default_rng(2)
    co = 5
    xp = rng.standard_normal((7, 8 * co)).astype(np.float32)
    parent = rng.integers(0, 7, 40)
    sub = rng.integers(0, 8, 40)
    exp = xp.reshape(7, 8, co)[parent, sub]
    assert np.array_equal(orc.c2s_gather(xp, parent, sub, co), exp)


@pytest.mark.parametrize("ci,co", [(256, 256), (3, 2), (8, 2), (16, 24), (64, 7)])
def test_skip_repeat_matches_repeat_interleave(ci, co):
    rng = np.random.default_rng(ci * 31 + co)
    x = rng.standard_normal((9, ci)).astype(np.float32)
    parent = rng.integers(0, 9, 50)
    sub = rng.integers(0, 8, 50)
    repeat = -(-8 * co // ci)
    exp = np.empty((50, co), np.float32)
    for r in range(50):
        rep = np.repeat(x[parent[r]], repeat)  # repeat-interleave of the parent row
        idx = np.minimum(np.arange(sub[r] * co, sub[r] * co + co), rep.size - 1)
        vals = rep[idx]
        # past the end of the interleaved row the reference clamps to the last channel
        vals[np.arange(sub[r] * co, sub[r] * co + co) >= ci * repeat] = x[parent[r], ci - 1]
        exp[r] = vals
    assert np.array_equal(orc.skip_repeat(x, parent, sub, ci, co), exp)
    if (8 * co) % ci and (8 * co) // ci >= 1:  # floor differs from ceil and is a usable repeat
        with orc.mutation(4):
            assert not np.array_equal(orc.skip_repeat(x, parent, sub, ci, co), exp)


# --------------------------------------------------- FlexiDualGrid mesh
def fdg_kat():
    """tests/test_trellis.c:581-627: four voxels of one z = 0 face, zero
    logits except channel 5 of voxel 0 (the axis-2 quad), resolution 4."""
    coords = np.array([[0, 0, 0, 0], [0, 0, 1, 0], [0, 1, 1, 0], [0, 1, 0, 0]], np.int32)
    feats = np.zeros((4, 7), np.float32)
    feats[0, 5] = 1.0
    return coords, feats


def test_fdg_mesh_known_answer_and_rejects():
    coords, feats = fdg_kat()
    rc, v, f = orc.fdg_mesh(coords, feats, 4)
    assert rc == 0 and v.shape == (4, 3) and f.shape == (2, 3)
    assert np.allclose(v[0], [-0.375, -0.375, -0.375], atol=1e-6)
    assert f.tolist() == [[0, 1, 3], [3, 1, 2]]
    with orc.mutation(11):  # ties split the other way
        assert orc.fdg_mesh(coords, feats, 4)[2].tolist() != [[0, 1, 3], [3, 1, 2]]
    bad = coords.copy(); bad[0, 0] = 1
    assert orc.fdg_mesh(bad, feats, 4)[0] == 4
    bad = coords.copy(); bad[0, 1] = -1
    assert orc.fdg_mesh(bad, feats, 4)[0] == 4
    bad[0, 1] = 4
    assert orc.fdg_mesh(bad, feats, 4)[0] == 4
    bad = coords.copy(); bad[1] = bad[0]
    assert orc.fdg_mesh(bad, feats, 4)[0] == 4
    nanf = feats.copy(); nanf[0, 3] = np.nan
    assert orc.fdg_mesh(coords, nanf, 4)[0] == 4
    assert orc.fdg_mesh(np.zeros((0, 4), np.int32), np.zeros((0, 7), np.float32), 4)[0] == 0


def py_quads(coords, feats):
    """Independent quad search: a Python dict of voxels, corners per axis from
    the face the quad lies in (x-faces span y/z, y-faces z/x, z-faces x/y)."""
    where = {tuple(c[1:]): i for i, c in enumerate(coords.tolist())}
    corners = {0: [(0, 0, 0), (0, 0, 1), (0, 1, 1), (0, 1, 0)], 1: [(0, 0, 0), (1, 0, 0), (1, 0, 1), (0, 0, 1)],
               2: [(0, 0, 0), (0, 1, 0), (1, 1, 0), (1, 0, 0)]}
    out = []
    for i, c in enumerate(coords.tolist()):
        for a in range(3):
            if feats[i, 3 + a] > 0:
                q = [where.get((c[1] + d[0], c[2] + d[1], c[3] + d[2]), -1) for d in corners[a]]
                if min(q) >= 0:
                    out.append(q)
    return out


def test_fdg_mesh_quads_and_vertices_on_random_sets():
    rng = np.random.default_rng(12)
    res = 24
    c = np.unique(rng.integers(0, res, (4000, 3)), axis=0)
    coords = np.concatenate([np.zeros((c.shape[0], 1), np.int64), c], axis=1).astype(np.int32)
    coords = coords[rng.permutation(coords.shape[0])]
    feats = rng.standard_normal((coords.shape[0], 9)).astype(np.float32) * 3
    rc, v, f = orc.fdg_mesh(coords, feats, res)
    assert rc == 0
    quads = py_quads(coords, feats)
    assert f.shape[0] == 2 * len(quads)
    # Each quad's two triangles use its four corners, split on one diagonal.
    for j, q in enumerate(quads):
        t0, t1 = f[2 * j].tolist(), f[2 * j + 1].tolist()
        assert set(t0) | set(t1) == set(q) and t0[:2] == [q[0], q[1]]
    sig = 1.0 / (1.0 + np.exp(-feats[:, :3].astype(np.float64)))
    exp_v = (coords[:, 1:] + 2.0 * sig - 0.5) / res - 0.5
    assert np.max(np.abs(v - exp_v)) < 1e-6
    with orc.mutation(12):
        assert orc.fdg_mesh(coords, feats, res)[2].shape != f.shape or not np.array_equal(
            orc.fdg_mesh(coords, feats, res)[2], f)


# ------------------------------------------------------------ S2C (encoder)
def s2c_kat():
    """tests/test_sparse_encoder_backend.c:84-110: five fine voxels (b, x, y, z),
    their features, the expected coarse voxels, parent and subidx, and the
    coarse channels the encoder produces with zero conv weights (the skip
    means, Ci = 2 -> Co = 8, identity input layer)."""
    coords = np.array([[0, 3, 1, 0], [0, 0, 0, 0], [0, 1, 0, 0], [0, 2, 1, 1], [0, 0, 2, 0]], np.int32)
    feats = np.array([[2, 4], [1, 3], [-2, 0], [6, 2], [5, -1]], np.float32)
    exp_coarse = np.array([[0, 0, 0, 0], [0, 0, 1, 0], [0, 1, 0, 0]], np.int32)
    exp_parent = np.array([2, 0, 0, 2, 1])
    exp_subidx = np.array([3, 0, 1, 6, 0])
    exp_channels = np.array([[2, -1, 0, 0, 0, 0, 0, 0], [2, 0, 0, 0, 0, 0, 0, 0], [0, 0, 0, 3, 0, 0, 4, 0]],
                            np.float32)
    return coords, feats, exp_coarse, exp_parent, exp_subidx, exp_channels


def test_s2c_map_and_skip_mean_known_answer():
    coords, feats, ec, ep, es, ech = s2c_kat()
    rc, oc, op, os_ = orc.s2c_map(coords)
    assert rc == 0
    assert np.array_equal(oc, ec) and np.array_equal(op, ep) and np.array_equal(os_, es)
    assert np.array_equal(orc.s2c_skip_mean(feats, op, os_, 3, 2, 8), ech)
    with orc.mutation(9):  # coarse order z-major
        rc, oc_bad, _, _ = orc.s2c_map(coords)
    assert rc == 0 and not np.array_equal(oc_bad, ec)
    with orc.mutation(10):  # channel-major skip groups
        assert not np.array_equal(orc.s2c_skip_mean(feats, op, os_, 3, 2, 8), ech)


def random_fine_set(rng, n, extent, batches):
    c = np.stack([rng.integers(0, batches, n), rng.integers(0, extent, n), rng.integers(0, extent, n),
                  rng.integers(0, extent, n)], axis=1).astype(np.int32)
    c = np.unique(c, axis=0)
    return c[rng.permutation(c.shape[0])]


@pytest.mark.parametrize("seed", [0, 1, 2])
def test_s2c_map_matches_numpy_unique(seed):
    rng = np.random.default_rng(seed)
    fine = random_fine_set(rng, 3000, 37, 3)
    coarse_of = fine.copy()
    coarse_of[:, 1:] //= 2
    exp_coarse, exp_parent = np.unique(coarse_of, axis=0, return_inverse=True)
    rc, oc, op, os_ = orc.s2c_map(fine)
    assert rc == 0
    assert np.array_equal(oc, exp_coarse) and np.array_equal(op, exp_parent.ravel())
    assert np.array_equal(os_, (fine[:, 1] & 1) | ((fine[:, 2] & 1) << 1) | ((fine[:, 3] & 1) << 2))
    with orc.mutation(9):
        _, oc_bad, _, _ = orc.s2c_map(fine)
    assert not np.array_equal(oc_bad, exp_coarse)


def test_s2c_inverts_c2s():
    """The S2C of a C2S map recovers the parents that have children, in
    order, with the C2S parent and subidx of every child."""
    rng = np.random.default_rng(4)
    parents = np.unique(np.stack([rng.integers(0, 2, 500), rng.integers(0, 50, 500), rng.integers(0, 50, 500),
                                  rng.integers(0, 50, 500)], axis=1).astype(np.int32), axis=0)
    logits = rng.choice([-1.0, 1.0], size=(parents.shape[0], 8)).astype(np.float32)
    rc, children, cpar, csub = orc.c2s_map(parents, logits)
    assert rc == 0
    perm = rng.permutation(children.shape[0])
    rc, coarse, par, sub = orc.s2c_map(children[perm])
    assert rc == 0
    has_child = np.unique(cpar)
    assert np.array_equal(coarse, parents[has_child])
    assert np.array_equal(has_child[par], cpar[perm]) and np.array_equal(sub, csub[perm])


def test_s2c_rejects_negative_and_duplicate():
    ok = np.array([[0, 1, 2, 3], [0, 4, 4, 4]], np.int32)
    assert orc.s2c_map(ok)[0] == 0
    assert orc.s2c_map(np.array([[0, 1, -2, 3]], np.int32))[0] == 2  # s2c_host.c:61-67
    assert orc.s2c_map(np.array([[-1, 1, 2, 3]], np.int32))[0] == 2
    assert orc.s2c_map(np.array([[0, 1, 2, 3], [0, 5, 5, 5], [0, 1, 2, 3]], np.int32))[0] == 4  # :80-88


@pytest.mark.parametrize("co", [8, 64, 24])
def test_s2c_pack_inverted_by_c2s_gather(co):
    rng = np.random.default_rng(co)
    fine = random_fine_set(rng, 800, 21, 2)
    rc, coarse, par, sub = orc.s2c_map(fine)
    pc = co // 8
    x = rng.standard_normal((fine.shape[0], pc)).astype(np.float32)
    packed = orc.s2c_pack(x, par, sub, coarse.shape[0], co)
    assert np.array_equal(orc.c2s_gather(packed, par, sub, pc), x)
    filled = np.zeros((coarse.shape[0], 8), bool)
    filled[par, sub] = True
    assert not np.any(packed.reshape(coarse.shape[0], 8, pc)[~filled])


@pytest.mark.parametrize("ci,co", [(2, 8), (64, 128), (128, 256), (96, 64)])
def test_s2c_skip_mean_closed_form(ci, co):
    rng = np.random.default_rng(ci + co)
    fine = random_fine_set(rng, 600, 17, 2)
    rc, coarse, par, sub = orc.s2c_map(fine)
    m, g, pc = coarse.shape[0], 8 * ci // co, co // 8
    x = rng.standard_normal((fine.shape[0], ci)).astype(np.float32)
    # Child slot s of a coarse row holds the g-channel group means of that
    # child, summed left to right in fp32 from zero.
    exp = np.zeros((m, 8, pc), np.float32)
    terms = (x / np.float32(g)).reshape(-1, pc, g)
    acc = np.zeros((fine.shape[0], pc), np.float32)
    for t in range(g):
        acc = (acc + terms[:, :, t]).astype(np.float32)
    exp[par, sub] = acc
    assert np.array_equal(orc.s2c_skip_mean(x, par, sub, m, ci, co), exp.reshape(m, co))
    # Groups of equal values come back unchanged through skip_repeat (g = 2^k).
    if g & (g - 1) == 0:
        xc = np.repeat(rng.integers(-8, 8, (fine.shape[0], pc)).astype(np.float32), g, axis=1)
        mean = orc.s2c_skip_mean(xc, par, sub, m, ci, co)
        assert np.array_equal(orc.skip_repeat(mean, par, sub, co, ci), xc)
    with orc.mutation(10):
        assert not np.array_equal(orc.s2c_skip_mean(x, par, sub, m, ci, co), exp.reshape(m, co))


# ------------------------------------------------------------------ row ops

def test_row_norm_matches_torch_layer_norm():
    torch = pytest.importorskip("torch")
    rng = np.random.default_rng(4)
    n, c = 33, 96
    x = (rng.standard_normal((n, c)) * 3 + 1).astype(np.float32)
    g = rng.standard_normal(c).astype(np.float32)
    b = rng.standard_normal(c).astype(np.float32)
    for eps in (1e-6, 1e-5):
        ref = torch.nn.functional.layer_norm(torch.from_numpy(x.astype(np.float64)), (c,),
                                             torch.from_numpy(g.astype(np.float64)),
                                             torch.from_numpy(b.astype(np.float64)), eps)
        assert close(orc.row_norm(x, g, b, n, c, eps), ref.numpy(), 1e-5)
        silu = torch.nn.functional.silu(ref).numpy()
        assert close(orc.row_norm(x, g, b, n, c, eps, silu=True), silu, 1e-5)
        plain = torch.nn.functional.layer_norm(torch.from_numpy(x.astype(np.float64)), (c,), eps=eps).numpy()
        assert close(orc.row_norm(x, None, None, n, c, eps), plain, 1e-5)
    with orc.mutation(5):
        assert not close(orc.row_norm(x, g, b, n, c, 1e-6), torch.nn.functional.layer_norm(
            torch.from_numpy(x.astype(np.float64)), (c,), torch.from_numpy(g.astype(np.float64)),
            torch.from_numpy(b.astype(np.float64)), 1e-6).numpy(), 1e-5)


def test_silu_add_linear_against_float64():
    rng = np.random.default_rng(6)
    a = rng.standard_normal(257).astype(np.float32) * 4
    b = rng.standard_normal(257).astype(np.float32)
    ad = a.astype(np.float64)
    assert close(orc.silu(a), ad / (1 + np.exp(-ad)), 1e-6)
    assert np.array_equal(orc.add(a, b), a + b)
    n, ci, co = 20, 17, 9
    x = rng.standard_normal((n, ci)).astype(np.float32)
    w = rng.standard_normal((co, ci)).astype(np.float32)
    bias = rng.standard_normal(co).astype(np.float32)
    exp = x.astype(np.float64) @ w.T.astype(np.float64) + bias
    assert close(orc.linear(x, w, bias, n, ci, co), exp, 1e-5)
    assert close(orc.linear(x, w, bias, n, ci, co, silu=True), exp / (1 + np.exp(-exp)), 1e-5)
