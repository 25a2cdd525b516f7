"""GPU parity of the FlexiDualGrid mesh extraction from decoder logits.

The reference extracts the mesh on the host from the downloaded decoder output
(src/ops/mesh/flex_dual_grid.c:166-313, called at latent_decode.c:146); the
backend does it on the device (trellis_sparse_hip_flex_dual_grid_mesh).  The
oracle runs on the same storage-rounded logits.  Vertices meet the fp32
tolerance (1e-5, check_close of test_sparse_decoder_backend.c:16-24).  Faces
are identical, except that a quad whose two diagonal weight products are
equal to within the fp32 tolerance may split the other way (exp / log1p
round differently on the device and in libm); each such quad is checked to be
that near-tie.
"""
import sys

import numpy as np
import pytest

import oracle_lib as orc
import sparse_hip as sh
import workloads as wl

pytestmark = pytest.mark.gpu


def say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


@pytest.fixture(scope="module")
def backends():
    bes = {dt: sh.Backend(0, dt) for dt in (sh.F32, sh.F16, sh.BF16)}
    yield bes
    for b in bes.values():
        b.destroy()


def softplus64(v):
    v = v.astype(np.float64)
    return np.where(v > 20, v, np.where(v < -20, np.exp(v), np.log1p(np.exp(v))))


def quad_corners(t):
    """Corners q0..q3 of a quad from its two triangles (either split)."""
    if t[1][0] == t[0][0]:  # (q0,q1,q2),(q0,q2,q3): w02 > w13
        return t[0][0], t[0][1], t[0][2], t[1][2]
    return t[0][0], t[0][1], t[1][2], t[0][2]  # (q0,q1,q3),(q3,q1,q2)


def compare_mesh(got_v, got_f, exp_v, exp_f, feats):
    """Vertices to 1e-5; faces identical except near-tie splits of one quad."""
    scale = np.maximum(1.0, np.maximum(np.abs(got_v), np.abs(exp_v)))
    assert np.max(np.abs(got_v - exp_v) / scale) <= 1e-5
    assert got_f.shape == exp_f.shape
    diff = np.unique(np.nonzero(np.any(got_f != exp_f, axis=1))[0] // 2)
    w = softplus64(feats[:, 6])
    for qd in diff:
        te = exp_f[2 * qd: 2 * qd + 2].tolist()
        tg = got_f[2 * qd: 2 * qd + 2].tolist()
        q = quad_corners(te)
        assert quad_corners(tg) == q  # the same quad, split the other way
        w02, w13 = w[q[0]] * w[q[2]], w[q[1]] * w[q[3]]
        assert abs(w02 - w13) <= 1e-5 * max(w02, w13)
    return len(diff)


def test_mesh_known_answer_and_rejects(backends):
    """tests/test_trellis.c:581-627."""
    be = backends[sh.F32]
    coords = np.array([[0, 0, 0, 0], [0, 0, 1, 0], [0, 1, 1, 0], [0, 1, 0, 0]], np.int32)
    feats = np.zeros((4, 7), np.float32)
    feats[0, 5] = 1.0
    fb = be.upload(feats)
    v, f = be.flex_dual_grid_mesh(fb, 4, 7, 4, coords=coords)
    assert v.shape == (4, 3) and np.allclose(v[0], [-0.375, -0.375, -0.375], atol=1e-6)
    assert f.tolist() == [[0, 1, 3], [3, 1, 2]]
    for bad in ([1, 0, 0, 0, 0], [0, -1, 0, 0, 0], [0, 4, 0, 0, 0]):
        c = coords.copy()
        c[0] = bad[:4]
        with pytest.raises(sh.HipError) as ei:
            be.flex_dual_grid_mesh(fb, 4, 7, 4, coords=c)
        assert ei.value.status == sh.PARSE_ERROR
    c = coords.copy()
    c[1] = c[0]
    with pytest.raises(sh.HipError) as ei:
        be.flex_dual_grid_mesh(fb, 4, 7, 4, coords=c)
    assert ei.value.status == sh.PARSE_ERROR
    nanf = feats.copy()
    nanf[0, 3] = np.nan
    with pytest.raises(sh.HipError) as ei:
        be.flex_dual_grid_mesh(be.upload(nanf), 4, 7, 4, coords=coords)
    assert ei.value.status == sh.PARSE_ERROR
    with pytest.raises(sh.HipError) as ei:
        be.flex_dual_grid_mesh(fb, 4, 6, 4, coords=coords)
    assert ei.value.status == sh.INVALID_ARGUMENT
    with pytest.raises(sh.HipError) as ei:
        be.flex_dual_grid_mesh(fb, 4, 7, 70000, coords=coords)
    assert ei.value.status == sh.NOT_IMPLEMENTED
    v, f = be.flex_dual_grid_mesh(fb, 0, 7, 4, coords=coords)
    assert v.shape == (0, 3) and f.shape == (0, 3)
    v, f = be.flex_dual_grid_mesh(fb, 4, 7, 4, coords=coords)  # still usable after the errors
    assert f.tolist() == [[0, 1, 3], [3, 1, 2]]


@pytest.mark.parametrize("dtype", [sh.F32, sh.F16, sh.BF16])
@pytest.mark.parametrize("channels,res,n", [(7, 24, 4000), (9, 64, 60000), (7, 8, 512)])
def test_mesh_vs_oracle(backends, dtype, channels, res, n):
    be = backends[dtype]
    rng = np.random.default_rng(res + n + dtype)
    c = np.unique(rng.integers(0, res, (n, 3)), axis=0)
    coords = np.concatenate([np.zeros((c.shape[0], 1), np.int64), c], axis=1).astype(np.int32)
    coords = np.ascontiguousarray(coords[rng.permutation(coords.shape[0])])
    m = coords.shape[0]
    feats = sh.storage_round(rng.standard_normal((m, channels)).astype(np.float32) * 3, dtype)
    say(f"mesh dtype={dtype} channels={channels} res={res} voxels={m}")
    v, f = be.flex_dual_grid_mesh(be.upload(feats), m, channels, res, coords=coords)
    rc, ev, ef = orc.fdg_mesh(coords, feats, res)
    assert rc == 0
    flips = compare_mesh(v, f, ev, ef, feats)
    say(f"mesh faces={f.shape[0]} near-tie flips={flips}")


def test_mesh_config3_children_from_device_map(backends):
    """~1.26M voxels (config-3 children at R = 512) with coordinates in a
    device map, as the decoder leaves them."""
    be = backends[sh.BF16]
    w = wl.workload(3)
    rc, children, _, _ = orc.c2s_map(w["parent_coords"], w["logits"])
    assert rc == 0
    rng = np.random.default_rng(8)
    feats = sh.storage_round(rng.standard_normal((children.shape[0], 7)).astype(np.float32) * 2, sh.BF16)
    cmap = be.upload_coords(children)
    say(f"mesh config-3 children voxels={children.shape[0]}")
    v, f = be.flex_dual_grid_mesh(be.upload(feats), children.shape[0], 7, 512, coords_map=cmap)
    rc, ev, ef = orc.fdg_mesh(children, feats, 512)
    assert rc == 0
    flips = compare_mesh(v, f, ev, ef, feats)
    say(f"mesh config-3 faces={f.shape[0]} near-tie flips={flips}")
    be.free_map(cmap)
