"""GPU parity of the encoder's spatial-to-channel downsample (S2C).

The reference builds the S2C relation on the host
(src/architectures/sparse_unet_encoder/s2c_host.c:33-120) and packs the conv
output and the skip means on the host (sparse_unet_encoder/executor.c:258-300).
The backend does all three on the device (trellis_sparse_hip_s2c_*); maps are
compared bit-exactly with the oracle's restatement, pack and skip means
bit-exactly on the same storage-rounded inputs (their arithmetic is one fp32
division and ordered sums, the same on both sides).
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


def kat():
    """tests/test_sparse_encoder_backend.c:84-110 (see tests/test_oracle.py)."""
    coords = np.array([[0, 3, 1, 0], [0, 0, 0, 0], [0, 1, 0, 0], [0, 2, 1, 1], [0, 0, 2, 0]], np.int32)
    feats = np.array([[2, 4], [1, 3], [-2, 0], [6, 2], [5, -1]], np.float32)
    coarse = np.array([[0, 0, 0, 0], [0, 0, 1, 0], [0, 1, 0, 0]], np.int32)
    channels = np.array([[2, -1, 0, 0, 0, 0, 0, 0], [2, 0, 0, 0, 0, 0, 0, 0], [0, 0, 0, 3, 0, 0, 4, 0]], np.float32)
    return coords, feats, coarse, np.array([2, 0, 0, 2, 1]), np.array([3, 0, 1, 6, 0]), channels


def random_fine_set(rng, n, extent, batches, big=0):
    c = np.stack([rng.integers(0, batches, n), rng.integers(big, big + extent, n),
                  rng.integers(big, big + extent, n), rng.integers(big, big + extent, n)], axis=1).astype(np.int32)
    c = np.unique(c, axis=0)
    return np.ascontiguousarray(c[rng.permutation(c.shape[0])])


def check_map(be, fine, fmap, cmap):
    rc, ec, ep, es = orc.s2c_map(fine)
    assert rc == 0
    assert cmap.n == ec.shape[0] and fmap.n == fine.shape[0]
    assert np.array_equal(be.download_c2s_coords(cmap), ec)
    c, p, s = be.download_c2s_map(fmap)
    assert np.array_equal(c, fine) and np.array_equal(p, ep) and np.array_equal(s, es)
    return ec, ep, es


def test_s2c_known_answer(backends):
    be = backends[sh.F32]
    coords, feats, ec, ep, es, ech = kat()
    fmap, cmap = be.s2c_build_device(coords)
    assert cmap.n == 3
    assert np.array_equal(be.download_c2s_coords(cmap), ec)
    c, p, s = be.download_c2s_map(fmap)
    assert np.array_equal(c, coords) and np.array_equal(p, ep) and np.array_equal(s, es)
    x = be.upload(feats)
    y = be.alloc(3 * 8)
    be.s2c_skip_mean_device(x, fmap, y, 2, 8)
    assert np.array_equal(be.download(y).reshape(3, 8), ech)


@pytest.mark.parametrize("n,extent,batches,big", [
    (1, 4, 1, 0), (5, 3, 1, 0), (2047, 40, 2, 0), (2048, 40, 2, 0), (2049, 40, 2, 0),
    (100_000, 120, 4, 0), (30_000, 200, 3, 1_000_000_000), (20_000, 60, 1, 70_000),
])
def test_s2c_map_vs_oracle(backends, n, extent, batches, big):
    """Ragged tile edges, several batches, and coordinates above 2^16 and near
    2^30 (a key wider than 64 bits)."""
    be = backends[sh.BF16]
    rng = np.random.default_rng(n + extent)
    fine = random_fine_set(rng, n, extent, batches, big)
    if big >= 1_000_000_000:
        fine[:, 0] = rng.integers(0, 1 << 20, fine.shape[0])  # wide batch field too
        fine = np.unique(fine, axis=0)[rng.permutation(np.unique(fine, axis=0).shape[0])]
        fine = np.ascontiguousarray(fine)
    say(f"s2c map n={fine.shape[0]} extent={extent} batches={batches} big={big}")
    fmap, cmap = be.s2c_build_device(fine)
    check_map(be, fine, fmap, cmap)
    be.free_map(fmap)
    be.free_map(cmap)


def test_s2c_from_device_coords_and_rejects(backends):
    be = backends[sh.F16]
    rng = np.random.default_rng(9)
    fine = random_fine_set(rng, 5000, 50, 2)
    src = be.upload_coords(fine)
    fmap, cmap = be.s2c_build_device(coords_map=src)
    check_map(be, fine, fmap, cmap)
    with pytest.raises(sh.HipError) as ei:
        be.s2c_build_device(np.array([[0, 1, 2, 3], [0, 4, -1, 4]], np.int32))
    assert ei.value.status == sh.INVALID_ARGUMENT  # s2c_host.c:61-67
    # The same fine voxel twice, next to each other in row order ...
    with pytest.raises(sh.HipError) as ei:
        be.s2c_build_device(np.array([[0, 1, 2, 3], [0, 1, 2, 3], [0, 8, 8, 8]], np.int32))
    assert ei.value.status == sh.PARSE_ERROR  # s2c_host.c:80-88
    # ... and with another child of the same coarse voxel between the two rows.
    with pytest.raises(sh.HipError) as ei:
        be.s2c_build_device(np.array([[0, 0, 0, 0], [0, 1, 0, 0], [0, 0, 0, 0]], np.int32))
    assert ei.value.status == sh.PARSE_ERROR
    fmap2, cmap2 = be.s2c_build_device(fine)  # still usable after the errors
    check_map(be, fine, fmap2, cmap2)


def test_s2c_repeat_found_at_any_distance(backends):
    """A repeated fine voxel is a parse error wherever the repeat sits.  The
    build compares each row with the up to 8 rows before it in its coarse
    voxel (in input order); of any 9 rows of one coarse voxel two share a
    child slot, so that finds every repeat.  Cases: all eight children of one
    coarse voxel between the two rows, with rows of other coarse voxels
    interleaved (the repeat is then exactly 8 rows back in its coarse voxel),
    a coarse voxel with two repeats, and random sets with one row repeated at
    a random later position; a set without repeats still builds."""
    be = backends[sh.BF16]
    children = [[0, x, y, z] for x in (2, 3) for y in (4, 5) for z in (6, 7)]
    others = [[0, 10 + 2 * i, 0, 0] for i in range(8)]
    rows = []
    for c, o in zip(children, others):
        rows += [c, o]
    rows.append(children[0])
    with pytest.raises(sh.HipError) as ei:
        be.s2c_build_device(np.array(rows, np.int32))
    assert ei.value.status == sh.PARSE_ERROR
    rows2 = children + [children[5], children[2]]
    with pytest.raises(sh.HipError) as ei:
        be.s2c_build_device(np.array(rows2, np.int32))
    assert ei.value.status == sh.PARSE_ERROR
    rng = np.random.default_rng(123)
    for trial in range(12):
        fine = random_fine_set(rng, int(rng.integers(20, 3000)), int(rng.integers(3, 12)), 2)
        i = int(rng.integers(0, len(fine)))
        j = int(rng.integers(i + 1, len(fine) + 1))
        dup = np.ascontiguousarray(np.insert(fine, j, fine[i], axis=0))
        with pytest.raises(sh.HipError) as ei:
            be.s2c_build_device(dup)
        assert ei.value.status == sh.PARSE_ERROR, (trial, len(fine), i, j)
        fmap, cmap = be.s2c_build_device(fine)
        check_map(be, fine, fmap, cmap)


@pytest.mark.parametrize("dtype", [sh.F32, sh.F16, sh.BF16])
@pytest.mark.parametrize("ci,co", [(2, 8), (64, 128), (128, 256), (96, 64), (256, 16)])
def test_s2c_pack_and_skip_mean_vs_oracle(backends, dtype, ci, co):
    be = backends[dtype]
    rnd = lambda a: sh.storage_round(a, dtype)
    rng = np.random.default_rng(ci * 7 + co + dtype)
    fine = random_fine_set(rng, 6000, 30, 2)
    n = fine.shape[0]
    say(f"s2c pack/skip dtype={dtype} ci={ci} co={co} n={n}")
    fmap, cmap = be.s2c_build_device(fine)
    ec, ep, es = check_map(be, fine, fmap, cmap)
    m = cmap.n
    pc = co // 8
    conv1 = rnd(rng.standard_normal((n, pc)))
    h = rnd(rng.standard_normal((n, ci)))
    packed, skip = be.alloc(m * co), be.alloc(m * co)
    be.s2c_pack_device(be.upload(conv1), fmap, packed, co)
    be.s2c_skip_mean_device(be.upload(h), fmap, skip, ci, co)
    assert np.array_equal(be.download(packed).reshape(m, co), rnd(orc.s2c_pack(conv1, ep, es, m, co)))
    assert np.array_equal(be.download(skip).reshape(m, co), rnd(orc.s2c_skip_mean(h, ep, es, m, ci, co)))
    # The fine map is the decoder's guide: c2s_gather of the packed rows returns them.
    back = be.alloc(n * pc)
    be.c2s_gather_device(packed, fmap, back, pc)
    assert np.array_equal(be.download(back).reshape(n, pc), conv1)
    be.free_map(fmap)
    be.free_map(cmap)


def test_s2c_of_config3_children_returns_parents(backends):
    """Config-3 scale: the S2C of the ~1.26M subdivided children (rows
    shuffled) gives back the parents that kept a child, in order, with each
    child's parent and slot; checked against the oracle as well."""
    be = backends[sh.BF16]
    w = wl.workload(3)
    parents = w["parent_coords"]
    rc, children, cpar, csub = orc.c2s_map(parents, w["logits"])
    assert rc == 0
    perm = np.random.default_rng(3).permutation(children.shape[0])
    fine = np.ascontiguousarray(children[perm])
    say(f"s2c config-3 children n={fine.shape[0]}")
    fmap, cmap = be.s2c_build_device(fine)
    ec, ep, es = check_map(be, fine, fmap, cmap)
    kept = np.unique(cpar)
    assert np.array_equal(ec, parents[kept])
    assert np.array_equal(kept[ep], cpar[perm]) and np.array_equal(es, csub[perm])
    be.free_map(fmap)
    be.free_map(cmap)
