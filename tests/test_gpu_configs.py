"""GPU parity of the convs at the benchmark configurations' own sizes, and of
the deep-channel schedules (a 128-pair unit spanning several blocks of K
steps).

At full size the oracle (trellis_sparse_cpu.c:324-373 restated) runs on a
strided sample of output rows, from the same rounded inputs the backend
reads; the sampled rows are compared to the storage tolerance of
tests/test_sparse_decoder_backend.c:16-24 (|a-b| <= 2e-2 max(1,|a|,|b|)).
For configs 4 and 5 the stride is 255 rows plus the last row, so every
256-row map tile (the kernels' unit of work) holds at least one sampled row,
including the last, partial tile, and the sampled positions within a tile
cycle through all 256 (both half tiles of the 256-channel blocks).

  config 2  conv(128->128) -> LayerNorm -> SiLU -> conv(128->128) + skip, fp16,
            419,340 voxels: each fused launch against the oracle, the second
            from the backend's own intermediate rows
  config 4  conv 64->64 bf16 on the 3,788,747-voxel R=1024 shell set
  config 5  conv 512->512 bf16 on the four batched structures (327,680 voxels)

The deep-channel cases include the decoder's own widths
(sparse_unet_decoder/decoder.c:248-249, the C2S conv Ci -> 8 Co of
executor.c:456): 1024 -> 1024 (the level-0 ConvNeXt conv), 512 -> 2048 and
1024 -> 4096 (levels 1 and 0 of the upsample).  They run Ci = 384, 512 and
1024 with 64- and 128-channel output blocks on ragged row counts: with Ci >= 512 (or Ci = 384) one unit of
128 pairs takes more than one block of 8 (or 4) K steps, so the kernels'
mid-unit block prefetch is executed.  Co % 256 == 0 (with Ci % 128 == 0) runs
256-channel blocks over half map tiles: those cases include a last tile whose
second half is short (900 and 1500 rows) or empty (1300 and 600 rows), and a
single 200-row tile.
"""
import math
import sys

import numpy as np
import pytest

import oracle_lib as orc
import sparse_hip as sh
import workloads as wl

pytestmark = pytest.mark.gpu

TOL = {sh.F16: 2e-2, sh.BF16: 2e-2}


def say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def max_rel_err(got, exp):
    got = np.asarray(got, dtype=np.float64).ravel()
    exp = np.asarray(exp, dtype=np.float64).ravel()
    assert got.shape == exp.shape
    scale = np.maximum(1.0, np.maximum(np.abs(got), np.abs(exp)))
    return float(np.max(np.abs(got - exp) / scale)) if got.size else 0.0


@pytest.fixture(scope="module")
def backends():
    bes = {dt: sh.Backend(0, dt) for dt in (sh.F16, sh.BF16)}
    yield bes
    for b in bes.values():
        b.destroy()


def sample_rows(n, want):
    step = max(1, n // want)
    return (min(3, n - 1), n, step)


@pytest.mark.parametrize("cfg", [4, 5])
def test_config_conv_full_size_vs_oracle_sample(backends, cfg):
    be = backends[sh.BF16]
    w = wl.workload(cfg)
    coords, ci, co = w["coords"], w["ci"], w["co"]
    n = coords.shape[0]
    x = sh.bf16_round(w["feats"])
    wr = sh.bf16_round(w["weight"])
    rng = np.random.default_rng(cfg)
    bias = (0.1 * rng.standard_normal(co)).astype(np.float32)
    say(f"cfg{cfg} full conv {ci}->{co} bf16 n={n}")
    rb = be.build_rulebook(coords)
    stats = be.rulebook_stats(rb)
    xb, yb = be.upload(x), be.alloc(n * co)
    be.conv(rb, xb, w["weight"], bias, yb, ci, co)
    got = be.download(yb).reshape(n, co)
    del xb, yb
    assert np.all(np.isfinite(got))
    # One row in every 255: each 256-row tile holds a sampled row, at a
    # position that moves by one per tile; plus the last row.
    rows = (3, n, 255)
    orb = orc.Rulebook(coords)
    exp = orb.conv(x, wr, bias, ci, co, rows=rows)
    err = max_rel_err(got[rows[0]:rows[1]:rows[2]], exp)
    exp_last = orb.conv(x, wr, bias, ci, co, rows=(n - 1, n, 1))
    err = max(err, max_rel_err(got[n - 1:n], exp_last))
    tiles = (n + 255) // 256
    sampled_tiles = np.unique(np.concatenate([np.arange(rows[0], n, rows[2]), [n - 1]]) // 256)
    assert sampled_tiles.size == tiles
    say(f"cfg{cfg} full conv pairs={stats['pairs']} sampled rows={exp.shape[0] + 1} of {tiles} tiles "
        f"max_rel_err={err:.3e}")
    assert err <= 2e-2
    rb.free()


def test_config2_fused_block_full_size_vs_oracle_sample(backends):
    """Config 2 at full size: conv_norm (SiLU) and conv_add, each checked on a
    row sample against the oracle's conv -> round -> row_norm_silu -> round
    and conv -> round -> add -> round, the second from the backend's own
    intermediate (already in the storage type)."""
    dtype = sh.F16
    be = backends[dtype]
    rnd = lambda a: sh.storage_round(a, dtype)
    w = wl.workload(2)
    coords, c = w["coords"], 128
    n = coords.shape[0]
    x = rnd(w["feats"])
    w1, w2 = rnd(w["weight"]), rnd(w["weight2"])
    rng = np.random.default_rng(22)
    b1 = (0.1 * rng.standard_normal(c)).astype(np.float32)
    b2 = (0.1 * rng.standard_normal(c)).astype(np.float32)
    gamma = (1 + 0.1 * rng.standard_normal(c)).astype(np.float32)
    beta = (0.1 * rng.standard_normal(c)).astype(np.float32)
    say(f"cfg2 fused block fp16 n={n}")
    rb = be.build_rulebook(coords)
    xb, hb, ob = be.upload(x), be.alloc(n * c), be.alloc(n * c)
    be.conv_norm(rb, xb, w1, b1, gamma, beta, 1e-6, hb, c, c, silu=True)
    be.conv_add(rb, hb, w2, b2, xb, ob, c, c)
    h = be.download(hb).reshape(n, c)
    out = be.download(ob).reshape(n, c)
    rows = sample_rows(n, 4000)
    sl = slice(rows[0], rows[1], rows[2])
    orb = orc.Rulebook(coords)
    e_conv1 = rnd(orb.conv(x, w1, b1, c, c, rows=rows))
    e_h = rnd(orc.row_norm(e_conv1, gamma, beta, e_conv1.shape[0], c, 1e-6, silu=True))
    err_h = max_rel_err(h[sl], e_h)
    e_out = rnd(orc.add(rnd(orb.conv(h, w2, b2, c, c, rows=rows)), x[sl]))
    err_o = max_rel_err(out[sl], e_out)
    say(f"cfg2 fused block sampled rows={e_h.shape[0]} err_conv_norm={err_h:.3e} err_conv_add={err_o:.3e}")
    assert err_h <= TOL[dtype]
    assert err_o <= TOL[dtype]
    rb.free()


DEEP_CASES = [(512, 128, 3001), (384, 128, 2000), (1024, 128, 1200), (512, 64, 2500), (1024, 64, 1777),
              (512, 512, 1300), (128, 256, 900), (256, 1024, 600), (384, 256, 1500), (256, 256, 200),
              (1024, 1024, 700), (512, 2048, 650), (1024, 4096, 520)]


@pytest.mark.parametrize("dtype", [sh.BF16, sh.F16])
@pytest.mark.parametrize("ci,co,n", DEEP_CASES)
def test_conv_deep_channels_vs_oracle(backends, dtype, ci, co, n):
    be = backends[dtype]
    coords = np.ascontiguousarray(wl.make_coords(1)[:n])
    rng = np.random.default_rng(ci + 3 * co + n + dtype)
    x = sh.storage_round(rng.standard_normal((n, ci)), dtype)
    w = sh.storage_round(rng.standard_normal((co, 27, ci)) / math.sqrt(27 * ci), dtype)
    bias = (0.1 * rng.standard_normal(co)).astype(np.float32)
    say(f"deep conv dtype={dtype} ci={ci} co={co} n={n}")
    rb = be.build_rulebook(coords)
    xb, yb = be.upload(x), be.alloc(n * co)
    be.conv(rb, xb, w, bias, yb, ci, co)
    got = be.download(yb).reshape(n, co)
    rows = sample_rows(n, 400 if ci * co <= 512 * 1024 else 120)
    exp = orc.Rulebook(coords).conv(x, w, bias, ci, co, rows=rows)
    err = max_rel_err(got[rows[0]:rows[1]:rows[2]], exp)
    say(f"deep conv dtype={dtype} ci={ci} co={co} n={n} rows={exp.shape[0]} max_rel_err={err:.3e}")
    assert err <= TOL[dtype]
    # Fused epilogues on the multi-block path (128-channel blocks only).
    if co % 128 == 0:
        res = sh.storage_round(rng.standard_normal((n, co)), dtype)
        rs = be.upload(res)
        be.conv_add(rb, xb, w, bias, rs, yb, ci, co)
        got_add = be.download(yb).reshape(n, co)
        e_add = sh.storage_round(orc.add(sh.storage_round(exp, dtype), res[rows[0]:rows[1]:rows[2]]), dtype)
        err_add = max_rel_err(got_add[rows[0]:rows[1]:rows[2]], e_add)
        say(f"deep conv_add dtype={dtype} ci={ci} co={co} max_rel_err={err_add:.3e}")
        assert err_add <= TOL[dtype]
    if co == 128:
        gamma = (1 + 0.1 * rng.standard_normal(co)).astype(np.float32)
        beta = (0.1 * rng.standard_normal(co)).astype(np.float32)
        be.conv_norm(rb, xb, w, bias, gamma, beta, 1e-6, yb, ci, co, silu=True)
        got_n = be.download(yb).reshape(n, co)
        e_n = sh.storage_round(orc.row_norm(sh.storage_round(exp, dtype), gamma, beta, exp.shape[0], co, 1e-6,
                                            silu=True), dtype)
        err_n = max_rel_err(got_n[rows[0]:rows[1]:rows[2]], e_n)
        say(f"deep conv_norm dtype={dtype} ci={ci} max_rel_err={err_n:.3e}")
        assert err_n <= TOL[dtype]
    rb.free()


def mixed_density_sets(rng):
    """A solid 12^3 box and, far from it, a 40^3 region filled at 30 %.  Of
    the map tiles' offsets with pairs, 9 in 10 have more than 128 in the box
    (Co % 256 == 0 takes the 256-column layout there), 1 in 27 in the sparse
    part and 1 in 8 in the union (the 128-column layout)."""
    g = np.stack(np.meshgrid(*(np.arange(12),) * 3, indexing="ij"), -1).reshape(-1, 3)
    box = np.concatenate([np.zeros((g.shape[0], 1), np.int64), g], 1)
    pts = rng.integers(0, 40, (int(0.3 * 40 ** 3), 3)) + 100
    sparse = np.unique(np.concatenate([np.zeros((pts.shape[0], 1), np.int64), pts], 1), axis=0)
    sparse = sparse[rng.permutation(sparse.shape[0])]
    return np.ascontiguousarray(box.astype(np.int32)), np.ascontiguousarray(sparse.astype(np.int32))


@pytest.mark.parametrize("dtype", [sh.BF16, sh.F16])
@pytest.mark.parametrize("ci,co", [(128, 256), (256, 512), (512, 256), (256, 1024), (512, 2048)])
def test_conv_layouts_bitexact(backends, dtype, ci, co):
    """Co % 256 == 0 runs the 256-column layout on dense sets and the
    128-column one on sparse sets (the kernel map's statistics decide).  The
    box alone takes the first, the union of box and sparse part the second:
    the union's rows must equal, bit for bit, the same rows computed from
    each part alone (a row's sums are formed in the same order in both
    layouts, and the parts are too far apart to be neighbours), with and
    without the residual epilogue (in place), and match the oracle on a
    sample."""
    be = backends[dtype]
    rng = np.random.default_rng(ci + co)
    box, sparse = mixed_density_sets(rng)
    both = np.ascontiguousarray(np.concatenate([box, sparse]))
    nb, n = box.shape[0], both.shape[0]
    x = sh.storage_round(rng.standard_normal((n, ci)), dtype)
    w = sh.storage_round(rng.standard_normal((co, 27, ci)) / math.sqrt(27 * ci), dtype)
    bias = (0.1 * rng.standard_normal(co)).astype(np.float32)
    res = sh.storage_round(rng.standard_normal((n, co)), dtype)
    say(f"conv layouts dtype={dtype} ci={ci} co={co} box={nb} sparse={n - nb}")

    def run(coords, xs, rs):
        rb = be.build_rulebook(coords)
        m = coords.shape[0]
        xb, yb = be.upload(xs), be.alloc(m * co)
        be.conv(rb, xb, w, bias, yb, ci, co)
        plain = be.download(yb).reshape(m, co)
        r = be.upload(rs)
        be.conv_add(rb, xb, w, bias, r, r, ci, co)  # in place: the output overwrites the residual
        added = be.download(r).reshape(m, co)
        rb.free()
        return plain, added

    p_all, a_all = run(both, x, res)
    p_box, a_box = run(box, x[:nb], res[:nb])
    p_sp, a_sp = run(sparse, x[nb:], res[nb:])
    assert np.array_equal(p_all[:nb], p_box) and np.array_equal(p_all[nb:], p_sp)
    assert np.array_equal(a_all[:nb], a_box) and np.array_equal(a_all[nb:], a_sp)
    rows = sample_rows(n, 300)
    exp = orc.Rulebook(both).conv(x, w, bias, ci, co, rows=rows)
    err = max_rel_err(p_all[rows[0]:rows[1]:rows[2]], exp)
    e_add = sh.storage_round(orc.add(sh.storage_round(exp, dtype), res[rows[0]:rows[1]:rows[2]]), dtype)
    err_add = max_rel_err(a_all[rows[0]:rows[1]:rows[2]], e_add)
    say(f"conv layouts ci={ci} co={co} max_rel_err={err:.3e} add={err_add:.3e}")
    assert err <= TOL[dtype] and err_add <= TOL[dtype]


@pytest.mark.parametrize("dtype", [sh.BF16, sh.F16])
@pytest.mark.parametrize("n", [1, 2, 127, 129, 257])
@pytest.mark.parametrize("ci,co", [(256, 512), (128, 256), (512, 256)])
def test_conv_wide_outputs_tiny_sets(backends, dtype, n, ci, co):
    """Co % 256 == 0 on sets of one to two map tiles (a single voxel, a short
    second half tile, one row past a tile), with the plain and the in-place
    residual epilogue, against the oracle on every row."""
    be = backends[dtype]
    g = np.stack(np.meshgrid(*(np.arange(7),) * 3, indexing="ij"), -1).reshape(-1, 3)[:n]
    coords = np.ascontiguousarray(np.concatenate([np.zeros((n, 1), np.int64), g], 1).astype(np.int32))
    rng = np.random.default_rng(n * 3 + ci + co + dtype)
    x = sh.storage_round(rng.standard_normal((n, ci)), dtype)
    w = sh.storage_round(rng.standard_normal((co, 27, ci)) / math.sqrt(27 * ci), dtype)
    bias = (0.1 * rng.standard_normal(co)).astype(np.float32)
    res = sh.storage_round(rng.standard_normal((n, co)), dtype)
    rb = be.build_rulebook(coords)
    xb, yb = be.upload(x), be.alloc(n * co)
    be.conv(rb, xb, w, bias, yb, ci, co)
    exp = orc.Rulebook(coords).conv(x, w, bias, ci, co)
    assert max_rel_err(be.download(yb).reshape(n, co), exp) <= TOL[dtype]
    r = be.upload(res)
    be.conv_add(rb, xb, w, bias, r, r, ci, co)
    e_add = sh.storage_round(orc.add(sh.storage_round(exp, dtype), res), dtype)
    assert max_rel_err(be.download(r).reshape(n, co), e_add) <= TOL[dtype]
    rb.free()


def decoder_level_set(levels):
    """The decoder's voxel sets: the config-3 parent shell reduced to R = 64,
    subdivided `levels` times with seeded random logits (about half the
    children kept), as `bench.py --decoder` builds them; 7-11 neighbours per
    voxel, the sparse sets that take the 128-column conv layout."""
    pc = wl.workload(3)["parent_coords"].copy()
    pc[:, 1:] >>= 2
    cur = np.ascontiguousarray(np.unique(pc, axis=0), dtype=np.int32)
    rng = np.random.default_rng(41)
    for _ in range(levels):
        rc, cur, _, _ = orc.c2s_map(cur, rng.standard_normal((cur.shape[0], 8)).astype(np.float32))
        assert rc == 0
    return np.ascontiguousarray(cur, dtype=np.int32)


@pytest.mark.parametrize("levels,ci,co", [(1, 512, 512), (1, 512, 2048), (2, 256, 256), (2, 256, 1024), (3, 128, 512)])
def test_conv_decoder_levels_vs_oracle(backends, levels, ci, co):
    """The decoder's sparse levels at their real size and widths (the
    ConvNeXt convs and the up-blocks' Ci -> 8 Co convs), bf16, against the
    oracle on a strided sample that puts a row in every 256-row map tile."""
    be = backends[sh.BF16]
    coords = decoder_level_set(levels)
    n = coords.shape[0]
    rng = np.random.default_rng(levels * 1000 + ci + co)
    x = sh.storage_round(rng.standard_normal((n, ci)), sh.BF16)
    w = sh.storage_round(rng.standard_normal((co, 27, ci)) / math.sqrt(27 * ci), sh.BF16)
    bias = (0.1 * rng.standard_normal(co)).astype(np.float32)
    say(f"decoder level {levels} conv {ci}->{co} n={n}")
    rb = be.build_rulebook(coords)
    xb, yb = be.upload(x), be.alloc(n * co)
    be.conv(rb, xb, w, bias, yb, ci, co)
    got = be.download(yb).reshape(n, co)
    rows = (5, n, 255)
    exp = orc.Rulebook(coords).conv(x, w, bias, ci, co, rows=rows)
    err = max_rel_err(got[rows[0]:rows[1]:rows[2]], exp)
    say(f"decoder level {levels} conv {ci}->{co} rows={exp.shape[0]} max_rel_err={err:.3e}")
    assert err <= TOL[sh.BF16]
    rb.free()


_ENCODER_SETS = {}


def encoder_level_set(level):
    """The encoder's voxel sets: the config-4 shells (R = 1024) and their S2C
    coarsenings, as `bench.py --encoder` builds them (13-16 neighbours per
    voxel below the input level)."""
    if not _ENCODER_SETS:
        cur = np.ascontiguousarray(wl.make_coords(4), dtype=np.int32)
        _ENCODER_SETS[0] = cur
        for lv in range(1, 5):
            rc, cur, _, _ = orc.s2c_map(cur)
            assert rc == 0
            _ENCODER_SETS[lv] = np.ascontiguousarray(cur, dtype=np.int32)
    return _ENCODER_SETS[level]


@pytest.mark.parametrize("level,ci,co", [(0, 64, 16), (1, 128, 32), (2, 256, 256), (3, 512, 512), (3, 512, 128),
                                         (4, 1024, 1024)])
def test_conv_encoder_levels_vs_oracle(backends, level, ci, co):
    """The encoder's levels at their real size and widths (the ConvNeXt convs
    and the down-blocks' Ci -> Co / 8 convs), bf16, against the oracle on a
    strided sample that puts a row in every 256-row map tile."""
    be = backends[sh.BF16]
    coords = encoder_level_set(level)
    n = coords.shape[0]
    rng = np.random.default_rng(level * 1000 + ci + co)
    x = sh.storage_round(rng.standard_normal((n, ci)), sh.BF16)
    w = sh.storage_round(rng.standard_normal((co, 27, ci)) / math.sqrt(27 * ci), sh.BF16)
    bias = (0.1 * rng.standard_normal(co)).astype(np.float32)
    say(f"encoder level {level} conv {ci}->{co} n={n}")
    rb = be.build_rulebook(coords)
    xb, yb = be.upload(x), be.alloc(n * co)
    be.conv(rb, xb, w, bias, yb, ci, co)
    got = be.download(yb).reshape(n, co)
    rows = (7, n, 255)
    exp = orc.Rulebook(coords).conv(x, w, bias, ci, co, rows=rows)
    err = max_rel_err(got[rows[0]:rows[1]:rows[2]], exp)
    say(f"encoder level {level} conv {ci}->{co} rows={exp.shape[0]} max_rel_err={err:.3e}")
    assert err <= TOL[sh.BF16]
    rb.free()


@pytest.mark.parametrize("ci,co,n", [(512, 128, 2100), (384, 64, 1500)])
def test_conv_deep_channels_masked_vs_oracle(ci, co, n):
    """The masked schedule on the same deep shapes (it walks K in 32-channel
    steps per offset; no unit blocks)."""
    be = sh.Backend(0, sh.BF16, conv_algo=sh.CONV_MASKED)
    try:
        coords = np.ascontiguousarray(wl.make_coords(1)[:n])
        rng = np.random.default_rng(ci * 5 + co + n)
        x = sh.bf16_round(rng.standard_normal((n, ci)))
        w = sh.bf16_round(rng.standard_normal((co, 27, ci)) / math.sqrt(27 * ci))
        rb = be.build_rulebook(coords)
        xb, yb = be.upload(x), be.alloc(n * co)
        be.conv(rb, xb, w, None, yb, ci, co)
        got = be.download(yb).reshape(n, co)
        rows = sample_rows(n, 300)
        exp = orc.Rulebook(coords).conv(x, w, None, ci, co, rows=rows)
        err = max_rel_err(got[rows[0]:rows[1]:rows[2]], exp)
        say(f"deep masked ci={ci} co={co} n={n} max_rel_err={err:.3e}")
        assert err <= 2e-2
        rb.free()
    finally:
        be.destroy()
