"""GPU parity: the HIP backend through the C ABI vs the CPU oracle.

Bar: bit-exact for neighbour tables, pair lists, subdivide maps and copies;
fp32 conv within 1e-5 (and checked bit-exact against the reference operation
order); bf16/fp16 within 2e-2 with the oracle run on the same rounded inputs.
Error measure: check_close of tests/test_sparse_decoder_backend.c:16-24,
|a-b| <= tol * max(1, |a|, |b|).
"""
import math
import sys

import numpy as np
import pytest

import oracle_lib as orc
import sparse_hip as sh
import workloads as wl

pytestmark = pytest.mark.gpu

TOL = {sh.F32: 1e-5, sh.F16: 2e-2, sh.BF16: 2e-2}


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
def be32():
    b = sh.Backend(0, sh.F32)
    yield b
    b.destroy()


@pytest.fixture(scope="module")
def be16():
    b = sh.Backend(0, sh.F16)
    yield b
    b.destroy()


@pytest.fixture(scope="module")
def bebf():
    b = sh.Backend(0, sh.BF16)
    yield b
    b.destroy()


def backend_for(dtype, be32, be16, bebf):
    return {sh.F32: be32, sh.F16: be16, sh.BF16: bebf}[dtype]


@pytest.fixture(scope="module")
def kernel_linears():
    """16-bit backends whose linear slots always run this library's kernels
    (policy linear_algo = KERNEL), beside the default ones that send wide
    shapes to the platform GEMM library."""
    bes = {dt: sh.Backend(0, dt, linear_algo=sh.LINEAR_KERNEL) for dt in (sh.F16, sh.BF16)}
    yield bes
    for b in bes.values():
        b.destroy()


# ------------------------------------------------------------ hash / kernel map

def edge_coord_sets():
    rng = np.random.default_rng(11)
    dup = np.stack([rng.integers(0, 2, 700), rng.integers(-3, 9, 700), rng.integers(-3, 9, 700),
                    rng.integers(-3, 9, 700)], 1).astype(np.int32)
    dup[-40:] = dup[:40]  # later duplicates win
    wrap = np.array([[0, 0, 5, 5], [0, 65535, 5, 5], [0, 1, 5, 5], [3, 65535, 65535, 65535], [3, 0, 0, 0]], np.int32)
    single = np.array([[7, 100, 200, 300]], np.int32)
    ragged = wl.make_coords(1)[:1000 + 37]
    batches = wl.make_coords(5)[::7]
    return {"duplicates": dup, "wrap": wrap, "single": single, "ragged": ragged, "batches": batches}


@pytest.mark.parametrize("name", ["duplicates", "wrap", "single", "ragged", "batches"])
def test_kernel_map_edge_cases_bitexact(be32, name):
    c = edge_coord_sets()[name]
    say(f"kernel map edge case {name}: n={c.shape[0]}")
    rb = be32.build_rulebook(c)
    exp = orc.Rulebook(c).neighbors()
    got = be32.neighbors(rb)
    assert np.array_equal(got, exp)
    counts, src, dst = be32.pairs(rb)
    ec, es, ed = orc.pairs(exp)
    assert np.array_equal(counts, ec) and np.array_equal(src, es) and np.array_equal(dst, ed)
    rb.free()


@pytest.mark.parametrize("cfg", [1, 2, 4, 5])
def test_kernel_map_configs_bitexact(be32, cfg):
    c = wl.make_coords(cfg)
    say(f"kernel map cfg{cfg}: n={c.shape[0]}")
    rb = be32.build_rulebook(c)
    stats = be32.rulebook_stats(rb)
    exp = orc.Rulebook(c).neighbors()
    assert stats["pairs"] == int((exp >= 0).sum())
    if cfg == 1:
        assert stats["pairs"] == 261416
    assert np.array_equal(be32.neighbors(rb), exp)
    counts, src, dst = be32.pairs(rb)
    ec, es, ed = orc.pairs(exp)
    assert np.array_equal(counts, ec) and np.array_equal(src, es) and np.array_equal(dst, ed)
    rb.free()


def random_coord_set(seed):
    """Seeded random voxel sets of varied shape: uniform boxes from dense to
    sparse, Gaussian clusters, sets straddling the 16-bit wrap of every axis,
    many batches with large batch ids, and repeated coordinates."""
    rng = np.random.default_rng(1000 + seed)
    kind = seed % 5
    n = int(rng.integers(1, 60000))
    if kind == 0:  # uniform box, density from ~1 to ~0.001
        side = int(max(2, round((n / rng.uniform(0.001, 1.0)) ** (1 / 3))))
        c = np.stack([np.zeros(n), *(rng.integers(0, side, n) for _ in range(3))], 1)
    elif kind == 1:  # clusters
        centres = rng.integers(0, 3000, (int(rng.integers(1, 40)), 3))
        pick = rng.integers(0, centres.shape[0], n)
        pts = centres[pick] + rng.normal(0, rng.uniform(1, 12), (n, 3))
        c = np.concatenate([rng.integers(0, 3, (n, 1)), np.rint(pts)], 1)
    elif kind == 2:  # around the 16-bit wrap on every axis
        c = np.stack([rng.integers(0, 2, n), *(rng.integers(-9, 9, n) for _ in range(3))], 1)
        c[:, 1:][c[:, 1:] < 0] += 65536
    elif kind == 3:  # many batches, large batch ids
        c = np.stack([rng.integers(60000, 65536, n), *(rng.integers(0, 20, n) for _ in range(3))], 1)
    else:  # repeated rows among a small set
        base = np.stack([rng.integers(0, 4, n), *(rng.integers(0, 24, n) for _ in range(3))], 1)
        c = base[rng.integers(0, base.shape[0], n)]
    return np.ascontiguousarray(c.astype(np.int32))


@pytest.mark.parametrize("seed", list(range(15)))
def test_kernel_map_random_sets_bitexact(be32, bebf, seed):
    """Neighbour table and pair lists equal the oracle's on seeded random
    sets, on an fp32 backend (the neighbour table) and a bf16 one (the
    compact lists the MFMA convs read)."""
    c = random_coord_set(seed)
    say(f"kernel map random set seed={seed} kind={seed % 5}: n={c.shape[0]}")
    exp = orc.Rulebook(c).neighbors()
    ec, es, ed = orc.pairs(exp)
    rb = be32.build_rulebook(c)
    assert np.array_equal(be32.neighbors(rb), exp)
    rb.free()
    rb = bebf.build_rulebook(c)
    counts, src, dst = bebf.pairs(rb)
    assert np.array_equal(counts, ec) and np.array_equal(src, es) and np.array_equal(dst, ed)
    rb.free()


def test_rulebook_rejects_bad_arguments(be32):
    with pytest.raises(sh.HipError) as e:
        be32.build_rulebook(np.zeros((0, 4), np.int32))
    assert e.value.status == sh.INVALID_ARGUMENT


@pytest.mark.parametrize("name", ["duplicates", "wrap", "single", "ragged", "batches"])
@pytest.mark.parametrize("ci,co", [(128, 128), (256, 128), (64, 64)])
def test_compact_conv_edge_cases_vs_oracle(be_sched, name, ci, co):
    """The compacted conv on the map's edge cases.  Each tile starts with the
    centre offset's pairs, which with duplicate coordinates point at the last
    duplicate rather than the row itself; wrapped coordinates, a one-voxel
    input, a ragged last tile and several batches exercise the tile
    bookkeeping of both compacted kernels (128-channel and 64-channel blocks).
    Against the oracle's conv on the same rounded inputs, to the storage
    tolerance."""
    be = be_sched[("compact", sh.BF16)]
    c = edge_coord_sets()[name]
    n = c.shape[0]
    say(f"compact conv edge case {name}: n={n} ci={ci} co={co}")
    rng = np.random.default_rng(ci + co + n)
    x = sh.storage_round(rng.standard_normal((n, ci)), sh.BF16)
    w = sh.storage_round(rng.standard_normal((co, 27, ci)) / math.sqrt(27 * ci), sh.BF16)
    bias = (0.1 * rng.standard_normal(co)).astype(np.float32)
    got = run_conv(be, c, x, w, bias, ci, co)
    exp = orc.Rulebook(c).conv(x, w, bias, ci, co)
    err = max_rel_err(got, sh.storage_round(exp, sh.BF16))
    say(f"compact conv edge case {name} ci={ci} co={co} max_rel_err={err:.3e}")
    assert err <= 2e-2


def test_reject_duplicates_policy():
    b = sh.Backend(0, sh.F32, reject_duplicates=True)
    c = np.array([[0, 1, 1, 1], [0, 2, 2, 2], [0, 1, 1, 1]], np.int32)
    with pytest.raises(sh.HipError) as e:
        b.build_rulebook(c)
    assert e.value.status == sh.INVALID_ARGUMENT
    b.build_rulebook(c[:2]).free()
    b.destroy()


# ------------------------------------------------------------------------ conv

def run_conv(be, coords, feats, w, bias, ci, co):
    rb = be.build_rulebook(coords)
    x = be.upload(feats)
    y = be.alloc(coords.shape[0] * co)
    be.conv(rb, x, w, bias, y, ci, co)
    out = be.download(y).reshape(-1, co)
    rb.free()
    x.free()
    y.free()
    return out


def small_conv_cases():
    from test_oracle import reference_direct_case, reference_trellis_case

    return {"direct": reference_direct_case(), "trellis": reference_trellis_case()}


@pytest.mark.parametrize("name", ["direct", "trellis"])
def test_conv_fp32_reference_inputs(be32, name):
    coords, feats, w, bias, ci, co = small_conv_cases()[name]
    got = run_conv(be32, coords, feats, w, bias, ci, co)
    exp = orc.Rulebook(coords).conv(feats, w, bias, ci, co)
    assert max_rel_err(got, exp) <= 1e-5
    assert np.array_equal(got, exp), "fp32 generic path follows the reference operation order"


def test_conv_fp32_config1_full(be32):
    w = wl.workload(1)
    c, x, wt = w["coords"], w["feats"], w["weight"]
    rng = np.random.default_rng(1)
    bias = rng.standard_normal(64).astype(np.float32) * 0.1
    say(f"cfg1 fp32 conv n={c.shape[0]}")
    got = run_conv(be32, c, x, wt, bias, 64, 64)
    exp = orc.Rulebook(c).conv(x, wt, bias, 64, 64)
    err = max_rel_err(got, exp)
    say(f"cfg1 fp32 max_rel_err={err:.3e} bitexact={np.array_equal(got, exp)}")
    assert err <= 1e-5
    assert np.array_equal(got, exp)


SCHEDULES = {"masked": sh.CONV_MASKED, "compact": sh.CONV_COMPACT}


@pytest.fixture(scope="module")
def be_sched():
    """One backend per (MFMA schedule, storage type)."""
    b = {(name, dt): sh.Backend(0, dt, conv_algo=algo) for name, algo in SCHEDULES.items()
         for dt in (sh.BF16, sh.F16)}
    yield b
    for v in b.values():
        v.destroy()


@pytest.mark.parametrize("algo", ["compact", "masked"])
@pytest.mark.parametrize("dtype", [sh.BF16, sh.F16])
@pytest.mark.parametrize("ci,co", [(64, 64), (128, 128), (256, 128), (32, 192), (64, 512), (128, 256)])
def test_conv_mfma_vs_oracle(be_sched, algo, dtype, ci, co):
    be = be_sched[(algo, dtype)]
    c = wl.make_coords(1)
    rng = np.random.default_rng(ci + co + dtype)
    x = sh.storage_round(rng.standard_normal((c.shape[0], ci)).astype(np.float32), dtype)
    w = (rng.standard_normal((co, 27, ci)) / math.sqrt(27 * ci)).astype(np.float32)
    bias = rng.standard_normal(co).astype(np.float32) * 0.1
    wr = sh.storage_round(w, dtype)
    got = run_conv(be, c, x, w, bias, ci, co)
    exp = orc.Rulebook(c).conv(x, wr, bias, ci, co)
    err = max_rel_err(got, exp)
    say(f"mfma {algo} dtype={dtype} ci={ci} co={co} max_rel_err={err:.3e}")
    assert err <= TOL[dtype]


@pytest.mark.parametrize("algo", ["compact", "masked"])
def test_conv_mfma_dense_block_vs_torch(be_sched, algo):
    """Fully occupied block: every interior row has all 27 neighbours, so a
    256-row tile holds more than 128 pairs per offset (several units each)."""
    from test_oracle import dense_block, torch_dense_conv

    coords, feats, w, bias, side = dense_block(side=12, ci=64, co=64, seed=3)
    x = sh.bf16_round(feats)
    wr = sh.bf16_round(w)
    got = run_conv(be_sched[(algo, sh.BF16)], coords, x, w, bias, 64, 64)
    exp = torch_dense_conv(x, wr, bias, side)
    err = max_rel_err(got, exp)
    say(f"dense block bf16 {algo} vs torch conv3d max_rel_err={err:.3e}")
    assert err <= 2e-2


@pytest.mark.parametrize("algo", ["compact", "masked"])
@pytest.mark.parametrize("n", [1, 37, 300, 777])
def test_conv_mfma_ragged_rows(be_sched, algo, n):
    """Row counts that leave the last 64/256-row tile partly empty."""
    c = wl.make_coords(1)[:n]
    ci, co = 128, 64
    rng = np.random.default_rng(n)
    x = sh.bf16_round(rng.standard_normal((n, ci)).astype(np.float32))
    w = (rng.standard_normal((co, 27, ci)) / math.sqrt(27 * ci)).astype(np.float32)
    bias = rng.standard_normal(co).astype(np.float32)
    got = run_conv(be_sched[(algo, sh.BF16)], c, x, w, bias, ci, co)
    exp = orc.Rulebook(c).conv(x, sh.bf16_round(w), bias, ci, co)
    err = max_rel_err(got, exp)
    say(f"ragged {algo} n={n} max_rel_err={err:.3e}")
    assert err <= 2e-2


@pytest.mark.parametrize("algo", ["compact", "masked"])
@pytest.mark.parametrize("dtype", [sh.BF16, sh.F16])
@pytest.mark.parametrize("ci,co,n", [(64, 16, 14648), (128, 32, 14648), (256, 32, 5000), (32, 16, 300),
                                     (64, 16, 1), (64, 32, 129)])
def test_conv_narrow_output_vs_oracle(be_sched, algo, dtype, ci, co, n):
    """16 and 32 output channels (the encoder's S2C conv to co/8 channels):
    the compacted schedule with one 16/32-channel block (Ci = 64 or a
    multiple of 128; Ci = 32 falls back to the masked one) and the masked one
    with all four wavefronts on rows; ragged row counts and a single row."""
    be = be_sched[(algo, dtype)]
    c = wl.make_coords(1)[:n]
    rng = np.random.default_rng(ci * 3 + co + n + dtype)
    x = sh.storage_round(rng.standard_normal((c.shape[0], ci)).astype(np.float32), dtype)
    w = (rng.standard_normal((co, 27, ci)) / math.sqrt(27 * ci)).astype(np.float32)
    bias = rng.standard_normal(co).astype(np.float32) * 0.1
    got = run_conv(be, c, x, w, bias, ci, co)
    exp = orc.Rulebook(c).conv(x, sh.storage_round(w, dtype), bias, ci, co)
    err = max_rel_err(got, exp)
    say(f"narrow {algo} dtype={dtype} ci={ci} co={co} n={n} max_rel_err={err:.3e}")
    assert err <= TOL[dtype]


def test_conv_generic_small_channels_all_dtypes(be32, be16, bebf):
    coords, feats, w, bias, ci, co = small_conv_cases()["direct"]
    for dtype in (sh.F16, sh.BF16):
        be = backend_for(dtype, be32, be16, bebf)
        x = sh.storage_round(feats, dtype)
        got = run_conv(be, coords, x, w, bias, ci, co)
        exp = orc.Rulebook(coords).conv(x, w, bias, ci, co)
        assert max_rel_err(got, exp) <= TOL[dtype]


@pytest.mark.parametrize("algo", ["compact", "masked"])
def test_conv_deterministic(be_sched, algo):
    be = be_sched[(algo, sh.BF16)]
    c = wl.make_coords(1)
    rng = np.random.default_rng(4)
    x = rng.standard_normal((c.shape[0], 128)).astype(np.float32)
    w = (rng.standard_normal((128, 27, 128)) * 0.02).astype(np.float32)
    a = run_conv(be, c, x, w, None, 128, 128)
    b = run_conv(be, c, x, w, None, 128, 128)
    assert np.array_equal(a, b)


def test_conv_argument_errors(be32):
    c = wl.make_coords(1)[:100]
    rb = be32.build_rulebook(c)
    x = be32.upload(np.zeros((100, 8), np.float32))
    y = be32.alloc(100 * 4)
    w = np.zeros((4, 27, 8), np.float32)
    with pytest.raises(sh.HipError) as e:
        be32.conv(rb, x, w, None, y, 8, 5)  # output too small
    assert e.value.status == sh.INVALID_ARGUMENT
    with pytest.raises(sh.HipError):
        be32.conv(rb, x, w, None, y, 9, 4)  # input too small
    rb.free()


def test_large_dispatch_centre_only(be32):
    """tests/test_sparse_decoder_backend.c:461-590: 102x102x101 stride-2 grid (no
    neighbours but the centre), centre-only weights, rows at the old grid limits."""
    dx, dy, dz, ci, co = 102, 102, 101, 3, 2
    n = dx * dy * dz
    iz, iy, ix = np.meshgrid(np.arange(dz), np.arange(dy), np.arange(dx), indexing="ij")
    coords = np.stack([np.zeros(n, np.int32), (ix * 2).ravel(), (iy * 2).ravel(), (iz * 2).ravel()], 1).astype(np.int32)
    r = np.arange(n)
    x = np.stack([np.sin((r % 997) * 0.013 + c * 0.17) + 0.001 * ((r + c * 11) % 23) for c in range(ci)],
                 1).astype(np.float32)
    w = np.zeros((co, 27, ci), np.float32)
    for o in range(co):
        for i in range(ci):
            w[o, 13, i] = 0.07 * (o + 1) - 0.03 * i
    bias = np.array([-0.05, 0.15], np.float32)
    got = run_conv(be32, coords, x, w, bias, ci, co)
    for row in (0, 1, 65535 * 16 - 1, 65535 * 16, n - 1):
        exp = bias + x[row].astype(np.float64) @ w[:, 13, :].T
        assert max_rel_err(got[row], exp) <= 2e-4


# -------------------------------------------------------------------- subdivide

def test_c2s_known_answer_host_and_device(be32):
    from test_oracle import c2s_kat

    coords, subdiv, ec, ep, es = c2s_kat()
    lg = be32.upload(subdiv)
    oc, op, os_ = be32.build_c2s_map(coords, lg)
    assert np.array_equal(oc, ec) and np.array_equal(op, ep) and np.array_equal(os_, es)
    dm = be32.build_c2s_map_device(lg, 4, coords=coords)
    assert dm.n == 6
    c2, p2, s2 = be32.download_c2s_map(dm)
    assert np.array_equal(c2, ec) and np.array_equal(p2, ep) and np.array_equal(s2, es)
    assert np.array_equal(be32.download_c2s_coords(dm), ec)
    # A second level can take the first level's device map as its coordinates.
    lg2 = be32.upload(np.where(np.arange(48).reshape(6, 8) % 3 == 0, 1.0, -1.0).astype(np.float32))
    dm2 = be32.build_c2s_map_device(lg2, 6, coords_map=dm)
    rc, e2c, e2p, e2s = orc.c2s_map(ec, np.where(np.arange(48).reshape(6, 8) % 3 == 0, 1.0, -1.0))
    c3, p3, s3 = be32.download_c2s_map(dm2)
    assert np.array_equal(c3, e2c) and np.array_equal(p3, e2p) and np.array_equal(s3, e2s)


@pytest.mark.parametrize("dtype", [sh.F16, sh.BF16])
def test_c2s_exact_on_fp32_logits_with_16bit_storage(be16, bebf, dtype):
    """The voxel set of a 16-bit backend equals the reference's on the same
    fp32 logits (executor.c:119-150: child s exists iff logit > 0), also for
    positives too small for the storage type (fp16 keeps nothing below
    ~3e-8, so round-to-nearest would give +0 and drop the child), +-0.0 and
    tiny negatives.  Both producers of logits are covered: upload_f32 of
    host fp32 values, and the linear slot (the decoder's to_subdiv Ci -> 8),
    here with zero weights so that every row's logits are the bias exactly."""
    be = backend_for(dtype, None, be16, bebf)
    rng = np.random.default_rng(17 + dtype)
    n = 2500
    coords = np.unique(np.stack([rng.integers(0, 2, n), rng.integers(0, 40, n), rng.integers(0, 40, n),
                                 rng.integers(0, 40, n)], 1), axis=0).astype(np.int32)
    n = coords.shape[0]
    special = np.array([1e-7, 6e-8, 3e-8, 2.9e-8, 1e-9, 1e-12, 1e-30, 1.5e-38, -0.0, 0.0, -1e-30, -1e-9, -3e-8,
                        1.0, -1.0, 7e4, -7e4], np.float32)
    logits = np.where(rng.random((n, 8)) < 0.7, special[rng.integers(0, special.size, (n, 8))],
                      rng.standard_normal((n, 8))).astype(np.float32)
    rc, ec, ep, es = orc.c2s_map(coords, logits)
    assert rc == 0
    lg = be.upload(logits)
    dm = be.build_c2s_map_device(lg, n, coords=coords)
    c2, p2, s2 = be.download_c2s_map(dm)
    say(f"c2s fp32 logits dtype={dtype}: {ec.shape[0]} children of {n} parents, got {dm.n}")
    assert np.array_equal(c2, ec) and np.array_equal(p2, ep) and np.array_equal(s2, es)
    hc, hp, hs = be.build_c2s_map(coords, lg)
    assert np.array_equal(hc, ec) and np.array_equal(hp, ep) and np.array_equal(hs, es)
    # Through the linear slot.
    ci = 64
    h = be.upload(sh.storage_round(rng.standard_normal((n, ci)), dtype))
    w = np.zeros((8, ci), np.float32)
    bias = np.array([1e-9, -1e-9, 0.0, -0.0, 2e-8, 1e-30, 1.0, -1.0], np.float32)
    sub = be.alloc(n * 8)
    be.linear(h, w, bias, sub, n, ci, 8)
    rc, ec2, ep2, es2 = orc.c2s_map(coords, np.tile(bias, (n, 1)))
    dm2 = be.build_c2s_map_device(sub, n, coords=coords)
    c3, p3, s3 = be.download_c2s_map(dm2)
    assert dm2.n == 4 * n
    assert np.array_equal(c3, ec2) and np.array_equal(p3, ep2) and np.array_equal(s3, es2)


@pytest.mark.parametrize("dtype", [sh.F32, sh.BF16])
def test_device_map_survives_trim(be32, be16, bebf, dtype):
    """Device C2S maps and guides stay valid across trim (the vtable contract,
    trellis_sparse_backend.h:183-188; the texture decode reuses the shape
    decode's guides, executor.c:304-320): build a map, its rulebook, and the
    gather / broadcast / conv results over it; trim FREE_BUFFERS | WEIGHTS;
    then the map downloads unchanged and the same calls on the same map (and a
    rulebook rebuilt from it) give bit-identical results."""
    be = backend_for(dtype, be32, be16, bebf)
    w = wl.workload(3)
    pc, logits = w["parent_coords"][:40000], w["logits"][:40000]
    npar = pc.shape[0]
    rng = np.random.default_rng(5)
    ci, co = 128, 64
    h = be.upload(sh.storage_round(rng.standard_normal((npar, ci)), dtype))
    up = be.upload(sh.storage_round(rng.standard_normal((npar, 8 * co)), dtype))
    wt = sh.storage_round(rng.standard_normal((co, 27, co)) / math.sqrt(27 * co), dtype)
    dm = be.build_c2s_map_device(be.upload(logits), npar, coords=pc)
    m = dm.n
    rb = be.build_rulebook_for_c2s_map(dm)

    def run_all(rulebook):
        g, s, y = be.alloc(m * co), be.alloc(m * co), be.alloc(m * co)
        be.c2s_gather_device(up, dm, g, co)
        be.skip_repeat_device(h, dm, s, ci, co)
        be.conv(rulebook, g, wt, None, y, co, co)
        return [be.download(b) for b in (g, s, y)]

    before = run_all(rb)
    maps_before = be.download_c2s_map(dm)
    released = be.trim(sh.TRIM_FREE_BUFFERS | sh.TRIM_WEIGHTS)
    say(f"device map survives trim dtype={dtype}: {m} children, trim released {released} bytes")
    assert released > 0
    maps_after = be.download_c2s_map(dm)
    for a, b in zip(maps_before, maps_after):
        assert np.array_equal(a, b)
    rc, ec, ep, es = orc.c2s_map(pc, logits)
    assert np.array_equal(maps_after[0], ec) and np.array_equal(maps_after[1], ep)
    after = run_all(rb)
    for a, b in zip(before, after):
        assert np.array_equal(a, b)
    rb2 = be.build_rulebook_for_c2s_map(dm)
    again = run_all(rb2)
    assert np.array_equal(before[2], again[2])
    rb.free()
    rb2.free()


def test_c2s_no_children_is_error(be32):
    lg = be32.upload(-np.ones((3, 8), np.float32))
    with pytest.raises(sh.HipError) as e:
        be32.build_c2s_map(np.zeros((3, 4), np.int32), lg)
    assert e.value.status == sh.ERROR
    with pytest.raises(sh.HipError) as e:
        be32.build_c2s_map_device(lg, 3, coords=np.zeros((3, 4), np.int32))
    assert e.value.status == sh.ERROR


@pytest.mark.parametrize("dtype", [sh.F32, sh.BF16])
def test_c2s_config3_full_pipeline(be32, be16, bebf, dtype):
    be = backend_for(dtype, be32, be16, bebf)
    w = wl.workload(3)
    pc, logits, pf = w["parent_coords"], w["logits"], w["parent_feats"]
    say(f"cfg3 pipeline dtype={dtype} parents={pc.shape[0]}")
    rc, ec, ep, es = orc.c2s_map(pc, logits)
    assert rc == 0
    lg = be.upload(logits)
    dm = be.build_c2s_map_device(lg, pc.shape[0], coords=pc)
    assert dm.n == ec.shape[0]
    c2, p2, s2 = be.download_c2s_map(dm)
    assert np.array_equal(c2, ec) and np.array_equal(p2, ep) and np.array_equal(s2, es)
    rb = be.build_rulebook_for_c2s_map(dm)
    exp_nbr = orc.Rulebook(ec).neighbors()
    assert np.array_equal(be.neighbors(rb), exp_nbr)
    # Broadcast parent features to the children, then conv 256 -> 128.
    xr = sh.storage_round(pf, dtype)
    xp = be.upload(xr)
    xc = be.alloc(dm.n * 256)
    be.skip_repeat_device(xp, dm, xc, 256, 256)
    child = be.download(xc).reshape(-1, 256)
    exp_child = orc.skip_repeat(xr, ep, es, 256, 256)
    assert np.array_equal(child, exp_child)
    y = be.alloc(dm.n * 128)
    be.conv(rb, xc, w["weight"], None, y, 256, 128)
    got = be.download(y).reshape(-1, 128)
    rows = (5, dm.n, 61)
    exp = orc.Rulebook(ec).conv(exp_child, sh.storage_round(w["weight"], dtype), None, 256, 128, rows=rows)
    err = max_rel_err(got[rows[0]:rows[1]:rows[2]], exp)
    say(f"cfg3 conv dtype={dtype} max_rel_err={err:.3e} on {exp.shape[0]} rows")
    assert err <= TOL[dtype]


@pytest.mark.parametrize("dtype", [sh.F32, sh.F16, sh.BF16])
@pytest.mark.parametrize("ci,co", [(256, 256), (3, 2), (16, 24), (128, 64)])
def test_broadcasts_bitexact(be32, be16, bebf, dtype, ci, co):
    be = backend_for(dtype, be32, be16, bebf)
    rng = np.random.default_rng(ci * 7 + co)
    npar, m = 50, 300
    parent = np.sort(rng.integers(0, npar, m)).astype(np.int32)
    sub = rng.integers(0, 8, m).astype(np.int32)
    x = sh.storage_round(rng.standard_normal((npar, ci)), dtype)
    xb = be.upload(x)
    y = be.alloc(m * co)
    be.skip_repeat(xb, parent, sub, y, ci, co)
    assert np.array_equal(be.download(y).reshape(m, co), orc.skip_repeat(x, parent, sub, ci, co))
    x8 = sh.storage_round(rng.standard_normal((npar, 8 * co)), dtype)
    x8b = be.upload(x8)
    be.c2s_gather(x8b, parent, sub, y, co)
    assert np.array_equal(be.download(y).reshape(m, co), orc.c2s_gather(x8, parent, sub, co))


def test_broadcast_rejects_out_of_range_parent(be32):
    x = be32.upload(np.zeros((4, 8), np.float32))
    y = be32.alloc(2 * 8)
    with pytest.raises(sh.HipError):
        be32.skip_repeat(x, [0, 4], [0, 1], y, 8, 8)


# --------------------------------------------------------------------- row ops

@pytest.mark.parametrize("dtype", [sh.F32, sh.BF16])
def test_row_ops(be32, be16, bebf, dtype):
    be = backend_for(dtype, be32, be16, bebf)
    rng = np.random.default_rng(8)
    n, c = 1031, 128
    x = sh.storage_round(rng.standard_normal((n, c)) * 2 + 0.5, dtype)
    g = rng.standard_normal(c).astype(np.float32)
    b = rng.standard_normal(c).astype(np.float32)
    xb = be.upload(x)
    yb = be.alloc(n * c)
    tol = TOL[dtype]
    for silu in (False, True):
        for gg, bb in ((g, b), (None, None)):
            be.row_norm(xb, gg, bb, yb, n, c, 1e-6, silu=silu)
            assert max_rel_err(be.download(yb), orc.row_norm(x, gg, bb, n, c, 1e-6, silu)) <= tol
    be.silu_inplace(xb, n * c)
    assert max_rel_err(be.download(xb), orc.silu(x)) <= tol
    a = be.upload(x)
    bb_ = be.upload(sh.storage_round(x * 0.5, dtype))
    be.add(a, bb_, yb, n * c)
    assert max_rel_err(be.download(yb), orc.add(x, sh.storage_round(x * 0.5, dtype))) <= tol
    w = (rng.standard_normal((48, c)) * 0.1).astype(np.float32)
    bias = rng.standard_normal(48).astype(np.float32)
    y2 = be.alloc(n * 48)
    for silu in (False, True):
        be.linear(a, w, bias, y2, n, c, 48, silu=silu)
        exp = orc.linear(x, w, bias, n, c, 48, silu)
        got = be.download(y2)
        assert max_rel_err(got, exp) <= tol
        if dtype == sh.F32 and not silu:
            # Same operation order as the reference; SiLU's expf differs from libm by an ulp.
            assert np.array_equal(got.reshape(n, 48), exp)


@pytest.mark.parametrize("dtype", [sh.F16, sh.BF16])
@pytest.mark.parametrize("c,n", [(64, 33), (128, 1031), (256, 7), (512, 300), (1024, 65), (2048, 3), (96, 50)])
def test_row_norm_widths(be16, bebf, dtype, c, n):
    """Vectorised rows (power-of-two widths) and the general kernel (c = 96)."""
    be = backend_for(dtype, None, be16, bebf)
    rng = np.random.default_rng(c + n)
    x = sh.storage_round(rng.standard_normal((n, c)) * 3 - 1, dtype)
    g = rng.standard_normal(c).astype(np.float32)
    b = rng.standard_normal(c).astype(np.float32)
    xb = be.upload(x)
    yb = be.alloc(n * c)
    for silu in (False, True):
        for gg, bb in ((g, b), (None, None), (g, None)):
            be.row_norm(xb, gg, bb, yb, n, c, 1e-6, silu=silu)
            assert max_rel_err(be.download(yb), orc.row_norm(x, gg, bb, n, c, 1e-6, silu)) <= TOL[dtype]


# Shapes of the MFMA linear: 64- and 128-channel column tiles, Ci = 64 (two
# tiles per 4-step block) and Ci % 128 == 0, ragged row counts, and enough
# tiles that every block walks several of them.
LINEAR_MFMA_CASES = [
    (64, 64, 1), (64, 256, 37), (128, 512, 1000), (512, 128, 777), (256, 192, 300), (128, 128, 40000),
    (1024, 256, 2049),
]


@pytest.mark.parametrize("dtype", [sh.F16, sh.BF16])
@pytest.mark.parametrize("ci,co,n", LINEAR_MFMA_CASES)
def test_linear_mfma_vs_oracle(kernel_linears, dtype, ci, co, n):
    be = kernel_linears[dtype]
    say(f"linear mfma dtype={dtype} ci={ci} co={co} n={n}")
    rng = np.random.default_rng(ci * 7 + co + n)
    x = sh.storage_round(rng.standard_normal((n, ci)), dtype)
    w = sh.storage_round(rng.standard_normal((co, ci)) / math.sqrt(ci), dtype)
    bias = rng.standard_normal(co).astype(np.float32)
    xb = be.upload(x)
    yb = be.alloc(n * co)
    for silu in (False, True):
        for bb in (bias, None):
            be.linear(xb, w, bb, yb, n, ci, co, silu=silu)
            exp = orc.linear(x, w, bb, n, ci, co, silu)
            assert max_rel_err(be.download(yb), exp) <= TOL[dtype]


@pytest.mark.parametrize("dtype", [sh.F32, sh.F16, sh.BF16])
@pytest.mark.parametrize("ci,co,n", [(6, 64, 100003), (1, 8, 1), (16, 256, 1031), (3, 24, 77), (6, 64, 1000003)])
def test_linear_small_k_bitexact(be32, be16, bebf, dtype, ci, co, n):
    """Few input channels (the encoder's 6 -> 64 input layer, Ci <= 16): one
    thread per row and 8 outputs.  Bias, then the products in channel order,
    as the oracle (and the reference's linear) sums them: the outputs equal
    the oracle's rounded to the storage type, bit for bit, without SiLU (its
    expf differs from libm by an ulp), and to the storage tolerance with it."""
    be = backend_for(dtype, be32, be16, bebf)
    say(f"linear small K dtype={dtype} ci={ci} co={co} n={n}")
    rng = np.random.default_rng(ci * 7 + co + n)
    x = sh.storage_round(rng.standard_normal((n, ci)), dtype)
    w = rng.standard_normal((co, ci)).astype(np.float32)
    bias = rng.standard_normal(co).astype(np.float32)
    xb = be.upload(x)
    yb = be.alloc(n * co)
    for bb in (bias, None):
        be.linear(xb, w, bb, yb, n, ci, co)
        exp = orc.linear(x, w, bb, n, ci, co)
        assert np.array_equal(be.download(yb).reshape(n, co), sh.storage_round(exp, dtype))
    be.linear(xb, w, bias, yb, n, ci, co, silu=True)
    assert max_rel_err(be.download(yb), orc.linear(x, w, bias, n, ci, co, True)) <= TOL[dtype]


@pytest.mark.parametrize("dtype", [sh.F16, sh.BF16])
@pytest.mark.parametrize("ci,co,n", [(256, 8, 316027), (64, 8, 1), (128, 16, 17), (1024, 3, 1000), (32, 1, 50),
                                     (512, 8, 4099)])
def test_linear_narrow_vs_oracle(be16, bebf, dtype, ci, co, n):
    """Co <= 16 (the subdivide logits, Ci -> 8) on the narrow MFMA kernel:
    ragged 16-row blocks, a single row, bias and SiLU on and off."""
    be = backend_for(dtype, None, be16, bebf)
    say(f"linear narrow dtype={dtype} ci={ci} co={co} n={n}")
    rng = np.random.default_rng(ci * 5 + co + n)
    x = sh.storage_round(rng.standard_normal((n, ci)), dtype)
    w = sh.storage_round(rng.standard_normal((co, ci)) / math.sqrt(ci), dtype)
    bias = rng.standard_normal(co).astype(np.float32)
    xb = be.upload(x)
    yb = be.alloc(n * co)
    for silu in (False, True):
        for bb in (bias, None):
            be.linear(xb, w, bb, yb, n, ci, co, silu=silu)
            exp = orc.linear(x, w, bb, n, ci, co, silu)
            assert max_rel_err(be.download(yb), exp) <= TOL[dtype]


@pytest.mark.parametrize("dtype", [sh.F16, sh.BF16])
@pytest.mark.parametrize("ci,co,n", [(256, 1024, 2048), (1024, 256, 5001), (512, 2048, 3001), (2048, 512, 2050)])
def test_linear_library_vs_oracle_and_kernel(be16, bebf, kernel_linears, dtype, ci, co, n):
    """Wide 16-bit shapes (Ci, Co >= 256, n >= 2048) go to the platform GEMM
    library under the default policy: each result against the oracle
    (trellis_sparse_cpu.c:122-171) and against this library's MFMA kernel,
    bias and SiLU on and off."""
    be, bk = backend_for(dtype, None, be16, bebf), kernel_linears[dtype]
    say(f"linear library dtype={dtype} ci={ci} co={co} n={n}")
    rng = np.random.default_rng(ci * 3 + co + n)
    x = sh.storage_round(rng.standard_normal((n, ci)), dtype)
    w = sh.storage_round(rng.standard_normal((co, ci)) / math.sqrt(ci), dtype)
    bias = rng.standard_normal(co).astype(np.float32)
    xb, yb, yk = be.upload(x), be.alloc(n * co), bk.alloc(n * co)
    xk = bk.upload(x)
    for silu, bb in ((True, bias), (False, None), (False, bias)):
        be.linear(xb, w, bb, yb, n, ci, co, silu=silu)
        bk.linear(xk, w, bb, yk, n, ci, co, silu=silu)
        got, ker = be.download(yb), bk.download(yk)
        exp = orc.linear(x, w, bb, n, ci, co, silu)
        assert max_rel_err(got, exp) <= TOL[dtype]
        assert max_rel_err(ker, exp) <= TOL[dtype]
        assert max_rel_err(got, ker) <= TOL[dtype]
    # trim(FREE_BUFFERS) takes the library's workspace; the next call takes it
    # again and gives the same bits.
    be.trim(sh.TRIM_FREE_BUFFERS)
    be.linear(xb, w, bias, yb, n, ci, co)
    assert np.array_equal(be.download(yb), got)


def test_linear_mfma_rows_independent(bebf):
    """Each row depends on its own input row only (no stale tile state)."""
    ci, co, n = 128, 256, 3000
    rng = np.random.default_rng(5)
    x = sh.storage_round(rng.standard_normal((n, ci)), sh.BF16)
    w = sh.storage_round(rng.standard_normal((co, ci)) / math.sqrt(ci), sh.BF16)
    xb = bebf.upload(x)
    yb = bebf.alloc(n * co)
    bebf.linear(xb, w, None, yb, n, ci, co)
    full = bebf.download(yb).reshape(n, co)
    sub = x[1234:1234 + 129]
    sb = bebf.upload(np.ascontiguousarray(sub))
    ys = bebf.alloc(129 * co)
    bebf.linear(sb, w, None, ys, 129, ci, co)
    assert np.array_equal(bebf.download(ys).reshape(129, co), full[1234:1234 + 129])


def test_trim_releases_and_weights_reload(be32):
    coords, feats, w, bias, ci, co = small_conv_cases()["direct"]
    a = run_conv(be32, coords, feats, w, bias, ci, co)
    released = be32.trim(sh.TRIM_FREE_BUFFERS | sh.TRIM_WEIGHTS)
    assert released > 0
    b = run_conv(be32, coords, feats, w, bias, ci, co)
    assert np.array_equal(a, b)
    with pytest.raises(sh.HipError):
        be32.trim(8)
