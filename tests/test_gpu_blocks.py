"""GPU parity of the decoder blocks the backend's slots compose into.

The reference decoder builds its blocks from the vtable slots:
- ConvNeXt block (src/architectures/sparse_unet_decoder/executor.c:176-255):
  conv(C->C) -> row_norm(gamma, beta, 1e-6) -> linear_silu(C->4C)
  -> linear(4C->C) -> add(h, .).
- C2S up-block, device-map path (executor.c:257-554): linear(Ci->8) logits
  -> build_c2s_map_device -> build_rulebook_for_c2s_map;
  row_norm_silu(h) -> conv(Ci->8Co) on the parent rulebook
  -> c2s_gather_device; skip_repeat_device(h);
  row_norm_silu(h_up, no affine) -> conv(Co->Co) on the child rulebook
  -> add(conv2, skip).
- The encoder's S2C down-block (src/architectures/sparse_unet_encoder/
  executor.c:160-360), with the device S2C steps in place of the host build
  and pack round trip (:209-300): s2c_build_device -> coarse rulebook;
  row_norm_silu(h) -> conv(Ci->Co/8) on the fine rulebook -> s2c_pack;
  s2c_skip_mean(h); row_norm_silu(packed, no affine) -> conv(Co->Co) on the
  coarse rulebook -> add(conv2, skip).
Here the same sequences run through the C ABI and are compared with the
oracle's restatement of each slot, chained with the storage rounding the
backend applies between slots.  Maps stay bit-exact; values meet the
per-dtype tolerance of check_close (tests/test_sparse_decoder_backend.c:16-24).
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
def backends():
    bes = {dt: sh.Backend(0, dt) for dt in (sh.F32, sh.F16, sh.BF16)}
    yield bes
    for b in bes.values():
        b.destroy()


def shell_coords(n_max):
    """Config-1 sphere shell (batch 0), first n_max voxels in generator order."""
    return np.ascontiguousarray(wl.make_coords(1)[:n_max])


def weights(rng, co, k, ci, dtype):
    return sh.storage_round(rng.standard_normal((co, k, ci)) / math.sqrt(k * ci), dtype)


@pytest.mark.parametrize("dtype", [sh.F32, sh.F16, sh.BF16])
@pytest.mark.parametrize("c", [64, 128])
def test_convnext_block_vs_oracle(backends, dtype, c):
    be = backends[dtype]
    rnd = lambda a: sh.storage_round(a, dtype)
    rng = np.random.default_rng(c + dtype)
    coords = shell_coords(6000)
    n = coords.shape[0]
    say(f"convnext dtype={dtype} c={c} n={n}")
    h = rnd(rng.standard_normal((n, c)))
    conv_w = weights(rng, c, 27, c, dtype)
    conv_b = rng.standard_normal(c).astype(np.float32) * 0.1
    gamma = (1 + 0.1 * rng.standard_normal(c)).astype(np.float32)
    beta = (0.1 * rng.standard_normal(c)).astype(np.float32)
    w0 = rnd(rng.standard_normal((4 * c, c)) / math.sqrt(c))
    b0 = (0.1 * rng.standard_normal(4 * c)).astype(np.float32)
    w2 = rnd(rng.standard_normal((c, 4 * c)) / math.sqrt(4 * c))
    b2 = (0.1 * rng.standard_normal(c)).astype(np.float32)

    rb = be.build_rulebook(coords)
    hb = be.upload(h)
    conv = be.alloc(n * c)
    norm = be.alloc(n * c)
    mlp1 = be.alloc(n * 4 * c)
    mlp2 = be.alloc(n * c)
    out = be.alloc(n * c)
    be.conv(rb, hb, conv_w, conv_b, conv, c, c)
    be.row_norm(conv, gamma, beta, norm, n, c, 1e-6)
    be.linear(norm, w0, b0, mlp1, n, c, 4 * c, silu=True)
    be.linear(mlp1, w2, b2, mlp2, n, 4 * c, c)
    be.add(hb, mlp2, out, n * c)
    got = be.download(out).reshape(n, c)

    # Oracle chain on the values the backend holds after each slot: the conv
    # is compared first, then each later slot runs on the backend's own input
    # so the tolerance applies per slot, not compounded.
    e_conv = rnd(orc.Rulebook(coords).conv(h, conv_w, conv_b, c, c))
    g_conv = be.download(conv).reshape(n, c)
    assert max_rel_err(g_conv, e_conv) <= TOL[dtype]
    g_norm = be.download(norm).reshape(n, c)
    assert max_rel_err(g_norm, rnd(orc.row_norm(g_conv, gamma, beta, n, c, 1e-6))) <= TOL[dtype]
    g_mlp1 = be.download(mlp1).reshape(n, 4 * c)
    assert max_rel_err(g_mlp1, rnd(orc.linear(g_norm, w0, b0, n, c, 4 * c, silu=True))) <= TOL[dtype]
    g_mlp2 = be.download(mlp2).reshape(n, c)
    assert max_rel_err(g_mlp2, rnd(orc.linear(g_mlp1, w2, b2, n, 4 * c, c))) <= TOL[dtype]
    assert max_rel_err(got, rnd(orc.add(h, g_mlp2))) <= TOL[dtype]
    # End to end against the oracle chain from the block input alone.
    e = rnd(orc.row_norm(e_conv, gamma, beta, n, c, 1e-6))
    e = rnd(orc.linear(e, w0, b0, n, c, 4 * c, silu=True))
    e = rnd(orc.linear(e, w2, b2, n, 4 * c, c))
    e = rnd(orc.add(h, e))
    err = max_rel_err(got, e)
    say(f"convnext dtype={dtype} c={c} end-to-end max_rel_err={err:.3e}")
    assert err <= (TOL[dtype] if dtype == sh.F32 else 5e-2)
    rb.free()


def mlp_params(rng, c, dtype):
    rnd = lambda a: sh.storage_round(a, dtype)
    gamma = (1 + 0.1 * rng.standard_normal(c)).astype(np.float32)
    beta = (0.1 * rng.standard_normal(c)).astype(np.float32)
    w0 = rnd(rng.standard_normal((4 * c, c)) / math.sqrt(c))
    b0 = (0.1 * rng.standard_normal(4 * c)).astype(np.float32)
    w2 = rnd(rng.standard_normal((c, 4 * c)) / math.sqrt(4 * c))
    b2 = (0.1 * rng.standard_normal(c)).astype(np.float32)
    return gamma, beta, w0, b0, w2, b2


@pytest.mark.parametrize("dtype", [sh.F16, sh.BF16])
@pytest.mark.parametrize("c", [64, 128, 256])
@pytest.mark.parametrize("n", [1, 63, 65, 127, 129, 4099])
def test_convnext_mlp_fused_vs_oracle(backends, dtype, c, n):
    """The fused tail against the oracle's slot chain with the same storage
    roundings (norm, hidden, second linear, add); rows past a tile edge (64-row
    tiles at c = 64 and 128, 128-row tiles at c = 256) and a single row
    included."""
    be = backends[dtype]
    rnd = lambda a: sh.storage_round(a, dtype)
    rng = np.random.default_rng(1000 * c + n + dtype)
    say(f"convnext_mlp fused dtype={dtype} c={c} n={n}")
    x = rnd(2 * rng.standard_normal((n, c)) + 0.5)
    res = rnd(rng.standard_normal((n, c)))
    gamma, beta, w0, b0, w2, b2 = mlp_params(rng, c, dtype)
    xb, rb_, yb = be.upload(x), be.upload(res), be.alloc(n * c)
    be.convnext_mlp(xb, gamma, beta, w0, b0, w2, b2, rb_, yb, n, c, 1e-6)
    got = be.download(yb).reshape(n, c)
    e = rnd(orc.row_norm(x, gamma, beta, n, c, 1e-6))
    e = rnd(orc.linear(e, w0, b0, n, c, 4 * c, silu=True))
    e = rnd(orc.linear(e, w2, b2, n, 4 * c, c))
    e = rnd(orc.add(res, e))
    err = max_rel_err(got, e)
    say(f"convnext_mlp fused dtype={dtype} c={c} n={n} max_rel_err={err:.3e}")
    assert err <= TOL[dtype]


@pytest.mark.parametrize("dtype", [sh.F16, sh.BF16])
@pytest.mark.parametrize("c", [64, 128, 256])
def test_convnext_mlp_fused_vs_slots(backends, dtype, c):
    """At a size where blocks walk many tiles (and the weight ring runs
    across tile boundaries), the fused tail matches the slot sequence it
    replaces, itself checked against the oracle above; calling it twice with
    the same weights (cached packing) gives identical results."""
    be = backends[dtype]
    rnd = lambda a: sh.storage_round(a, dtype)
    n = 250_007
    rng = np.random.default_rng(31 + c + dtype)
    say(f"convnext_mlp fused vs slots dtype={dtype} c={c} n={n}")
    x = rnd(rng.standard_normal((n, c)))
    res = rnd(rng.standard_normal((n, c)))
    gamma, beta, w0, b0, w2, b2 = mlp_params(rng, c, dtype)
    xb, rb_ = be.upload(x), be.upload(res)
    norm, hid, lin2, ref = be.alloc(n * c), be.alloc(n * 4 * c), be.alloc(n * c), be.alloc(n * c)
    be.row_norm(xb, gamma, beta, norm, n, c, 1e-6)
    be.linear(norm, w0, b0, hid, n, c, 4 * c, silu=True)
    be.linear(hid, w2, b2, lin2, n, 4 * c, c)
    be.add(rb_, lin2, ref, n * c)
    y1, y2 = be.alloc(n * c), be.alloc(n * c)
    be.convnext_mlp(xb, gamma, beta, w0, b0, w2, b2, rb_, y1, n, c, 1e-6)
    be.convnext_mlp(xb, gamma, beta, w0, b0, w2, b2, rb_, y2, n, c, 1e-6)
    g1, g2 = be.download(y1), be.download(y2)
    assert np.array_equal(g1, g2)
    err = max_rel_err(g1, be.download(ref))
    say(f"convnext_mlp fused vs slots dtype={dtype} c={c} max_rel_err={err:.3e}")
    assert err <= TOL[dtype]


def oracle_mlp_rows(x, res, params, c, dtype, idx):
    """The tail's slot chain on the oracle for the rows idx only (every slot
    is row-wise), rounded where the slots store."""
    rnd = lambda a: sh.storage_round(a, dtype)
    gamma, beta, w0, b0, w2, b2 = params
    m = len(idx)
    e = rnd(orc.row_norm(np.ascontiguousarray(x[idx]), gamma, beta, m, c, 1e-6))
    e = rnd(orc.linear(e, w0, b0, m, c, 4 * c, silu=True))
    e = rnd(orc.linear(e, w2, b2, m, 4 * c, c))
    return rnd(orc.add(np.ascontiguousarray(res[idx]), e))


def sample_idx(n, step):
    """Every step-th row, the last row and the first of each 128-row tile edge."""
    return np.unique(np.concatenate([np.arange(0, n, step), [n - 1], np.arange(127, n, 128)[:8]]))


@pytest.fixture(scope="module")
def kernel_backends():
    """16-bit backends whose linears never take the GEMM library."""
    bes = {dt: sh.Backend(0, dt, linear_algo=sh.LINEAR_KERNEL) for dt in (sh.F16, sh.BF16)}
    yield bes
    for b in bes.values():
        b.destroy()


@pytest.mark.parametrize("dtype", [sh.F16, sh.BF16])
@pytest.mark.parametrize("c", [512, 1024])
@pytest.mark.parametrize("n", [1, 300, 2100])
def test_convnext_mlp_composed_vs_oracle(backends, kernel_backends, dtype, c, n):
    """Widths 512 and 1024 (the decoder's two deepest levels): the tail runs
    as row_norm, mlp0 + SiLU and mlp2 with the residual added to its sums.
    Both routes against the oracle's slot chain on sampled rows: the GEMM
    library's (n >= 2048; one rounding of residual + mlp2 where the slots
    round twice, within the storage tolerance) and the kernels' (n < 2048, or
    the LINEAR_KERNEL policy: the slot roundings), and the two against each
    other."""
    rnd = lambda a: sh.storage_round(a, dtype)
    rng = np.random.default_rng(7000 + c + n + dtype)
    say(f"convnext_mlp composed dtype={dtype} c={c} n={n}")
    x = rnd(2 * rng.standard_normal((n, c)) + 0.5)
    res = rnd(rng.standard_normal((n, c)))
    params = mlp_params(rng, c, dtype)
    idx = sample_idx(n, 37)
    exp = oracle_mlp_rows(x, res, params, c, dtype, idx)
    outs = []
    for be in (backends[dtype], kernel_backends[dtype]):
        xb, rb_, yb = be.upload(x), be.upload(res), be.alloc(n * c)
        be.convnext_mlp(xb, *params, rb_, yb, n, c, 1e-6)
        got = be.download(yb).reshape(n, c)
        err = max_rel_err(got[idx], exp)
        say(f"convnext_mlp composed dtype={dtype} c={c} n={n} linear_algo={be.linear_algo} max_rel_err={err:.3e}")
        assert err <= TOL[dtype]
        outs.append(got)
        xb.free(), rb_.free(), yb.free()
    err = max_rel_err(outs[0], outs[1])
    say(f"convnext_mlp composed dtype={dtype} c={c} n={n} library vs kernels max_rel_err={err:.3e}")
    assert err <= TOL[dtype]


@pytest.mark.parametrize("dtype", [sh.BF16])
def test_convnext_mlp_composed_residual_is_output(backends, dtype):
    """y may be the residual buffer itself (the library adds C = y in place;
    the kernels' fallback goes through the row_norm intermediate)."""
    c, n = 512, 2100
    rnd = lambda a: sh.storage_round(a, dtype)
    rng = np.random.default_rng(77)
    x = rnd(rng.standard_normal((n, c)))
    res = rnd(rng.standard_normal((n, c)))
    params = mlp_params(rng, c, dtype)
    be = backends[dtype]
    xb, rb_, yb = be.upload(x), be.upload(res), be.alloc(n * c)
    be.convnext_mlp(xb, *params, rb_, yb, n, c, 1e-6)
    be.convnext_mlp(xb, *params, rb_, rb_, n, c, 1e-6)
    assert np.array_equal(be.download(yb), be.download(rb_))


def test_convnext_mlp_rejects_unsupported(backends):
    """fp32 storage and widths other than 64 / 128 / 256 or a multiple of 128
    from 512 report NOT_IMPLEMENTED (the caller then runs the slot sequence);
    nothing is launched."""
    rng = np.random.default_rng(5)
    for dtype, c in ((sh.F32, 64), (sh.BF16, 96), (sh.F16, 384), (sh.BF16, 576), (sh.F32, 512)):
        be = backends[dtype]
        n = 10
        gamma, beta, w0, b0, w2, b2 = mlp_params(rng, c, dtype)
        xb, yb = be.upload(np.zeros((n, c), np.float32)), be.alloc(n * c)
        with pytest.raises(sh.HipError) as ei:
            be.convnext_mlp(xb, gamma, beta, w0, b0, w2, b2, xb, yb, n, c, 1e-6)
        assert ei.value.status == sh.NOT_IMPLEMENTED


def convnext_block_params(rng, c, dtype):
    conv_w = weights(rng, c, 27, c, dtype)
    conv_b = (0.1 * rng.standard_normal(c)).astype(np.float32)
    return (conv_w, conv_b) + mlp_params(rng, c, dtype)


def oracle_convnext_block(coords, h, params, c, dtype):
    """The slot chain row by row on the oracle, rounded where the slots store."""
    rnd = lambda a: sh.storage_round(a, dtype)
    conv_w, conv_b, gamma, beta, w0, b0, w2, b2 = params
    n = h.shape[0]
    e = rnd(orc.Rulebook(coords).conv(h, conv_w, conv_b, c, c))
    e = rnd(orc.row_norm(e, gamma, beta, n, c, 1e-6))
    e = rnd(orc.linear(e, w0, b0, n, c, 4 * c, silu=True))
    e = rnd(orc.linear(e, w2, b2, n, 4 * c, c))
    return rnd(orc.add(h, e))


@pytest.mark.parametrize("dtype", [sh.F16, sh.BF16])
@pytest.mark.parametrize("c,n", [(c, n) for c in (64, 128, 256) for n in (1, 300, 6000)] + [(512, 300), (512, 2100)])
def test_convnext_block_entry_vs_oracle(backends, dtype, c, n):
    """trellis_sparse_hip_convnext_block (the conv, then the fused tail)
    against the oracle's slot chain from the block input; the tolerance is the
    end-to-end one of the slot sequence above (each slot within the storage
    tolerance, compounded)."""
    be = backends[dtype]
    rnd = lambda a: sh.storage_round(a, dtype)
    rng = np.random.default_rng(500 + c + n + dtype)
    coords = shell_coords(n)
    say(f"convnext_block entry dtype={dtype} c={c} n={n}")
    h = rnd(rng.standard_normal((n, c)))
    params = convnext_block_params(rng, c, dtype)
    rb = be.build_rulebook(coords)
    hb, out = be.upload(h), be.alloc(n * c)
    be.convnext_block(rb, hb, *params, out, c, 1e-6)
    got = be.download(out).reshape(n, c)
    err = max_rel_err(got, oracle_convnext_block(coords, h, params, c, dtype))
    say(f"convnext_block entry dtype={dtype} c={c} n={n} max_rel_err={err:.3e}")
    assert err <= 5e-2
    rb.free()


@pytest.mark.parametrize("dtype", [sh.F16, sh.BF16])
@pytest.mark.parametrize("c", [64, 128, 256])
def test_convnext_block_entry_vs_slots(backends, dtype, c):
    """On the config-2 voxels: the block entry against the five slots on the
    same inputs, to the storage tolerance (the MLP's sums run in another order
    than the linear slots')."""
    be = backends[dtype]
    rnd = lambda a: sh.storage_round(a, dtype)
    rng = np.random.default_rng(900 + c + dtype)
    coords = np.ascontiguousarray(wl.make_coords(2))
    n = coords.shape[0]
    say(f"convnext_block entry vs slots dtype={dtype} c={c} n={n}")
    h = rnd(rng.standard_normal((n, c)))
    conv_w, conv_b, gamma, beta, w0, b0, w2, b2 = convnext_block_params(rng, c, dtype)
    rb = be.build_rulebook(coords)
    hb = be.upload(h)
    conv, norm, mlp1, mlp2, ref = (be.alloc(n * c), be.alloc(n * c), be.alloc(n * 4 * c), be.alloc(n * c),
                                   be.alloc(n * c))
    be.conv(rb, hb, conv_w, conv_b, conv, c, c)
    be.row_norm(conv, gamma, beta, norm, n, c, 1e-6)
    be.linear(norm, w0, b0, mlp1, n, c, 4 * c, silu=True)
    be.linear(mlp1, w2, b2, mlp2, n, 4 * c, c)
    be.add(hb, mlp2, ref, n * c)
    out = be.alloc(n * c)
    be.convnext_block(rb, hb, conv_w, conv_b, gamma, beta, w0, b0, w2, b2, out, c, 1e-6)
    got, exp = be.download(out), be.download(ref)
    err = max_rel_err(got, exp)
    say(f"convnext_block entry vs slots dtype={dtype} c={c} max_rel_err={err:.3e}")
    assert err <= TOL[dtype]
    rb.free()


def test_convnext_block_entry_rejects(backends):
    """fp32 storage, c other than 64 / 128 / 256 or a multiple of 128 from
    512, and out aliasing h are refused before anything is launched."""
    rng = np.random.default_rng(6)
    coords = shell_coords(50)
    n = coords.shape[0]
    for dtype, c, status in ((sh.F32, 64, sh.NOT_IMPLEMENTED), (sh.BF16, 96, sh.NOT_IMPLEMENTED),
                             (sh.F16, 384, sh.NOT_IMPLEMENTED)):
        be = backends[dtype]
        rb = be.build_rulebook(coords)
        hb, out = be.upload(np.zeros((n, c), np.float32)), be.alloc(n * c)
        with pytest.raises(sh.HipError) as ei:
            be.convnext_block(rb, hb, *convnext_block_params(rng, c, sh.F32), out, c, 1e-6)
        assert ei.value.status == status
        rb.free()
    be = backends[sh.BF16]
    rb = be.build_rulebook(coords)
    hb = be.upload(np.zeros((n, 128), np.float32))
    with pytest.raises(sh.HipError) as ei:
        be.convnext_block(rb, hb, *convnext_block_params(rng, 128, sh.F32), hb, 128, 1e-6)
    assert ei.value.status == sh.INVALID_ARGUMENT
    rb.free()


@pytest.mark.parametrize("dtype", [sh.F32, sh.BF16])
def test_c2s_upblock_vs_oracle(backends, dtype):
    be = backends[dtype]
    rnd = lambda a: sh.storage_round(a, dtype)
    ci, co = 64, 32
    rng = np.random.default_rng(77 + dtype)
    coords = shell_coords(3000)
    n = coords.shape[0]
    say(f"c2s up-block dtype={dtype} parents={n} {ci}->{co}")
    h = rnd(rng.standard_normal((n, ci)))
    ws = (rng.standard_normal((8, ci)) / math.sqrt(ci)).astype(np.float32)
    bs = (0.1 * rng.standard_normal(8)).astype(np.float32)
    g1 = (1 + 0.1 * rng.standard_normal(ci)).astype(np.float32)
    b1 = (0.1 * rng.standard_normal(ci)).astype(np.float32)
    w1 = weights(rng, 8 * co, 27, ci, dtype)
    c1b = (0.1 * rng.standard_normal(8 * co)).astype(np.float32)
    w2 = weights(rng, co, 27, co, dtype)
    c2b = (0.1 * rng.standard_normal(co)).astype(np.float32)

    pmap = be.upload_coords(coords)
    rb = be.build_rulebook_for_c2s_map(pmap)
    hb = be.upload(h)
    subdiv = be.alloc(n * 8)
    be.linear(hb, ws, bs, subdiv, n, ci, 8)
    logits = be.download(subdiv).reshape(n, 8)
    assert max_rel_err(logits, rnd(orc.linear(h, ws, bs, n, ci, 8))) <= TOL[dtype]
    dm = be.build_c2s_map_device(subdiv, n, coords_map=pmap)
    rc, ec, ep, es = orc.c2s_map(coords, logits)
    assert rc == 0
    c2, p2, s2 = be.download_c2s_map(dm)
    assert np.array_equal(c2, ec) and np.array_equal(p2, ep) and np.array_equal(s2, es)
    m = dm.n
    nrb = be.build_rulebook_for_c2s_map(dm)
    assert np.array_equal(be.neighbors(nrb), orc.Rulebook(ec).neighbors())

    norm1 = be.alloc(n * ci)
    be.row_norm(hb, g1, b1, norm1, n, ci, 1e-6, silu=True)
    conv1 = be.alloc(n * 8 * co)
    be.conv(rb, norm1, w1, c1b, conv1, ci, 8 * co)
    h_up = be.alloc(m * co)
    be.c2s_gather_device(conv1, dm, h_up, co)
    skip = be.alloc(m * co)
    be.skip_repeat_device(hb, dm, skip, ci, co)
    norm2 = be.alloc(m * co)
    be.row_norm(h_up, None, None, norm2, m, co, 1e-6, silu=True)
    conv2 = be.alloc(m * co)
    be.conv(nrb, norm2, w2, c2b, conv2, co, co)
    out = be.alloc(m * co)
    be.add(conv2, skip, out, m * co)

    # Per slot, each on the backend's own input (see the ConvNeXt test).
    g_n1 = be.download(norm1).reshape(n, ci)
    assert max_rel_err(g_n1, rnd(orc.row_norm(h, g1, b1, n, ci, 1e-6, silu=True))) <= TOL[dtype]
    g_c1 = be.download(conv1).reshape(n, 8 * co)
    assert max_rel_err(g_c1, rnd(orc.Rulebook(coords).conv(g_n1, w1, c1b, ci, 8 * co))) <= TOL[dtype]
    g_up = be.download(h_up).reshape(m, co)
    assert np.array_equal(g_up, orc.c2s_gather(g_c1, ep, es, co))
    g_skip = be.download(skip).reshape(m, co)
    assert np.array_equal(g_skip, orc.skip_repeat(h, ep, es, ci, co))
    g_n2 = be.download(norm2).reshape(m, co)
    assert max_rel_err(g_n2, rnd(orc.row_norm(g_up, None, None, m, co, 1e-6, silu=True))) <= TOL[dtype]
    g_c2 = be.download(conv2).reshape(m, co)
    assert max_rel_err(g_c2, rnd(orc.Rulebook(ec).conv(g_n2, w2, c2b, co, co))) <= TOL[dtype]
    got = be.download(out).reshape(m, co)
    assert max_rel_err(got, rnd(orc.add(g_c2, g_skip))) <= TOL[dtype]
    say(f"c2s up-block dtype={dtype} children={m}")
    rb.free()
    nrb.free()


@pytest.mark.parametrize("dtype", [sh.F32, sh.F16, sh.BF16])
@pytest.mark.parametrize("ci,co", [(64, 128), (128, 256)])
def test_s2c_downblock_vs_oracle(backends, dtype, ci, co):
    be = backends[dtype]
    rnd = lambda a: sh.storage_round(a, dtype)
    pc = co // 8
    rng = np.random.default_rng(91 + ci + dtype)
    coords = shell_coords(6000)
    n = coords.shape[0]
    say(f"s2c down-block dtype={dtype} fine={n} {ci}->{co}")
    h = rnd(rng.standard_normal((n, ci)))
    g1 = (1 + 0.1 * rng.standard_normal(ci)).astype(np.float32)
    b1 = (0.1 * rng.standard_normal(ci)).astype(np.float32)
    w1 = weights(rng, pc, 27, ci, dtype)
    c1b = (0.1 * rng.standard_normal(pc)).astype(np.float32)
    w2 = weights(rng, co, 27, co, dtype)
    c2b = (0.1 * rng.standard_normal(co)).astype(np.float32)

    pmap = be.upload_coords(coords)
    rb = be.build_rulebook_for_c2s_map(pmap)
    hb = be.upload(h)
    fmap, cmap = be.s2c_build_device(coords_map=pmap)
    rc, ec, ep, es = orc.s2c_map(coords)
    assert rc == 0
    m = cmap.n
    assert np.array_equal(be.download_c2s_coords(cmap), ec)
    c, p, s = be.download_c2s_map(fmap)
    assert np.array_equal(c, coords) and np.array_equal(p, ep) and np.array_equal(s, es)
    crb = be.build_rulebook_for_c2s_map(cmap)
    assert np.array_equal(be.neighbors(crb), orc.Rulebook(ec).neighbors())

    norm1 = be.alloc(n * ci)
    be.row_norm(hb, g1, b1, norm1, n, ci, 1e-6, silu=True)
    conv1 = be.alloc(n * pc)
    be.conv(rb, norm1, w1, c1b, conv1, ci, pc)
    packed = be.alloc(m * co)
    be.s2c_pack_device(conv1, fmap, packed, co)
    skip = be.alloc(m * co)
    be.s2c_skip_mean_device(hb, fmap, skip, ci, co)
    norm2 = be.alloc(m * co)
    be.row_norm(packed, None, None, norm2, m, co, 1e-6, silu=True)
    conv2 = be.alloc(m * co)
    be.conv(crb, norm2, w2, c2b, conv2, co, co)
    out = be.alloc(m * co)
    be.add(conv2, skip, out, m * co)

    # Per slot, each on the backend's own input (see the ConvNeXt test).
    g_n1 = be.download(norm1).reshape(n, ci)
    assert max_rel_err(g_n1, rnd(orc.row_norm(h, g1, b1, n, ci, 1e-6, silu=True))) <= TOL[dtype]
    g_c1 = be.download(conv1).reshape(n, pc)
    assert max_rel_err(g_c1, rnd(orc.Rulebook(coords).conv(g_n1, w1, c1b, ci, pc))) <= TOL[dtype]
    g_pk = be.download(packed).reshape(m, co)
    assert np.array_equal(g_pk, orc.s2c_pack(g_c1, ep, es, m, co))
    g_skip = be.download(skip).reshape(m, co)
    assert np.array_equal(g_skip, rnd(orc.s2c_skip_mean(h, ep, es, m, ci, co)))
    g_n2 = be.download(norm2).reshape(m, co)
    assert max_rel_err(g_n2, rnd(orc.row_norm(g_pk, None, None, m, co, 1e-6, silu=True))) <= TOL[dtype]
    g_c2 = be.download(conv2).reshape(m, co)
    assert max_rel_err(g_c2, rnd(orc.Rulebook(ec).conv(g_n2, w2, c2b, co, co))) <= TOL[dtype]
    got = be.download(out).reshape(m, co)
    assert max_rel_err(got, rnd(orc.add(g_c2, g_skip))) <= TOL[dtype]
    # The whole block on the oracle alone, from h: the rounding of each slot
    # mirrored, the slot errors compounding through two convs and two norms.
    e_c1 = rnd(orc.Rulebook(coords).conv(rnd(orc.row_norm(h, g1, b1, n, ci, 1e-6, silu=True)), w1, c1b, ci, pc))
    e_n2 = rnd(orc.row_norm(orc.s2c_pack(e_c1, ep, es, m, co), None, None, m, co, 1e-6, silu=True))
    e_out = rnd(orc.add(rnd(orc.Rulebook(ec).conv(e_n2, w2, c2b, co, co)), g_skip))
    assert max_rel_err(got, e_out) <= (1e-4 if dtype == sh.F32 else 5e-2)
    say(f"s2c down-block dtype={dtype} coarse={m}")
    rb.free()
    crb.free()
    be.free_map(fmap)
    be.free_map(cmap)
    be.free_map(pmap)
