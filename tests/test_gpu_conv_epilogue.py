"""GPU parity of the convs with a fused epilogue.

trellis_sparse_hip_conv_norm replaces the slot pair sparse_conv3d ->
row_norm(_silu) and trellis_sparse_hip_conv_add the pair sparse_conv3d -> add,
as the residual blocks compose them (src/architectures/sparse_unet_decoder/
executor.c:176-255, sparse_unet_encoder/executor.c:160-360).  Both are checked
against the oracle's slot chain with the storage rounding between slots, and
against the backend's own slot pair on the same inputs: the add is one fp32
sum of two 16-bit values and one rounding, so it must match the slot pair bit
for bit; the norm reduces in the same lane order as the row_norm slot and is
held to the per-dtype tolerance (tests/test_sparse_decoder_backend.c:16-24).
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
    bes = {dt: sh.Backend(0, dt) for dt in (sh.F32, sh.F16, sh.BF16)}
    yield bes
    for b in bes.values():
        b.destroy()


def shell_coords(n_max):
    """Config-1 sphere shell (batch 0), first n_max voxels in generator order."""
    return np.ascontiguousarray(wl.make_coords(1)[:n_max])


def conv_params(rng, ci, co, dtype):
    w = sh.storage_round(rng.standard_normal((co, 27, ci)) / math.sqrt(27 * ci), dtype)
    b = (0.1 * rng.standard_normal(co)).astype(np.float32)
    return w, b


@pytest.mark.parametrize("dtype", [sh.F16, sh.BF16])
@pytest.mark.parametrize("ci", [64, 128, 256])
@pytest.mark.parametrize("silu", [False, True])
@pytest.mark.parametrize("n", [1, 300, 6000])
def test_conv_norm_vs_oracle(backends, dtype, ci, silu, n):
    be = backends[dtype]
    rnd = lambda a: sh.storage_round(a, dtype)
    co = 128
    rng = np.random.default_rng(7 * ci + n + dtype + int(silu))
    coords = shell_coords(n)
    say(f"conv_norm dtype={dtype} ci={ci} co={co} silu={silu} n={n}")
    x = rnd(rng.standard_normal((n, ci)))
    w, b = conv_params(rng, ci, co, dtype)
    gamma = (1 + 0.1 * rng.standard_normal(co)).astype(np.float32)
    beta = (0.1 * rng.standard_normal(co)).astype(np.float32)
    rb = be.build_rulebook(coords)
    xb, yb = be.upload(x), be.alloc(n * co)
    be.conv_norm(rb, xb, w, b, gamma, beta, 1e-6, yb, ci, co, silu=silu)
    got = be.download(yb).reshape(n, co)
    e_conv = rnd(orc.Rulebook(coords).conv(x, w, b, ci, co))
    e = rnd(orc.row_norm(e_conv, gamma, beta, n, co, 1e-6, silu=silu))
    err = max_rel_err(got, e)
    # The slot pair on the same inputs.
    conv, ref = be.alloc(n * co), be.alloc(n * co)
    be.conv(rb, xb, w, b, conv, ci, co)
    be.row_norm(conv, gamma, beta, ref, n, co, 1e-6, silu=silu)
    g_ref = be.download(ref).reshape(n, co)
    err_slots = max_rel_err(got, g_ref)
    say(f"conv_norm dtype={dtype} ci={ci} silu={silu} n={n} err_oracle={err:.3e} err_slots={err_slots:.3e} "
        f"unequal={int(np.sum(got != g_ref))}")
    assert err <= TOL[dtype]
    assert err_slots <= TOL[dtype]
    rb.free()


def test_conv_norm_without_affine(backends):
    """gamma and beta may be NULL (the C2S block's second norm has no affine)."""
    dtype = sh.BF16
    be = backends[dtype]
    rnd = lambda a: sh.storage_round(a, dtype)
    rng = np.random.default_rng(77)
    coords = shell_coords(2000)
    n, ci, co = coords.shape[0], 128, 128
    x = rnd(rng.standard_normal((n, ci)))
    w, _ = conv_params(rng, ci, co, dtype)
    rb = be.build_rulebook(coords)
    xb, yb = be.upload(x), be.alloc(n * co)
    be.conv_norm(rb, xb, w, None, None, None, 1e-6, yb, ci, co, silu=True)
    got = be.download(yb).reshape(n, co)
    e = rnd(orc.row_norm(rnd(orc.Rulebook(coords).conv(x, w, None, ci, co)), None, None, n, co, 1e-6, silu=True))
    assert max_rel_err(got, e) <= TOL[dtype]
    rb.free()


@pytest.mark.parametrize("dtype", [sh.F16, sh.BF16])
@pytest.mark.parametrize("ci,co", [(64, 128), (128, 128), (256, 128), (128, 256)])
@pytest.mark.parametrize("n", [1, 300, 6000])
def test_conv_add_vs_oracle(backends, dtype, ci, co, n):
    be = backends[dtype]
    rnd = lambda a: sh.storage_round(a, dtype)
    rng = np.random.default_rng(11 * ci + co + n + dtype)
    coords = shell_coords(n)
    say(f"conv_add dtype={dtype} ci={ci} co={co} n={n}")
    x = rnd(rng.standard_normal((n, ci)))
    res = rnd(rng.standard_normal((n, co)))
    w, b = conv_params(rng, ci, co, dtype)
    rb = be.build_rulebook(coords)
    xb, resb, yb = be.upload(x), be.upload(res), be.alloc(n * co)
    be.conv_add(rb, xb, w, b, resb, yb, ci, co)
    got = be.download(yb).reshape(n, co)
    e = rnd(orc.add(rnd(orc.Rulebook(coords).conv(x, w, b, ci, co)), res))
    err = max_rel_err(got, e)
    conv, ref = be.alloc(n * co), be.alloc(n * co)
    be.conv(rb, xb, w, b, conv, ci, co)
    be.add(conv, resb, ref, n * co)
    say(f"conv_add dtype={dtype} ci={ci} co={co} n={n} err_oracle={err:.3e}")
    assert err <= TOL[dtype]
    assert np.array_equal(got, be.download(ref).reshape(n, co))
    # In place: out is the residual buffer.
    be.conv_add(rb, xb, w, b, resb, resb, ci, co)
    assert np.array_equal(be.download(resb).reshape(n, co), got)
    rb.free()


@pytest.mark.parametrize("dtype", [sh.F16, sh.BF16])
def test_residual_block_fused_vs_slots(backends, dtype):
    """The config-2 residual block (conv -> row_norm_silu -> conv -> add) on
    the config-2 voxels, fused pair against slot sequence."""
    be = backends[dtype]
    rnd = lambda a: sh.storage_round(a, dtype)
    rng = np.random.default_rng(2 + dtype)
    coords = np.ascontiguousarray(wl.make_coords(2))
    n, c = coords.shape[0], 128
    say(f"residual block fused vs slots dtype={dtype} n={n}")
    x = rnd(rng.standard_normal((n, c)))
    w1, b1 = conv_params(rng, c, c, dtype)
    w2, b2 = conv_params(rng, c, c, dtype)
    gamma = (1 + 0.1 * rng.standard_normal(c)).astype(np.float32)
    beta = (0.1 * rng.standard_normal(c)).astype(np.float32)
    rb = be.build_rulebook(coords)
    xb = be.upload(x)
    y, h, out = be.alloc(n * c), be.alloc(n * c), be.alloc(n * c)
    be.conv(rb, xb, w1, b1, y, c, c)
    be.row_norm(y, gamma, beta, h, n, c, 1e-6, silu=True)
    be.conv(rb, h, w2, b2, y, c, c)
    be.add(y, xb, out, n * c)
    ref = be.download(out).reshape(n, c)
    h2, out2 = be.alloc(n * c), be.alloc(n * c)
    be.conv_norm(rb, xb, w1, b1, gamma, beta, 1e-6, h2, c, c, silu=True)
    be.conv_add(rb, h2, w2, b2, xb, out2, c, c)
    got = be.download(out2).reshape(n, c)
    err = max_rel_err(got, ref)
    say(f"residual block fused vs slots dtype={dtype} max_rel_err={err:.3e} unequal={int(np.sum(got != ref))}")
    assert err <= TOL[dtype]
    rb.free()


def test_fused_conv_rejects_unsupported(backends):
    """fp32 storage, Co other than 128 for the norm (other than a multiple of
    128 for the add), Ci the compacted conv does not take, and a forced
    non-compacted conv policy report NOT_IMPLEMENTED; nothing is launched."""
    coords = shell_coords(100)
    n = coords.shape[0]
    rng = np.random.default_rng(3)
    cases = [(backends[sh.F32], 128, 128, "norm"), (backends[sh.F32], 128, 128, "add"),
             (backends[sh.BF16], 128, 64, "norm"), (backends[sh.BF16], 128, 256, "norm"),
             (backends[sh.BF16], 128, 64, "add"), (backends[sh.F16], 96, 128, "norm"),
             (backends[sh.F16], 96, 128, "add")]
    masked = sh.Backend(0, sh.BF16, conv_algo=sh.CONV_MASKED)
    cases += [(masked, 128, 128, "norm"), (masked, 128, 128, "add")]
    try:
        for be, ci, co, kind in cases:
            rb = be.build_rulebook(coords)
            xb, yb, rs = be.upload(np.zeros((n, ci), np.float32)), be.alloc(n * co), be.alloc(n * co)
            w, b = conv_params(rng, ci, co, sh.F32)
            with pytest.raises(sh.HipError) as ei:
                if kind == "norm":
                    be.conv_norm(rb, xb, w, b, None, None, 1e-6, yb, ci, co)
                else:
                    be.conv_add(rb, xb, w, b, rs, yb, ci, co)
            assert ei.value.status == sh.NOT_IMPLEMENTED, (ci, co, kind)
            rb.free()
    finally:
        masked.destroy()
