"""Seeded sweep of the 16-bit conv schedules against the oracle.

Each case draws a voxel set (uniform box, Gaussian clusters or repeated
rows, up to 6,000 voxels), channel counts, storage type, conv policy and
epilogue, so that every dispatch branch of the backend's conv runs on
irregular sets: the output-stationary 64 -> 64 kernel, 256-channel blocks over
half tiles, 4- and 8-wavefront 128-channel blocks, 64/32/16-channel blocks,
the masked schedule and the VALU kernel for shapes MFMA does not take.  The
oracle (trellis_sparse_cpu.c:324-373 restated) computes a strided sample of
output rows from the same rounded inputs; the bar is the storage tolerance of
tests/test_sparse_decoder_backend.c:16-24, |a-b| <= 2e-2 max(1,|a|,|b|).
"""
import math
import sys

import numpy as np
import pytest

import oracle_lib as orc
import sparse_hip as sh

pytestmark = pytest.mark.gpu

TOL = 2e-2
CHANNELS = [(64, 64), (128, 128), (256, 128), (128, 256), (256, 512), (384, 128), (64, 128), (512, 256),
            (128, 64), (256, 64), (64, 16), (128, 32), (32, 192), (96, 64), (3, 24), (40, 72)]
ALGOS = [sh.CONV_AUTO, sh.CONV_COMPACT, sh.CONV_MASKED]


def say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def max_rel_err(got, exp):
    return float(np.max(np.abs(got - exp) / np.maximum(1.0, np.maximum(np.abs(got), np.abs(exp))))) \
        if got.size else 0.0


def voxel_set(rng):
    n = int(rng.integers(1, 6000))
    kind = int(rng.integers(0, 3))
    if kind == 0:
        side = int(max(2, round((n / rng.uniform(0.05, 1.0)) ** (1 / 3))))
        c = np.stack([np.zeros(n), *(rng.integers(0, side, n) for _ in range(3))], 1)
    elif kind == 1:
        centres = rng.integers(0, 400, (int(rng.integers(1, 10)), 3))
        pts = centres[rng.integers(0, centres.shape[0], n)] + rng.normal(0, rng.uniform(1, 6), (n, 3))
        c = np.concatenate([rng.integers(0, 2, (n, 1)), np.rint(pts)], 1)
    else:
        base = np.stack([rng.integers(0, 2, n), *(rng.integers(0, 16, n) for _ in range(3))], 1)
        c = base[rng.integers(0, n, n)]
    return np.ascontiguousarray(c.astype(np.int32))


@pytest.fixture(scope="module")
def backends():
    bes = {}
    yield bes
    for b in bes.values():
        b.destroy()


@pytest.mark.parametrize("seed", list(range(32)))
def test_conv_sweep_vs_oracle(backends, seed):
    rng = np.random.default_rng(7000 + seed)
    ci, co = CHANNELS[seed % len(CHANNELS)]
    dtype = sh.BF16 if seed % 2 == 0 else sh.F16
    algo = ALGOS[(seed // 2) % len(ALGOS)]
    key = (dtype, algo)
    if key not in backends:
        backends[key] = sh.Backend(0, dtype, conv_algo=algo)
    be = backends[key]
    coords = voxel_set(rng)
    n = coords.shape[0]
    x = sh.storage_round(rng.standard_normal((n, ci)), dtype)
    w = sh.storage_round(rng.standard_normal((co, 27, ci)) / math.sqrt(27 * ci), dtype)
    bias = (0.1 * rng.standard_normal(co)).astype(np.float32)
    # Epilogue: plain, or residual add, or norm + SiLU where the fused call
    # applies (compacted policy, Co = 128 for the norm, Co % 128 == 0).
    epi = "plain"
    if algo != sh.CONV_MASKED and co % 128 == 0 and (ci == 64 or ci % 128 == 0):
        epi = ["plain", "add", "norm" if co == 128 else "add"][seed % 3]
    say(f"conv sweep seed={seed} n={n} ci={ci} co={co} dtype={dtype} algo={algo} epilogue={epi}")
    rb = be.build_rulebook(coords)
    xb, yb = be.upload(x), be.alloc(n * co)
    step = max(1, n // 300)
    rows = (0, n, step)
    exp = orc.Rulebook(coords).conv(x, w, bias, ci, co, rows=rows)
    if epi == "add":
        res = sh.storage_round(rng.standard_normal((n, co)), dtype)
        be.conv_add(rb, xb, w, bias, be.upload(res), yb, ci, co)
        exp = sh.storage_round(orc.add(sh.storage_round(exp, dtype), res[0:n:step]), dtype)
    elif epi == "norm":
        gamma = (1 + 0.1 * rng.standard_normal(co)).astype(np.float32)
        beta = (0.1 * rng.standard_normal(co)).astype(np.float32)
        be.conv_norm(rb, xb, w, bias, gamma, beta, 1e-6, yb, ci, co, silu=True)
        exp = sh.storage_round(orc.row_norm(sh.storage_round(exp, dtype), gamma, beta, exp.shape[0], co, 1e-6,
                                            silu=True), dtype)
    else:
        be.conv(rb, xb, w, bias, yb, ci, co)
    got = be.download(yb).reshape(n, co)[0:n:step]
    err = max_rel_err(got, exp)
    say(f"conv sweep seed={seed} rows={exp.shape[0]} max_rel_err={err:.3e}")
    assert err <= TOL
    rb.free()
