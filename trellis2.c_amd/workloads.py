"""Seeded synthetic workloads for the five benchmark configurations.

Coordinates come from the C generator in synth/ (deterministic, raster order
b, x, y, z).  Feature, weight and logit draws are counter-based N(0, std) /
Bernoulli fills keyed by (config seed, stream), so the GPU path and the CPU
oracle see bit-identical inputs.  bf16/fp16 configs use the round-to-nearest-
even rounding of the same fp32 draws.

  cfg 1  R=64 sphere shell, conv 64->64 fp32 (the reference CPU case)
  cfg 2  R=256 shells, conv(128->128) -> LayerNorm -> SiLU -> conv(128->128) + skip, fp16
  cfg 3  R=256 parent shells, 2x subdivide (Bernoulli 0.5 per child) to R=512,
         parent->child broadcast (skip_repeat 256->256), conv 256->128, bf16
  cfg 4  R=1024 thin shells, hash + kernel-map rebuild + conv 64->64, bf16
  cfg 5  2 dense 32^3 + 2 Bernoulli(0.5) 64^3 structures in one batch, conv 512->512, bf16
"""
from __future__ import annotations

import ctypes
import math
import os
from ctypes import POINTER, c_double, c_float, c_int, c_int32, c_int64, c_uint64

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
SYNTH_PATH = os.path.join(HERE, "synth", "libtrellis_synth.so")

F32, F16, BF16 = 0, 1, 2
DTYPE_NAMES = {F32: "f32", F16: "f16", BF16: "bf16"}

_S = None


def synth():
    global _S
    if _S is None:
        if not os.path.exists(SYNTH_PATH):
            raise RuntimeError(f"{SYNTH_PATH} is missing: run __graft_entry__.build() first")
        s = ctypes.CDLL(SYNTH_PATH)
        s.ts_make_coords.argtypes = [c_int, POINTER(POINTER(c_int32)), POINTER(c_int64)]
        s.ts_make_coords.restype = c_int
        s.ts_normal.argtypes = [c_uint64, c_uint64, c_float, POINTER(c_float), c_int64]
        s.ts_normal.restype = None
        s.ts_pm1.argtypes = [c_uint64, c_uint64, c_double, POINTER(c_float), c_int64]
        s.ts_pm1.restype = None
        s.ts_free.argtypes = [ctypes.c_void_p]
        _S = s
    return _S


def make_coords(cfg: int) -> np.ndarray:
    s = synth()
    p = POINTER(c_int32)()
    n = c_int64()
    rc = s.ts_make_coords(cfg, ctypes.byref(p), ctypes.byref(n))
    if rc != 0:
        raise RuntimeError(f"ts_make_coords({cfg}) failed: {rc}")
    try:
        return np.ctypeslib.as_array(p, shape=(n.value, 4)).copy()
    finally:
        s.ts_free(ctypes.cast(p, ctypes.c_void_p))


def normal(seed: int, stream: int, count: int, std: float = 1.0) -> np.ndarray:
    out = np.empty(count, dtype=np.float32)
    synth().ts_normal(seed, stream, std, out.ctypes.data_as(POINTER(c_float)), count)
    return out


def pm1(seed: int, stream: int, count: int, p: float = 0.5) -> np.ndarray:
    out = np.empty(count, dtype=np.float32)
    synth().ts_pm1(seed, stream, p, out.ctypes.data_as(POINTER(c_float)), count)
    return out


# Draw streams.
STREAM_FEATS, STREAM_W1, STREAM_W2, STREAM_LOGITS, STREAM_BIAS = 1, 2, 3, 4, 5

CONFIGS = {
    1: dict(name="cfg1_r64_sphere_conv64_f32", dtype=F32, ci=64, co=64),
    2: dict(name="cfg2_r256_shells_resblock128_f16", dtype=F16, ci=128, co=128),
    3: dict(name="cfg3_r512_subdivide_conv256to128_bf16", dtype=BF16, ci=256, co=128),
    4: dict(name="cfg4_r1024_shells_map_conv64_bf16", dtype=BF16, ci=64, co=64),
    5: dict(name="cfg5_batch4_blocks_conv512_bf16", dtype=BF16, ci=512, co=512),
}


def conv_weight(seed: int, stream: int, ci: int, co: int) -> np.ndarray:
    """W [co][27][ci] ~ N(0, 1/sqrt(27*ci)) (the reference layout, trellis_sparse_cpu.c:361)."""
    return normal(seed, stream, co * 27 * ci, 1.0 / math.sqrt(27.0 * ci)).reshape(co, 27, ci)


def workload(cfg: int) -> dict:
    """Inputs of one configuration as fp32 numpy arrays (not yet rounded to the storage type)."""
    c = dict(CONFIGS[cfg])
    c["cfg"] = cfg
    coords = make_coords(cfg)
    c["coords"] = coords
    if cfg == 3:
        npar = coords.shape[0]
        c["parent_coords"] = coords
        c["logits"] = pm1(cfg, STREAM_LOGITS, npar * 8, 0.5).reshape(npar, 8)
        c["parent_feats"] = normal(cfg, STREAM_FEATS, npar * c["ci"]).reshape(npar, c["ci"])
        c["weight"] = conv_weight(cfg, STREAM_W1, c["ci"], c["co"])
        c["bias"] = None
        return c
    n = coords.shape[0]
    c["feats"] = normal(cfg, STREAM_FEATS, n * c["ci"]).reshape(n, c["ci"])
    c["weight"] = conv_weight(cfg, STREAM_W1, c["ci"], c["co"])
    c["bias"] = None
    if cfg == 2:
        c["weight2"] = conv_weight(cfg, STREAM_W2, c["co"], c["co"])
        c["gamma"] = np.ones(c["co"], dtype=np.float32)
        c["beta"] = np.zeros(c["co"], dtype=np.float32)
    return c


def conv_flops(pairs: int, ci: int, co: int) -> float:
    """Effective work of one submanifold conv: 2 * P * Ci * Co."""
    return 2.0 * pairs * ci * co


def conv_bytes(n: int, ci: int, co: int, elem: int) -> float:
    """Compulsory conv traffic: features in and out, weights, neighbour table."""
    return n * ci * elem + n * co * elem + 27.0 * ci * co * elem + 108.0 * n


def hash_bytes(n: int) -> float:
    return 28.0 * n


def map_bytes(n: int, pairs: int) -> float:
    return 16.0 * n + 108.0 * n + 8.0 * pairs + 216.0


def subdivide_bytes(n_parent: int, m: int) -> float:
    return n_parent * 48.0 + m * 24.0


def broadcast_bytes(n_parent: int, m: int, ci: int, co: int, elem: int) -> float:
    return n_parent * ci * elem + m * co * elem
