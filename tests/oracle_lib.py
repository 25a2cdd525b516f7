"""ctypes binding of the CPU oracle (oracle/liborc.so) for the tests.

The oracle restates the reference CPU backend (src/ops/sparse/trellis_sparse_cpu.c)
and the decoder's host subdivide (sparse_unet_decoder/executor.c:108-154).  It is
the checker; only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline use it.
"""
import ctypes
import os
from ctypes import POINTER, c_float, c_int, c_int32, c_int64, c_size_t, c_uint64, c_void_p

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
ORC_PATH = os.path.join(ROOT, "oracle", "liborc.so")

_i32p = POINTER(c_int32)
_f32p = POINTER(c_float)


class OrcRulebook(ctypes.Structure):
    _fields_ = [("coords", _i32p), ("n", c_int64), ("keys", POINTER(c_uint64)), ("vals", _i32p), ("mask", c_int64)]


def _load():
    if not os.path.exists(ORC_PATH):
        raise RuntimeError(f"{ORC_PATH} missing: run make -C oracle")
    lib = ctypes.CDLL(ORC_PATH)
    sig = {
        "orc_set_mutation": (None, [c_int]),
        "orc_get_mutation": (c_int, []),
        "orc_pack_coord4": (c_uint64, [c_int32, c_int32, c_int32, c_int32]),
        "orc_hash_u64": (c_uint64, [c_uint64]),
        "orc_table_size": (c_int64, [c_int64]),
        "orc_rulebook_build": (c_int, [_i32p, c_int64, POINTER(OrcRulebook)]),
        "orc_rulebook_free": (None, [POINTER(OrcRulebook)]),
        "orc_rulebook_find": (c_int32, [POINTER(OrcRulebook), c_int32, c_int32, c_int32, c_int32]),
        "orc_neighbors": (None, [POINTER(OrcRulebook), _i32p]),
        "orc_neighbors_bruteforce": (None, [_i32p, c_int64, _i32p]),
        "orc_pairs": (c_int64, [_i32p, c_int64, POINTER(c_int64), _i32p, _i32p]),
        "orc_conv3d_rows": (c_int, [POINTER(OrcRulebook), _f32p, _f32p, _f32p, _f32p, c_int, c_int, c_int64, c_int64,
                                    c_int64]),
        "orc_conv3d_bruteforce": (None, [_i32p, _f32p, _f32p, _f32p, _f32p, c_int64, c_int, c_int, c_int, c_int, c_int,
                                         c_int, c_int, c_int]),
        "orc_c2s_map": (c_int, [_i32p, _f32p, c_int64, POINTER(_i32p), POINTER(_i32p), POINTER(_i32p),
                                POINTER(c_int64)]),
        "orc_free": (None, [c_void_p]),
        "orc_fdg_mesh": (c_int, [_i32p, _f32p, c_int64, c_int, c_int, POINTER(_f32p), POINTER(_i32p),
                                 POINTER(c_int64)]),
        "orc_s2c_map": (c_int, [_i32p, c_int64, POINTER(_i32p), POINTER(_i32p), POINTER(_i32p), POINTER(c_int64)]),
        "orc_s2c_pack": (None, [_f32p, _i32p, _i32p, _f32p, c_int64, c_int64, c_int]),
        "orc_s2c_skip_mean": (None, [_f32p, _i32p, _i32p, _f32p, c_int64, c_int64, c_int, c_int]),
        "orc_c2s_gather": (None, [_f32p, _i32p, _i32p, _f32p, c_int64, c_int]),
        "orc_skip_repeat": (None, [_f32p, _i32p, _i32p, _f32p, c_int64, c_int, c_int]),
        "orc_row_norm": (None, [_f32p, _f32p, _f32p, _f32p, c_int64, c_int, c_float, c_int]),
        "orc_silu": (None, [_f32p, c_size_t]),
        "orc_add": (None, [_f32p, _f32p, _f32p, c_size_t]),
        "orc_linear": (None, [_f32p, _f32p, _f32p, _f32p, c_int64, c_int, c_int, c_int]),
    }
    for name, (res, args) in sig.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    return lib


L = _load()


def _f(a):
    return None if a is None else np.ascontiguousarray(a, dtype=np.float32)


def _fp(a):
    return None if a is None else a.ctypes.data_as(_f32p)


def _ip(a):
    return None if a is None else a.ctypes.data_as(_i32p)


class mutation:
    """Context manager planting a mistake in the oracle (see trellis_oracle.h)."""

    def __init__(self, m):
        self.m = m

    def __enter__(self):
        L.orc_set_mutation(self.m)

    def __exit__(self, *a):
        L.orc_set_mutation(0)


class Rulebook:
    def __init__(self, coords):
        self.coords = np.ascontiguousarray(coords, dtype=np.int32).reshape(-1, 4)
        self.rb = OrcRulebook()
        rc = L.orc_rulebook_build(_ip(self.coords), self.coords.shape[0], ctypes.byref(self.rb))
        if rc != 0:
            raise RuntimeError(f"orc_rulebook_build: {rc}")
        self.n = self.coords.shape[0]

    def __del__(self):
        try:
            L.orc_rulebook_free(ctypes.byref(self.rb))
        except Exception:
            pass

    def find(self, b, x, y, z):
        return L.orc_rulebook_find(ctypes.byref(self.rb), b, x, y, z)

    def neighbors(self):
        out = np.empty((self.n, 27), dtype=np.int32)
        L.orc_neighbors(ctypes.byref(self.rb), _ip(out))
        return out

    def conv(self, feats, weight, bias, ci, co, rows=None):
        """Conv outputs for rows = range(begin, end, step) (default all)."""
        begin, end, step = (0, self.n, 1) if rows is None else rows
        count = len(range(begin, end, step))
        x, w, b = _f(feats), _f(weight), _f(bias)
        out = np.empty((count, co), dtype=np.float32)
        rc = L.orc_conv3d_rows(ctypes.byref(self.rb), _fp(x), _fp(w), _fp(b), _fp(out), ci, co, begin, end, step)
        if rc != 0:
            raise RuntimeError(f"orc_conv3d_rows: {rc}")
        return out


def neighbors_bruteforce(coords):
    c = np.ascontiguousarray(coords, dtype=np.int32).reshape(-1, 4)
    out = np.empty((c.shape[0], 27), dtype=np.int32)
    L.orc_neighbors_bruteforce(_ip(c), c.shape[0], _ip(out))
    return out


def pairs(nbr):
    nbr = np.ascontiguousarray(nbr, dtype=np.int32)
    n = nbr.shape[0]
    counts = (c_int64 * 27)()
    total = L.orc_pairs(_ip(nbr), n, counts, None, None)
    src = np.empty(total, dtype=np.int32)
    dst = np.empty(total, dtype=np.int32)
    L.orc_pairs(_ip(nbr), n, counts, _ip(src), _ip(dst))
    return np.array(list(counts), dtype=np.int64), src, dst


def conv_bruteforce(coords, feats, weight, bias, ci, co, kernel=(3, 3, 3), dilation=(1, 1, 1)):
    c = np.ascontiguousarray(coords, dtype=np.int32).reshape(-1, 4)
    x, w, b = _f(feats), _f(weight), _f(bias)
    out = np.empty((c.shape[0], co), dtype=np.float32)
    L.orc_conv3d_bruteforce(_ip(c), _fp(x), _fp(w), _fp(b), _fp(out), c.shape[0], ci, co, *kernel, *dilation)
    return out


def c2s_map(coords, logits):
    c = np.ascontiguousarray(coords, dtype=np.int32).reshape(-1, 4)
    lg = _f(logits)
    pc, pp, ps, m = _i32p(), _i32p(), _i32p(), c_int64()
    rc = L.orc_c2s_map(_ip(c), _fp(lg), c.shape[0], ctypes.byref(pc), ctypes.byref(pp), ctypes.byref(ps),
                       ctypes.byref(m))
    if rc != 0:
        return rc, None, None, None
    try:
        return (0, np.ctypeslib.as_array(pc, shape=(m.value, 4)).copy(),
                np.ctypeslib.as_array(pp, shape=(m.value,)).copy(), np.ctypeslib.as_array(ps, shape=(m.value,)).copy())
    finally:
        for q in (pc, pp, ps):
            L.orc_free(ctypes.cast(q, c_void_p))


def fdg_mesh(coords, feats, resolution):
    """(rc, vertices [n][3], faces [n_faces][3]); rc 0 ok, 2 bad argument, 4 rejected input."""
    c = np.ascontiguousarray(coords, dtype=np.int32).reshape(-1, 4)
    f = _f(feats).reshape(c.shape[0], -1) if c.shape[0] else np.zeros((0, 7), np.float32)
    pv, pf, nf = _f32p(), _i32p(), c_int64()
    rc = L.orc_fdg_mesh(_ip(c), _fp(np.ascontiguousarray(f)), c.shape[0], f.shape[1], resolution, ctypes.byref(pv),
                        ctypes.byref(pf), ctypes.byref(nf))
    if rc != 0:
        return rc, None, None
    try:
        v = np.ctypeslib.as_array(pv, shape=(c.shape[0], 3)).copy() if c.shape[0] else np.zeros((0, 3), np.float32)
        fc = np.ctypeslib.as_array(pf, shape=(nf.value, 3)).copy() if nf.value else np.zeros((0, 3), np.int32)
        return 0, v, fc
    finally:
        for q in (pv, pf):
            if q:
                L.orc_free(ctypes.cast(q, c_void_p))


def s2c_map(fine_coords):
    """(rc, coarse [m][4], parent [n], subidx [n]); rc 0 ok, 2 bad input, 4 duplicate."""
    c = np.ascontiguousarray(fine_coords, dtype=np.int32).reshape(-1, 4)
    pc, pp, ps, m = _i32p(), _i32p(), _i32p(), c_int64()
    rc = L.orc_s2c_map(_ip(c), c.shape[0], ctypes.byref(pc), ctypes.byref(pp), ctypes.byref(ps), ctypes.byref(m))
    if rc != 0:
        return rc, None, None, None
    n = c.shape[0]
    try:
        return (0, np.ctypeslib.as_array(pc, shape=(m.value, 4)).copy(),
                np.ctypeslib.as_array(pp, shape=(n,)).copy(), np.ctypeslib.as_array(ps, shape=(n,)).copy())
    finally:
        for q in (pc, pp, ps):
            L.orc_free(ctypes.cast(q, c_void_p))


def s2c_pack(x, parent, subidx, n_coarse, co):
    x = _f(x)
    p = np.ascontiguousarray(parent, dtype=np.int32)
    s = np.ascontiguousarray(subidx, dtype=np.int32)
    y = np.empty((n_coarse, co), dtype=np.float32)
    L.orc_s2c_pack(_fp(x), _ip(p), _ip(s), _fp(y), p.size, n_coarse, co)
    return y


def s2c_skip_mean(x, parent, subidx, n_coarse, ci, co):
    x = _f(x)
    p = np.ascontiguousarray(parent, dtype=np.int32)
    s = np.ascontiguousarray(subidx, dtype=np.int32)
    y = np.empty((n_coarse, co), dtype=np.float32)
    L.orc_s2c_skip_mean(_fp(x), _ip(p), _ip(s), _fp(y), p.size, n_coarse, ci, co)
    return y


def c2s_gather(x, parent, subidx, co):
    x = _f(x)
    p = np.ascontiguousarray(parent, dtype=np.int32)
    s = np.ascontiguousarray(subidx, dtype=np.int32)
    y = np.empty((p.size, co), dtype=np.float32)
    L.orc_c2s_gather(_fp(x), _ip(p), _ip(s), _fp(y), p.size, co)
    return y


def skip_repeat(x, parent, subidx, ci, co):
    x = _f(x)
    p = np.ascontiguousarray(parent, dtype=np.int32)
    s = np.ascontiguousarray(subidx, dtype=np.int32)
    y = np.empty((p.size, co), dtype=np.float32)
    L.orc_skip_repeat(_fp(x), _ip(p), _ip(s), _fp(y), p.size, ci, co)
    return y


def row_norm(x, gamma, beta, n, c, eps, silu=False):
    x, g, b = _f(x), _f(gamma), _f(beta)
    y = np.empty((n, c), dtype=np.float32)
    L.orc_row_norm(_fp(x), _fp(g), _fp(b), _fp(y), n, c, eps, 1 if silu else 0)
    return y


def silu(x):
    y = np.array(x, dtype=np.float32, copy=True)
    L.orc_silu(_fp(y), y.size)
    return y


def add(a, b):
    a, b = _f(a), _f(b)
    y = np.empty_like(a)
    L.orc_add(_fp(a), _fp(b), _fp(y), a.size)
    return y


def linear(x, w, bias, n, ci, co, silu=False):
    x, w, b = _f(x), _f(w), _f(bias)
    y = np.empty((n, co), dtype=np.float32)
    L.orc_linear(_fp(x), _fp(w), _fp(b), _fp(y), n, ci, co, 1 if silu else 0)
    return y


def pack_coord4(b, x, y, z):
    return L.orc_pack_coord4(b, x, y, z)


def hash_u64(v):
    return L.orc_hash_u64(v)


def table_size(n):
    return L.orc_table_size(n)
