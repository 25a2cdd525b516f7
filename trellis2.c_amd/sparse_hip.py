"""ctypes binding of libtrellis_sparse_hip.so (the MI355X sparse-voxel backend).

The library exposes trellis2.c's sparse backend vtable
(reference: src/ops/sparse/trellis_sparse_backend.h:24-207).  This module
mirrors that struct field by field and wraps it in a small `Backend` class so
host code (tests, the benchmark) drives the GPU through exactly the entry
points a C caller would use.  numpy arrays carry host data; device memory stays
inside the library.

There is no fallback: if the shared library is missing, importing this module
raises, and every op raises `HipError` on a non-OK status.
"""
from __future__ import annotations

import ctypes
import os
from ctypes import (CFUNCTYPE, POINTER, Structure, c_char_p, c_double, c_float, c_int, c_int32, c_int64, c_size_t,
                    c_uint, c_uint32, c_void_p)

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libtrellis_sparse_hip.so")

# trellis_status (include/trellis.h:30-40)
OK, ERROR, INVALID_ARGUMENT, IO_ERROR, PARSE_ERROR, OUT_OF_MEMORY, CUDA_UNAVAILABLE, NOT_FOUND, NOT_IMPLEMENTED = range(9)
STATUS_NAMES = ["OK", "ERROR", "INVALID_ARGUMENT", "IO_ERROR", "PARSE_ERROR", "OUT_OF_MEMORY", "CUDA_UNAVAILABLE",
                "NOT_FOUND", "NOT_IMPLEMENTED"]
BACKEND_KIND_HIP = 3
TRIM_FREE_BUFFERS, TRIM_WEIGHTS = 1, 2

F32, F16, BF16 = 0, 1, 2
CONV_AUTO, CONV_GENERIC, CONV_MASKED, CONV_COMPACT = 0, 1, 2, 3
LINEAR_AUTO, LINEAR_KERNEL = 0, 1
STAGES = ["hash", "map", "conv", "subdivide", "broadcast", "elementwise"]

_p = c_void_p  # opaque pointers (buffer, rulebook, device map, backend)
_i32p = POINTER(c_int32)
_f32p = POINTER(c_float)

# Vtable slot types in declaration order (trellis_sparse_backend.h:24-201).
OPS_FIELDS = [
    ("destroy", CFUNCTYPE(None, _p)),
    ("alloc_f32", CFUNCTYPE(c_int, _p, c_size_t, POINTER(_p))),
    ("upload_f32", CFUNCTYPE(c_int, _p, _f32p, c_size_t, POINTER(_p))),
    ("upload_i32", CFUNCTYPE(c_int, _p, _i32p, c_size_t, POINTER(_p))),
    ("download_f32", CFUNCTYPE(c_int, _p, _p, _f32p, c_size_t)),
    ("free_buffer", CFUNCTYPE(None, _p, _p)),
    ("linear", CFUNCTYPE(c_int, _p, _p, _f32p, _f32p, _p, c_int64, c_int, c_int)),
    ("linear_silu", CFUNCTYPE(c_int, _p, _p, _f32p, _f32p, _p, c_int64, c_int, c_int)),
    ("row_norm", CFUNCTYPE(c_int, _p, _p, _f32p, _f32p, _p, c_int64, c_int, c_float)),
    ("row_norm_silu", CFUNCTYPE(c_int, _p, _p, _f32p, _f32p, _p, c_int64, c_int, c_float)),
    ("silu_inplace", CFUNCTYPE(c_int, _p, _p, c_size_t)),
    ("add", CFUNCTYPE(c_int, _p, _p, _p, _p, c_size_t)),
    ("build_rulebook", CFUNCTYPE(c_int, _p, _i32p, c_int64, POINTER(_p))),
    ("sparse_conv3d", CFUNCTYPE(c_int, _p, _p, _p, _f32p, _f32p, _p, c_int64, c_int, c_int)),
    ("free_rulebook", CFUNCTYPE(None, _p, _p)),
    ("c2s_gather", CFUNCTYPE(c_int, _p, _p, _i32p, _i32p, _p, c_int64, c_int)),
    ("skip_repeat", CFUNCTYPE(c_int, _p, _p, _i32p, _i32p, _p, c_int64, c_int, c_int)),
    ("build_c2s_map", CFUNCTYPE(c_int, _p, _i32p, _p, c_int64, POINTER(_i32p), POINTER(_i32p), POINTER(_i32p),
                                POINTER(c_int64))),
    ("alias_c2s_map", CFUNCTYPE(c_int, _p, _i32p, _i32p, _i32p, c_int64, _i32p, _i32p, _i32p)),
    ("build_c2s_map_device", CFUNCTYPE(c_int, _p, _i32p, _p, _p, c_int64, POINTER(_p), POINTER(c_int64))),
    ("build_rulebook_for_c2s_map", CFUNCTYPE(c_int, _p, _p, POINTER(_p))),
    ("c2s_gather_device", CFUNCTYPE(c_int, _p, _p, _p, _p, c_int64, c_int)),
    ("skip_repeat_device", CFUNCTYPE(c_int, _p, _p, _p, _p, c_int64, c_int, c_int)),
    ("download_c2s_coords", CFUNCTYPE(c_int, _p, _p, _i32p, c_int64)),
    ("download_c2s_map", CFUNCTYPE(c_int, _p, _p, _i32p, _i32p, _i32p, c_int64)),
    ("trim", CFUNCTYPE(c_int, _p, c_uint, POINTER(c_size_t))),
    ("pixal_naf_attention_project_sparse", CFUNCTYPE(c_int, _p, _f32p, _f32p, _f32p, _i32p, c_int64, _p, _p, _f32p,
                                                     c_size_t)),
]


class Ops(Structure):
    _fields_ = OPS_FIELDS


class BackendStruct(Structure):
    _fields_ = [("ops", POINTER(Ops)), ("kind", c_int), ("device", c_int)]


class Policy(Structure):
    _fields_ = [("struct_size", c_uint32), ("compute_dtype", c_int32), ("conv_algo", c_int32),
                ("cache_weights", c_int32), ("reject_duplicates", c_int32), ("linear_algo", c_int32)]


class StageTimes(Structure):
    _fields_ = [("ms", c_double * 6), ("launches", c_int64 * 6)]


class Mesh(Structure):
    """trellis_mesh_host (include/trellis.h:790-796)."""
    _fields_ = [("vertices", POINTER(c_float)), ("vertex_colors", POINTER(c_float)), ("faces", _i32p),
                ("n_vertices", c_int64), ("n_faces", c_int64)]


# The C ABI of include/trellis_sparse_hip.h: name -> (restype, argtypes).
ABI = {
    "trellis_sparse_hip_policy_init": (None, [POINTER(Policy)]),
    "trellis_sparse_hip_backend_create": (c_int, [c_int, POINTER(_p)]),
    "trellis_sparse_hip_backend_create_ex": (c_int, [c_int, POINTER(Policy), POINTER(_p)]),
    "trellis_sparse_hip_device_count": (c_int, []),
    "trellis_sparse_hip_last_error": (c_char_p, [_p]),
    "trellis_sparse_hip_synchronize": (c_int, [_p]),
    "trellis_sparse_hip_fail_alloc": (c_int, [_p, c_int64, c_int64]),
    "trellis_sparse_hip_rulebook_stats": (c_int, [_p, _p, POINTER(c_int64), POINTER(c_int64), POINTER(c_int64),
                                                  POINTER(c_int64)]),
    "trellis_sparse_hip_download_neighbors": (c_int, [_p, _p, _i32p, c_int64]),
    "trellis_sparse_hip_download_pairs": (c_int, [_p, _p, POINTER(c_int64), _i32p, _i32p, c_int64]),
    "trellis_sparse_hip_upload_raw": (c_int, [_p, c_void_p, c_size_t, POINTER(_p)]),
    "trellis_sparse_hip_download_raw": (c_int, [_p, _p, c_void_p, c_size_t]),
    "trellis_sparse_hip_upload_coords": (c_int, [_p, _i32p, c_int64, POINTER(_p)]),
    "trellis_sparse_hip_free_c2s_map": (c_int, [_p, _p]),
    "trellis_sparse_hip_build_c2s_map_into": (c_int, [_p, _p, _p, c_int64, _p, _p, _p, POINTER(c_int64)]),
    "trellis_sparse_hip_profile_enable": (c_int, [_p, c_int]),
    "trellis_sparse_hip_profile_read": (c_int, [_p, POINTER(StageTimes), c_int]),
    "trellis_sparse_hip_event_record": (c_int, [_p, c_int]),
    "trellis_sparse_hip_event_elapsed": (c_int, [_p, c_int, c_int, POINTER(c_float)]),
    "trellis_sparse_hip_s2c_build_device": (c_int, [_p, _i32p, _p, c_int64, POINTER(_p), POINTER(_p), POINTER(c_int64)]),
    "trellis_sparse_hip_s2c_pack_device": (c_int, [_p, _p, _p, _p, c_int]),
    "trellis_sparse_hip_s2c_skip_mean_device": (c_int, [_p, _p, _p, _p, c_int, c_int]),
    "trellis_sparse_hip_flex_dual_grid_mesh": (c_int, [_p, _i32p, _p, _p, c_int64, c_int, c_int, POINTER(Mesh)]),
    "trellis_sparse_hip_read_f32": (c_int, [c_char_p, POINTER(_f32p), POINTER(c_size_t)]),
    "trellis_sparse_hip_read_coords_i32": (c_int, [c_char_p, c_int, POINTER(_i32p), POINTER(c_int64)]),
    "trellis_sparse_hip_dump_open": (c_int, [c_char_p, c_char_p, POINTER(_p)]),
    "trellis_sparse_hip_dump_close": (c_int, [_p]),
    "trellis_sparse_hip_dump_host_f32": (c_int, [_p, c_char_p, _f32p, c_int64, c_int]),
    "trellis_sparse_hip_dump_host_i32": (c_int, [_p, c_char_p, _i32p, c_int64, c_int]),
    "trellis_sparse_hip_dump_buffer": (c_int, [_p, _p, c_char_p, _p, c_int64, c_int]),
    "trellis_sparse_hip_dump_map_coords": (c_int, [_p, _p, c_char_p, _p]),
    "trellis_sparse_hip_convnext_mlp": (c_int, [_p, _p, _f32p, _f32p, _f32p, _f32p, _f32p, _f32p, _p, _p, c_int64,
                                                c_int, c_float]),
    "trellis_sparse_hip_convnext_block": (c_int, [_p, _p, _p, _f32p, _f32p, _f32p, _f32p, _f32p, _f32p, _f32p, _f32p,
                                                  _p, c_int64, c_int, c_float]),
    "trellis_sparse_hip_conv_norm": (c_int, [_p, _p, _p, _f32p, _f32p, _f32p, _f32p, c_float, c_int, _p, c_int64,
                                             c_int, c_int]),
    "trellis_sparse_hip_conv_add": (c_int, [_p, _p, _p, _f32p, _f32p, _p, _p, c_int64, c_int, c_int]),
}


def load_library(path: str = LIB_PATH) -> ctypes.CDLL:
    if not os.path.exists(path):
        raise RuntimeError(f"{path} is missing: run __graft_entry__.build() (or make -C trellis2.c_amd) first")
    lib = ctypes.CDLL(path)
    for name, (res, args) in ABI.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    return lib


LIB = load_library()


def _status(st: int, what: str):
    if st != OK:
        raise HipError(st, what)


def _free(ptr):
    libc = ctypes.CDLL(None)
    libc.free.argtypes = [c_void_p]
    libc.free(ctypes.cast(ptr, c_void_p))


def read_f32(path: str) -> np.ndarray:
    """trellis_sparse_hip_read_f32: a whole file of floats."""
    p, n = _f32p(), c_size_t()
    _status(LIB.trellis_sparse_hip_read_f32(path.encode(), ctypes.byref(p), ctypes.byref(n)), "read_f32")
    try:
        return np.ctypeslib.as_array(p, shape=(n.value,)).copy() if n.value else np.zeros(0, np.float32)
    finally:
        _free(p)


def read_coords_i32(path: str, force_xyz: bool = False) -> np.ndarray:
    """trellis_sparse_hip_read_coords_i32: [N,4] or [N,3] (batch 0 added)."""
    p, n = _i32p(), c_int64()
    _status(LIB.trellis_sparse_hip_read_coords_i32(path.encode(), 1 if force_xyz else 0, ctypes.byref(p),
                                                   ctypes.byref(n)), "read_coords_i32")
    try:
        return np.ctypeslib.as_array(p, shape=(n.value, 4)).copy() if n.value else np.zeros((0, 4), np.int32)
    finally:
        _free(p)


class Dump:
    """trellis_sparse_hip_dump_*: a dump directory with a manifest."""

    def __init__(self, directory: str, manifest: str):
        self.h = c_void_p()
        _status(LIB.trellis_sparse_hip_dump_open(directory.encode(), manifest.encode(), ctypes.byref(self.h)),
                "dump_open")

    def host(self, name: str, a):
        """int32 arrays as .i32, floating arrays as .f32 (other dtypes are refused)."""
        a = np.asarray(a)
        if a.dtype != np.int32 and not np.issubdtype(a.dtype, np.floating):
            raise TypeError(f"dump {name}: int32 or floating data, not {a.dtype}")
        rows, cols = (a.shape[0], int(np.prod(a.shape[1:]))) if a.ndim > 1 else (a.size, 1)
        if a.dtype == np.int32:
            a = np.ascontiguousarray(a)
            _status(LIB.trellis_sparse_hip_dump_host_i32(self.h, name.encode(), _ptr(a, _i32p), rows, cols), "dump")
        else:
            a = np.ascontiguousarray(a, dtype=np.float32)
            _status(LIB.trellis_sparse_hip_dump_host_f32(self.h, name.encode(), _ptr(a, _f32p), rows, cols), "dump")

    def buffer(self, be, name: str, buf, rows: int, cols: int):
        _status(LIB.trellis_sparse_hip_dump_buffer(self.h, be.ptr, name.encode(), buf.handle, rows, cols), "dump")

    def map_coords(self, be, name: str, dmap):
        _status(LIB.trellis_sparse_hip_dump_map_coords(self.h, be.ptr, name.encode(), dmap.handle), "dump")

    def close(self):
        if self.h:
            _status(LIB.trellis_sparse_hip_dump_close(self.h), "dump_close")
            self.h = c_void_p()


class HipError(RuntimeError):
    def __init__(self, status: int, what: str, detail: str = ""):
        self.status = status
        name = STATUS_NAMES[status] if 0 <= status < len(STATUS_NAMES) else str(status)
        super().__init__(f"{what}: {name}" + (f" ({detail})" if detail else ""))


def device_count() -> int:
    return LIB.trellis_sparse_hip_device_count()


def _f32(a):
    return None if a is None else np.ascontiguousarray(a, dtype=np.float32)


def _ptr(a, t):
    return None if a is None else a.ctypes.data_as(t)


class Buffer:
    """A backend-owned device buffer (count elements of the storage type)."""

    def __init__(self, backend: "Backend", handle: c_void_p, count: int):
        self.backend = backend
        self.handle = handle
        self.count = count

    def free(self):
        if self.handle:
            self.backend.ops.free_buffer(self.backend.ptr, self.handle)
            self.handle = c_void_p()

    def __del__(self):
        try:
            if self.backend.alive:
                self.free()
        except Exception:
            pass


class Rulebook:
    def __init__(self, backend: "Backend", handle: c_void_p, n: int):
        self.backend = backend
        self.handle = handle
        self.n = n

    def free(self):
        if self.handle:
            self.backend.ops.free_rulebook(self.backend.ptr, self.handle)
            self.handle = c_void_p()

    def __del__(self):
        try:
            if self.backend.alive:
                self.free()
        except Exception:
            pass


class DeviceMap:
    """Backend-owned device C2S map (valid until the backend is destroyed)."""

    def __init__(self, handle: c_void_p, n: int):
        self.handle = handle
        self.n = n


class Backend:
    """One sparse backend instance on one device."""

    def __init__(self, device: int = 0, dtype: int = F32, conv_algo: int = CONV_AUTO, cache_weights: bool = True,
                 reject_duplicates: bool = False, linear_algo: int = LINEAR_AUTO):
        pol = Policy()
        LIB.trellis_sparse_hip_policy_init(ctypes.byref(pol))
        pol.compute_dtype = dtype
        pol.conv_algo = conv_algo
        pol.linear_algo = linear_algo
        pol.cache_weights = 1 if cache_weights else 0
        pol.reject_duplicates = 1 if reject_duplicates else 0
        out = c_void_p()
        st = LIB.trellis_sparse_hip_backend_create_ex(device, ctypes.byref(pol), ctypes.byref(out))
        if st != OK:
            raise HipError(st, "trellis_sparse_hip_backend_create_ex")
        self.ptr = out
        self.struct = ctypes.cast(out, POINTER(BackendStruct)).contents
        self.ops = self.struct.ops.contents
        self.dtype = dtype
        self.linear_algo = linear_algo
        self.alive = True
        self._keep = []  # host arrays whose pointers the weight cache is keyed on

    # -- housekeeping -------------------------------------------------------
    def _check(self, st: int, what: str):
        if st != OK:
            raise HipError(st, what, LIB.trellis_sparse_hip_last_error(self.ptr).decode())

    def destroy(self):
        if self.alive:
            self.ops.destroy(self.ptr)
            self.alive = False

    def __del__(self):
        try:
            self.destroy()
        except Exception:
            pass

    def synchronize(self):
        self._check(LIB.trellis_sparse_hip_synchronize(self.ptr), "synchronize")

    def fail_alloc(self, after: int, count: int = 1 << 62):
        """Device allocation attempts after .. after + count - 1 fail from now on (after < 0: off)."""
        self._check(LIB.trellis_sparse_hip_fail_alloc(self.ptr, after, count), "fail_alloc")

    def trim(self, flags: int) -> int:
        rel = c_size_t(0)
        self._check(self.ops.trim(self.ptr, flags, ctypes.byref(rel)), "trim")
        return rel.value

    def keep(self, arr):
        """Pins a host array for the backend's lifetime (weights are cached by pointer)."""
        self._keep.append(arr)
        return arr

    # -- buffers ------------------------------------------------------------
    def alloc(self, count: int) -> Buffer:
        h = c_void_p()
        self._check(self.ops.alloc_f32(self.ptr, count, ctypes.byref(h)), "alloc_f32")
        return Buffer(self, h, count)

    def upload(self, arr) -> Buffer:
        a = _f32(arr).ravel()
        h = c_void_p()
        self._check(self.ops.upload_f32(self.ptr, _ptr(a, _f32p), a.size, ctypes.byref(h)), "upload_f32")
        return Buffer(self, h, a.size)

    def upload_raw(self, arr) -> Buffer:
        a = np.ascontiguousarray(arr).ravel()
        h = c_void_p()
        self._check(LIB.trellis_sparse_hip_upload_raw(self.ptr, a.ctypes.data, a.size, ctypes.byref(h)), "upload_raw")
        return Buffer(self, h, a.size)

    def download(self, buf: Buffer, count: int | None = None) -> np.ndarray:
        count = buf.count if count is None else count
        out = np.empty(count, dtype=np.float32)
        self._check(self.ops.download_f32(self.ptr, buf.handle, _ptr(out, _f32p), count), "download_f32")
        return out

    def upload_i32(self, arr) -> Buffer:
        a = np.ascontiguousarray(arr, dtype=np.int32).ravel()
        h = c_void_p()
        self._check(self.ops.upload_i32(self.ptr, _ptr(a, _i32p), a.size, ctypes.byref(h)), "upload_i32")
        return Buffer(self, h, a.size)

    def download_i32(self, buf: Buffer, count: int | None = None) -> np.ndarray:
        """An int32 buffer (upload_i32) back to the host; download_f32 copies its bits unchanged."""
        count = buf.count if count is None else count
        out = np.empty(count, dtype=np.int32)
        self._check(self.ops.download_f32(self.ptr, buf.handle, out.ctypes.data_as(_f32p), count), "download_f32")
        return out

    def build_c2s_map_into(self, coords: Buffer, logits: Buffer, n: int, coords_out: Buffer, parent_out: Buffer,
                           subidx_out: Buffer) -> int:
        """Allocation-free subdivide into int32 buffers; returns the child count."""
        m = c_int64()
        st = LIB.trellis_sparse_hip_build_c2s_map_into(self.ptr, coords.handle, logits.handle, n, coords_out.handle,
                                                       parent_out.handle, subidx_out.handle, ctypes.byref(m))
        if st != OK:
            err = HipError(st, "build_c2s_map_into", LIB.trellis_sparse_hip_last_error(self.ptr).decode())
            err.n_out = m.value
            raise err
        return m.value

    def download_raw(self, buf: Buffer, count: int | None = None) -> np.ndarray:
        count = buf.count if count is None else count
        out = np.empty(count, dtype=np.float32 if self.dtype == F32 else np.uint16)
        self._check(LIB.trellis_sparse_hip_download_raw(self.ptr, buf.handle, out.ctypes.data, count), "download_raw")
        return out

    # -- rulebook / conv --------------------------------------------------------
    def build_rulebook(self, coords) -> Rulebook:
        c = np.ascontiguousarray(coords, dtype=np.int32).reshape(-1, 4)
        h = c_void_p()
        self._check(self.ops.build_rulebook(self.ptr, _ptr(c, _i32p), c.shape[0], ctypes.byref(h)), "build_rulebook")
        return Rulebook(self, h, c.shape[0])

    def rulebook_stats(self, rb: Rulebook):
        n, p, s, b = c_int64(), c_int64(), c_int64(), c_int64()
        self._check(LIB.trellis_sparse_hip_rulebook_stats(self.ptr, rb.handle, ctypes.byref(n), ctypes.byref(p),
                                                          ctypes.byref(s), ctypes.byref(b)), "rulebook_stats")
        return {"n": n.value, "pairs": p.value, "table_slots": s.value, "bricks": b.value}

    def neighbors(self, rb: Rulebook) -> np.ndarray:
        out = np.empty((rb.n, 27), dtype=np.int32)
        self._check(LIB.trellis_sparse_hip_download_neighbors(self.ptr, rb.handle, _ptr(out, _i32p), rb.n),
                    "download_neighbors")
        return out

    def pairs(self, rb: Rulebook):
        counts = (c_int64 * 27)()
        self._check(LIB.trellis_sparse_hip_download_pairs(self.ptr, rb.handle, counts, None, None, 0), "download_pairs")
        total = sum(counts)
        src = np.empty(total, dtype=np.int32)
        dst = np.empty(total, dtype=np.int32)
        self._check(LIB.trellis_sparse_hip_download_pairs(self.ptr, rb.handle, counts, _ptr(src, _i32p),
                                                          _ptr(dst, _i32p), total), "download_pairs")
        return np.array(list(counts), dtype=np.int64), src, dst

    def conv(self, rb: Rulebook, x: Buffer, weight, bias, out: Buffer, ci: int, co: int):
        w = self.keep(_f32(weight))
        b = None if bias is None else self.keep(_f32(bias))
        self._check(self.ops.sparse_conv3d(self.ptr, rb.handle, x.handle, _ptr(w, _f32p), _ptr(b, _f32p), out.handle,
                                           rb.n, ci, co), "sparse_conv3d")

    # -- dense row ops -------------------------------------------------------------
    def linear(self, x: Buffer, weight, bias, y: Buffer, n: int, ci: int, co: int, silu: bool = False):
        w = self.keep(_f32(weight))
        b = None if bias is None else self.keep(_f32(bias))
        fn = self.ops.linear_silu if silu else self.ops.linear
        self._check(fn(self.ptr, x.handle, _ptr(w, _f32p), _ptr(b, _f32p), y.handle, n, ci, co), "linear")

    def row_norm(self, x: Buffer, gamma, beta, y: Buffer, n: int, c: int, eps: float, silu: bool = False):
        g = None if gamma is None else self.keep(_f32(gamma))
        b = None if beta is None else self.keep(_f32(beta))
        fn = self.ops.row_norm_silu if silu else self.ops.row_norm
        self._check(fn(self.ptr, x.handle, _ptr(g, _f32p), _ptr(b, _f32p), y.handle, n, c, eps), "row_norm")

    def convnext_mlp(self, x: Buffer, gamma, beta, w0, b0, w2, b2, residual: Buffer, y: Buffer, n: int, c: int,
                     eps: float):
        """Fused row_norm -> linear_silu (c -> 4c) -> linear (4c -> c) -> add(residual, .)."""
        g, bt, b0a, b2a = (None if a is None else self.keep(_f32(a)) for a in (gamma, beta, b0, b2))
        w0a, w2a = self.keep(_f32(w0)), self.keep(_f32(w2))
        self._check(LIB.trellis_sparse_hip_convnext_mlp(self.ptr, x.handle, _ptr(g, _f32p), _ptr(bt, _f32p),
                                                        _ptr(w0a, _f32p), _ptr(b0a, _f32p), _ptr(w2a, _f32p),
                                                        _ptr(b2a, _f32p), residual.handle, y.handle, n, c, eps),
                    "convnext_mlp")

    def convnext_block(self, rb: Rulebook, h: Buffer, conv_w, conv_b, gamma, beta, w0, b0, w2, b2, out: Buffer,
                       c: int, eps: float):
        """The whole ConvNeXt block: out = h + MLP(row_norm(conv(h)))."""
        cw, w0a, w2a = self.keep(_f32(conv_w)), self.keep(_f32(w0)), self.keep(_f32(w2))
        cb, g, bt, b0a, b2a = (None if a is None else self.keep(_f32(a)) for a in (conv_b, gamma, beta, b0, b2))
        self._check(LIB.trellis_sparse_hip_convnext_block(self.ptr, rb.handle, h.handle, _ptr(cw, _f32p),
                                                          _ptr(cb, _f32p), _ptr(g, _f32p), _ptr(bt, _f32p),
                                                          _ptr(w0a, _f32p), _ptr(b0a, _f32p), _ptr(w2a, _f32p),
                                                          _ptr(b2a, _f32p), out.handle, rb.n, c, eps),
                    "convnext_block")

    def conv_norm(self, rb: Rulebook, x: Buffer, weight, bias, gamma, beta, eps: float, out: Buffer, ci: int,
                  co: int, silu: bool = False):
        """Fused sparse_conv3d -> row_norm(_silu); raises HipError(NOT_IMPLEMENTED) where it does not apply."""
        w = self.keep(_f32(weight))
        b, g, bt = (None if a is None else self.keep(_f32(a)) for a in (bias, gamma, beta))
        self._check(LIB.trellis_sparse_hip_conv_norm(self.ptr, rb.handle, x.handle, _ptr(w, _f32p), _ptr(b, _f32p),
                                                     _ptr(g, _f32p), _ptr(bt, _f32p), eps, int(silu), out.handle,
                                                     rb.n, ci, co), "conv_norm")

    def conv_add(self, rb: Rulebook, x: Buffer, weight, bias, residual: Buffer, out: Buffer, ci: int, co: int):
        """Fused sparse_conv3d -> add(residual); raises HipError(NOT_IMPLEMENTED) where it does not apply."""
        w = self.keep(_f32(weight))
        b = None if bias is None else self.keep(_f32(bias))
        self._check(LIB.trellis_sparse_hip_conv_add(self.ptr, rb.handle, x.handle, _ptr(w, _f32p), _ptr(b, _f32p),
                                                    residual.handle, out.handle, rb.n, ci, co), "conv_add")

    def silu_inplace(self, x: Buffer, count: int):
        self._check(self.ops.silu_inplace(self.ptr, x.handle, count), "silu_inplace")

    def add(self, a: Buffer, b: Buffer, y: Buffer, count: int):
        self._check(self.ops.add(self.ptr, a.handle, b.handle, y.handle, count), "add")

    # -- subdivide --------------------------------------------------------------
    def build_c2s_map(self, coords, logits: Buffer):
        c = np.ascontiguousarray(coords, dtype=np.int32).reshape(-1, 4)
        pc, pp, ps, m = _i32p(), _i32p(), _i32p(), c_int64()
        self._check(self.ops.build_c2s_map(self.ptr, _ptr(c, _i32p), logits.handle, c.shape[0], ctypes.byref(pc),
                                           ctypes.byref(pp), ctypes.byref(ps), ctypes.byref(m)), "build_c2s_map")
        libc = ctypes.CDLL(None)
        libc.free.argtypes = [c_void_p]
        try:
            coords_out = np.ctypeslib.as_array(pc, shape=(m.value, 4)).copy()
            parent = np.ctypeslib.as_array(pp, shape=(m.value,)).copy()
            subidx = np.ctypeslib.as_array(ps, shape=(m.value,)).copy()
        finally:
            for q in (pc, pp, ps):
                libc.free(ctypes.cast(q, c_void_p))
        return coords_out, parent, subidx

    def build_c2s_map_device(self, logits: Buffer, n: int, coords=None, coords_map: DeviceMap | None = None):
        c = None if coords is None else np.ascontiguousarray(coords, dtype=np.int32).reshape(-1, 4)
        h, m = c_void_p(), c_int64()
        self._check(self.ops.build_c2s_map_device(self.ptr, _ptr(c, _i32p), None if coords_map is None else
                                                  coords_map.handle, logits.handle, n, ctypes.byref(h),
                                                  ctypes.byref(m)), "build_c2s_map_device")
        return DeviceMap(h, m.value)

    def build_rulebook_for_c2s_map(self, dmap: DeviceMap) -> Rulebook:
        h = c_void_p()
        self._check(self.ops.build_rulebook_for_c2s_map(self.ptr, dmap.handle, ctypes.byref(h)),
                    "build_rulebook_for_c2s_map")
        return Rulebook(self, h, dmap.n)

    def download_c2s_map(self, dmap: DeviceMap):
        c = np.empty((dmap.n, 4), dtype=np.int32)
        p = np.empty(dmap.n, dtype=np.int32)
        s = np.empty(dmap.n, dtype=np.int32)
        self._check(self.ops.download_c2s_map(self.ptr, dmap.handle, _ptr(c, _i32p), _ptr(p, _i32p), _ptr(s, _i32p),
                                              dmap.n), "download_c2s_map")
        return c, p, s

    def download_c2s_coords(self, dmap: DeviceMap):
        c = np.empty((dmap.n, 4), dtype=np.int32)
        self._check(self.ops.download_c2s_coords(self.ptr, dmap.handle, _ptr(c, _i32p), dmap.n), "download_c2s_coords")
        return c

    def c2s_gather(self, x: Buffer, parent, subidx, y: Buffer, co: int):
        p = np.ascontiguousarray(parent, dtype=np.int32)
        s = np.ascontiguousarray(subidx, dtype=np.int32)
        self._check(self.ops.c2s_gather(self.ptr, x.handle, _ptr(p, _i32p), _ptr(s, _i32p), y.handle, p.size, co),
                    "c2s_gather")

    def skip_repeat(self, x: Buffer, parent, subidx, y: Buffer, ci: int, co: int):
        p = np.ascontiguousarray(parent, dtype=np.int32)
        s = np.ascontiguousarray(subidx, dtype=np.int32)
        self._check(self.ops.skip_repeat(self.ptr, x.handle, _ptr(p, _i32p), _ptr(s, _i32p), y.handle, p.size, ci, co),
                    "skip_repeat")

    def c2s_gather_device(self, x: Buffer, dmap: DeviceMap, y: Buffer, co: int):
        self._check(self.ops.c2s_gather_device(self.ptr, x.handle, dmap.handle, y.handle, dmap.n, co),
                    "c2s_gather_device")

    def skip_repeat_device(self, x: Buffer, dmap: DeviceMap, y: Buffer, ci: int, co: int):
        self._check(self.ops.skip_repeat_device(self.ptr, x.handle, dmap.handle, y.handle, dmap.n, ci, co),
                    "skip_repeat_device")

    def upload_coords(self, coords) -> DeviceMap:
        c = np.ascontiguousarray(coords, dtype=np.int32).reshape(-1, 4)
        h = c_void_p()
        self._check(LIB.trellis_sparse_hip_upload_coords(self.ptr, _ptr(c, _i32p), c.shape[0], ctypes.byref(h)),
                    "upload_coords")
        return DeviceMap(h, c.shape[0])

    # -- S2C downsample (encoder) ------------------------------------------------
    def s2c_build_device(self, coords=None, coords_map: DeviceMap | None = None, n: int | None = None):
        """(fine_map, coarse_map): the fine level's parent/subidx map and the
        coarse voxels; from host coordinates or a device coordinates map."""
        c = None if coords is None else np.ascontiguousarray(coords, dtype=np.int32).reshape(-1, 4)
        if n is None:
            n = coords_map.n if coords_map is not None else c.shape[0]
        hf, hc, m = c_void_p(), c_void_p(), c_int64()
        self._check(LIB.trellis_sparse_hip_s2c_build_device(self.ptr, _ptr(c, _i32p), None if coords_map is None else
                                                            coords_map.handle, n, ctypes.byref(hf), ctypes.byref(hc),
                                                            ctypes.byref(m)), "s2c_build_device")
        return DeviceMap(hf, n), DeviceMap(hc, m.value)

    def s2c_pack_device(self, x: Buffer, fine_map: DeviceMap, y: Buffer, co: int):
        self._check(LIB.trellis_sparse_hip_s2c_pack_device(self.ptr, x.handle, fine_map.handle, y.handle, co),
                    "s2c_pack_device")

    def s2c_skip_mean_device(self, x: Buffer, fine_map: DeviceMap, y: Buffer, ci: int, co: int):
        self._check(LIB.trellis_sparse_hip_s2c_skip_mean_device(self.ptr, x.handle, fine_map.handle, y.handle, ci, co),
                    "s2c_skip_mean_device")

    # -- FlexiDualGrid mesh ------------------------------------------------------
    def flex_dual_grid_mesh(self, feats: Buffer, n: int, channels: int, resolution: int, coords=None,
                            coords_map: DeviceMap | None = None):
        """(vertices [n][3] float32, faces [m][3] int32) from decoder logits on the device."""
        c = None if coords is None else np.ascontiguousarray(coords, dtype=np.int32).reshape(-1, 4)
        mesh = Mesh()
        self._check(LIB.trellis_sparse_hip_flex_dual_grid_mesh(self.ptr, _ptr(c, _i32p), None if coords_map is None
                                                               else coords_map.handle, feats.handle, n, channels,
                                                               resolution, ctypes.byref(mesh)), "flex_dual_grid_mesh")
        libc = ctypes.CDLL(None)
        libc.free.argtypes = [c_void_p]
        try:
            v = (np.ctypeslib.as_array(mesh.vertices, shape=(mesh.n_vertices, 3)).copy() if mesh.n_vertices
                 else np.zeros((0, 3), np.float32))
            f = (np.ctypeslib.as_array(mesh.faces, shape=(mesh.n_faces, 3)).copy() if mesh.n_faces
                 else np.zeros((0, 3), np.int32))
        finally:
            for q in (mesh.vertices, mesh.vertex_colors, mesh.faces):
                if q:
                    libc.free(ctypes.cast(q, c_void_p))
        return v, f

    def free_map(self, dmap: DeviceMap):
        self._check(LIB.trellis_sparse_hip_free_c2s_map(self.ptr, dmap.handle), "free_c2s_map")
        dmap.handle = c_void_p()

    # -- timing ---------------------------------------------------------------
    def profile(self, enable: bool):
        self._check(LIB.trellis_sparse_hip_profile_enable(self.ptr, 1 if enable else 0), "profile_enable")

    def profile_read(self, reset: bool = True):
        t = StageTimes()
        self._check(LIB.trellis_sparse_hip_profile_read(self.ptr, ctypes.byref(t), 1 if reset else 0), "profile_read")
        return {name: (t.ms[i], t.launches[i]) for i, name in enumerate(STAGES)}

    def event(self, slot: int):
        self._check(LIB.trellis_sparse_hip_event_record(self.ptr, slot), "event_record")

    def elapsed(self, a: int, b: int) -> float:
        ms = c_float()
        self._check(LIB.trellis_sparse_hip_event_elapsed(self.ptr, a, b, ctypes.byref(ms)), "event_elapsed")
        return ms.value


def bf16_round(a) -> np.ndarray:
    """fp32 -> bf16 -> fp32 with round-to-nearest-even (NaN kept quiet)."""
    a = np.ascontiguousarray(a, dtype=np.float32)
    u = a.view(np.uint32).astype(np.uint64)
    nan = (u & 0x7FFFFFFF) > 0x7F800000
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16) & 0xFFFF
    r = np.where(nan, (u >> 16) | 0x40, r).astype(np.uint32)
    return (r << 16).view(np.float32).reshape(a.shape)


def f16_round(a) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.float32).astype(np.float16).astype(np.float32)


def storage_round(a, dtype: int) -> np.ndarray:
    if dtype == BF16:
        return bf16_round(a)
    if dtype == F16:
        return f16_round(a)
    return np.ascontiguousarray(a, dtype=np.float32)
