"""Out-of-memory paths through the C ABI, forced with the allocation-failure
hook (trellis_sparse_hip_fail_alloc / TRELLIS_HIP_FAIL_ALLOC_AFTER).

The reference reports an exhausted device as TRELLIS_STATUS_OUT_OF_MEMORY
with the call's outputs NULL (include/trellis.h:30-40), and its Vulkan
backend trims its caches and retries once before giving up
(trellis_sparse_vulkan.c:533-561).  Here:
  * every slot that needs device memory returns OUT_OF_MEMORY, with its
    output handles NULL and counts 0, when every allocation fails;
  * the same call succeeds once the hook is off, so the backend stays usable;
  * an allocation that fails while the pool holds free blocks empties the
    pool and succeeds on the retry; when the retry fails too the status is
    OUT_OF_MEMORY, and with nothing pooled there is no retry.
No real device memory is exhausted: the hook fails attempts before hipMalloc.
"""
import ctypes
import os
import subprocess
import sys
from ctypes import POINTER, c_int32, c_int64, c_void_p

import numpy as np
import pytest

import sparse_hip as sh
import workloads as wl

pytestmark = pytest.mark.gpu

SENTINEL = 0x5A5A5A5A


def say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def i32p(a):
    return a.ctypes.data_as(POINTER(c_int32))


def f32p(a):
    return None if a is None else a.ctypes.data_as(POINTER(ctypes.c_float))


@pytest.fixture()
def bf():
    b = sh.Backend(0, sh.BF16)
    yield b
    b.fail_alloc(-1)
    b.destroy()


def starve(be):
    """Empties the pool and the weight cache, then fails every allocation."""
    be.synchronize()
    be.trim(sh.TRIM_FREE_BUFFERS | sh.TRIM_WEIGHTS)
    be.fail_alloc(0)


def test_each_slot_reports_out_of_memory_and_recovers(bf):
    be = bf
    ops, p = be.ops, be.ptr
    coords = np.ascontiguousarray(wl.make_coords(1)[:700])
    n = coords.shape[0]
    ci = co = 64
    rng = np.random.default_rng(0)
    x = rng.standard_normal((n, ci)).astype(np.float32)
    w = be.keep((rng.standard_normal((co, 27, ci)) * 0.02).astype(np.float32))
    lw = be.keep((rng.standard_normal((co, ci)) * 0.1).astype(np.float32))
    g = be.keep(np.ones(ci, np.float32))
    logits = np.where(rng.standard_normal((n, 8)) > 0, 1.0, -1.0).astype(np.float32)
    parent = np.ascontiguousarray(np.sort(rng.integers(0, n, 900)).astype(np.int32))
    sub = np.ascontiguousarray(rng.integers(0, 8, 900).astype(np.int32))
    fdg = np.ascontiguousarray(np.abs(coords) % 60)
    fdg[:, 0] = 0
    fdg = np.unique(fdg, axis=0).astype(np.int32)

    # Live inputs, created before the starvation.
    xb = be.upload(x)
    yb = be.alloc(n * co)
    big = be.alloc(900 * 8 * co)
    lgb = be.upload(logits)
    rb = be.build_rulebook(coords)
    dm = be.build_c2s_map_device(lgb, n, coords=coords)
    ffeats = be.upload(rng.standard_normal((fdg.shape[0], 7)).astype(np.float32))

    def h():
        return c_void_p(SENTINEL)

    def slot_alloc():
        out = h()
        st = ops.alloc_f32(p, 1 << 20, ctypes.byref(out))
        return st, [out.value]

    def slot_upload():
        out = h()
        st = ops.upload_f32(p, f32p(x), x.size, ctypes.byref(out))
        return st, [out.value]

    def slot_upload_i32():
        out = h()
        st = ops.upload_i32(p, i32p(coords), coords.size, ctypes.byref(out))
        return st, [out.value]

    def slot_rulebook():
        out = h()
        st = ops.build_rulebook(p, i32p(coords), n, ctypes.byref(out))
        return st, [out.value]

    def slot_conv():
        return ops.sparse_conv3d(p, rb.handle, xb.handle, f32p(w), None, yb.handle, n, ci, co), []

    def slot_linear():
        return ops.linear(p, xb.handle, f32p(lw), None, yb.handle, n, ci, co), []

    def slot_row_norm():
        return ops.row_norm(p, xb.handle, f32p(g), None, yb.handle, n, ci, 1e-6), []

    def slot_c2s_gather():
        return ops.c2s_gather(p, big.handle, i32p(parent), i32p(sub), yb.handle, 900, 8), []

    def slot_skip_repeat():
        return ops.skip_repeat(p, xb.handle, i32p(parent), i32p(sub), big.handle, 900, ci, co), []

    def slot_c2s_host():
        c, pa, s, m = POINTER(c_int32)(), POINTER(c_int32)(), POINTER(c_int32)(), c_int64(SENTINEL)
        st = ops.build_c2s_map(p, i32p(coords), lgb.handle, n, ctypes.byref(c), ctypes.byref(pa), ctypes.byref(s),
                               ctypes.byref(m))
        outs = [ctypes.cast(c, c_void_p).value, ctypes.cast(pa, c_void_p).value, ctypes.cast(s, c_void_p).value,
                m.value]
        if st == sh.OK:
            for ptr in outs[:3]:
                sh._free(ptr)
        return st, outs

    def slot_c2s_device():
        out, m = h(), c_int64(SENTINEL)
        st = ops.build_c2s_map_device(p, i32p(coords), None, lgb.handle, n, ctypes.byref(out), ctypes.byref(m))
        return st, [out.value, m.value]

    def slot_rulebook_for_map():
        out = h()
        st = ops.build_rulebook_for_c2s_map(p, dm.handle, ctypes.byref(out))
        if st == sh.OK:
            be.synchronize()
        return st, [out.value]

    def slot_upload_coords():
        out = h()
        st = sh.LIB.trellis_sparse_hip_upload_coords(p, i32p(coords), n, ctypes.byref(out))
        return st, [out.value]

    def slot_s2c():
        f, c, m = h(), h(), c_int64(SENTINEL)
        st = sh.LIB.trellis_sparse_hip_s2c_build_device(p, i32p(fdg), None, fdg.shape[0], ctypes.byref(f),
                                                        ctypes.byref(c), ctypes.byref(m))
        return st, [f.value, c.value, m.value]

    def slot_mesh():
        mesh = sh.Mesh()
        st = sh.LIB.trellis_sparse_hip_flex_dual_grid_mesh(p, i32p(fdg), None, ffeats.handle, fdg.shape[0], 7, 64,
                                                           ctypes.byref(mesh))
        outs = [ctypes.cast(mesh.vertices, c_void_p).value, ctypes.cast(mesh.faces, c_void_p).value,
                mesh.n_vertices, mesh.n_faces]
        if st == sh.OK:
            for ptr in outs[:2]:
                sh._free(ptr)
        return st, outs

    slots = [slot_alloc, slot_upload, slot_upload_i32, slot_rulebook, slot_conv, slot_linear, slot_row_norm,
             slot_c2s_gather, slot_skip_repeat, slot_c2s_host, slot_c2s_device, slot_rulebook_for_map,
             slot_upload_coords, slot_s2c, slot_mesh]
    for slot in slots:
        starve(be)
        st, outs = slot()
        be.fail_alloc(-1)
        say(f"{slot.__name__}: status {sh.STATUS_NAMES[st]} outputs {outs}")
        assert st == sh.OUT_OF_MEMORY, slot.__name__
        assert all(not v for v in outs), f"{slot.__name__}: outputs not cleared: {outs}"
        assert "hipMalloc" in sh.LIB.trellis_sparse_hip_last_error(p).decode()
        st2, _ = slot()
        assert st2 == sh.OK, f"{slot.__name__} after recovery: {sh.STATUS_NAMES[st2]}"

    # The inputs survived every failure: the conv still gives the same rows.
    be.conv(rb, xb, w, None, yb, ci, co)
    a = be.download(yb)
    starve(be)
    be.fail_alloc(-1)
    be.conv(rb, xb, w, None, yb, ci, co)
    assert np.array_equal(a, be.download(yb))
    rb.free()


def test_wide_linear_out_of_memory_and_recovers(bf):
    """A wide linear (Ci = Co = 256, n >= 2048: the GEMM library's route)
    under starvation: the library's workspace cannot be taken, the kernel
    route's weight upload fails too, and the slot returns OUT_OF_MEMORY; with
    the hook off the same call gives the result of the unstarved call."""
    be = bf
    n, ci, co = 2048, 256, 256
    rng = np.random.default_rng(4)
    x = rng.standard_normal((n, ci)).astype(np.float32)
    lw = be.keep((rng.standard_normal((co, ci)) * 0.05).astype(np.float32))
    xb, yb = be.upload(x), be.alloc(n * co)
    be.linear(xb, lw, None, yb, n, ci, co, silu=True)
    ref = be.download(yb)
    y2 = be.alloc(n * co)
    starve(be)
    st = be.ops.linear_silu(be.ptr, xb.handle, f32p(lw), None, y2.handle, n, ci, co)
    be.fail_alloc(-1)
    assert st == sh.OUT_OF_MEMORY
    be.linear(xb, lw, None, y2, n, ci, co, silu=True)
    assert np.array_equal(be.download(y2), ref)


def test_retry_releases_the_pool(bf):
    be = bf
    be.synchronize()
    be.trim(sh.TRIM_FREE_BUFFERS | sh.TRIM_WEIGHTS)
    # A pooled block of one size class ...
    a = be.alloc(1 << 20)
    a.free()
    # ... then an allocation of another class whose first attempt fails:
    # the pool is released and the retry succeeds.
    be.fail_alloc(0, 1)
    b = be.alloc(3 << 20)
    be.fail_alloc(-1)
    assert be.trim(sh.TRIM_FREE_BUFFERS) == 0, "the retry emptied the pool"
    b.free()
    # Both attempts fail: OUT_OF_MEMORY, and the pool is still released.
    c = be.alloc(1 << 20)
    c.free()
    be.fail_alloc(0, 2)
    with pytest.raises(sh.HipError) as e:
        be.alloc(5 << 20)
    assert e.value.status == sh.OUT_OF_MEMORY
    be.fail_alloc(-1)
    assert be.trim(sh.TRIM_FREE_BUFFERS) == 0
    # Nothing pooled: no retry, one failed attempt is enough.
    be.fail_alloc(0, 1)
    with pytest.raises(sh.HipError) as e:
        be.alloc(7 << 20)
    assert e.value.status == sh.OUT_OF_MEMORY
    d = be.alloc(7 << 20)  # the hook's one failure is spent
    be.fail_alloc(-1)
    d.free()


def test_fail_alloc_rejects_bad_arguments(bf):
    assert sh.LIB.trellis_sparse_hip_fail_alloc(None, 0, 1) == sh.INVALID_ARGUMENT
    assert sh.LIB.trellis_sparse_hip_fail_alloc(bf.ptr, 0, 0) == sh.INVALID_ARGUMENT


def test_environment_hook_at_creation():
    """TRELLIS_HIP_FAIL_ALLOC_AFTER=1,1: the first allocation succeeds, the
    second fails, the third succeeds (run in a child process so the variable
    does not reach other backends)."""
    code = (
        "import sparse_hip as sh\n"
        "be = sh.Backend(0, sh.F32)\n"
        "a = be.alloc(1 << 20)\n"
        "try:\n"
        "    be.alloc(2 << 20)\n"
        "    raise SystemExit('second allocation did not fail')\n"
        "except sh.HipError as e:\n"
        "    assert e.status == sh.OUT_OF_MEMORY, e.status\n"
        "b = be.alloc(2 << 20)\n"
        "be.destroy()\n"
        "print('env hook ok')\n")
    env = dict(os.environ, TRELLIS_HIP_FAIL_ALLOC_AFTER="1,1")
    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    env["PYTHONPATH"] = os.pathsep.join([os.path.join(root, "trellis2.c_amd"), env.get("PYTHONPATH", "")])
    r = subprocess.run([sys.executable, "-c", code], env=env, capture_output=True, text=True, timeout=120)
    say(r.stdout + r.stderr)
    assert r.returncode == 0 and "env hook ok" in r.stdout
