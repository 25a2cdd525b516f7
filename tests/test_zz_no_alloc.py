"""The allocation-free subdivide (trellis_sparse_hip_build_c2s_map_into)
against the allocating entry point it is a variant of, build_c2s_map_device
(src/architectures/sparse_unet_decoder/executor.c:108-154 semantics): the
same children, bit for bit, on two calls in a row, the second with fewer
parents than the first (its scratch keeps the first call's counts beyond
the second's parents, which must not leak into the result), and with every
device allocation attempt failing (the backend's allocation-failure hook
after its buffer pool is emptied), which the call must not notice; then the
argument errors: more parents than its scratch holds, outputs smaller than
the child count (reported in n_out), no children."""
import sys

import numpy as np
import pytest

import sparse_hip as sh
import workloads as wl

pytestmark = pytest.mark.gpu


def say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


@pytest.mark.parametrize("dtype", [sh.BF16, sh.F32])
def test_build_c2s_map_into_matches_device_map(dtype):
    be = sh.Backend(0, dtype)
    try:
        w = wl.workload(3)
        pc_all, lg_all = w["parent_coords"], w["logits"]
        for npar in (300000, 4099):
            pc, lg = np.ascontiguousarray(pc_all[:npar]), np.ascontiguousarray(lg_all[:npar])
            lgb = be.upload(lg)
            dm = be.build_c2s_map_device(lgb, npar, coords=pc)
            ec, ep, es = be.download_c2s_map(dm)
            cb = be.upload_i32(pc)
            cap = 8 * npar
            oc = be.upload_i32(np.full(4 * cap, -7, np.int32))
            op = be.upload_i32(np.full(cap, -7, np.int32))
            os_ = be.upload_i32(np.full(cap, -7, np.int32))
            # Every device allocation fails from here: the call allocates nothing.
            be.trim(sh.TRIM_FREE_BUFFERS)
            be.fail_alloc(0)
            try:
                m = be.build_c2s_map_into(cb, lgb, npar, oc, op, os_)
            finally:
                be.fail_alloc(-1)
            say(f"build_c2s_map_into dtype={dtype} parents={npar}: {m} children (device map {dm.n})")
            assert m == dm.n
            assert np.array_equal(be.download_i32(oc, 4 * m).reshape(m, 4), ec)
            assert np.array_equal(be.download_i32(op, m), ep)
            assert np.array_equal(be.download_i32(os_, m), es)
            # Past the children the outputs are untouched.
            assert np.all(be.download_i32(op)[m:] == -7)
            be.free_map(dm)
    finally:
        be.destroy()


def test_build_c2s_map_into_errors():
    be = sh.Backend(0, sh.BF16)
    try:
        rng = np.random.default_rng(3)
        n = 1000
        pc = np.stack([np.zeros(n), rng.integers(0, 100, n), rng.integers(0, 100, n), rng.integers(0, 100, n)],
                      1).astype(np.int32)
        lg = np.where(rng.random((n, 8)) < 0.5, 1.0, -1.0).astype(np.float32)
        m_exp = int((lg > 0).sum())
        cb, lgb = be.upload_i32(pc), be.upload(lg)
        small = [be.upload_i32(np.zeros(k, np.int32)) for k in (4 * 10, 10, 10)]
        with pytest.raises(sh.HipError) as e:
            be.build_c2s_map_into(cb, lgb, n, *small)
        assert e.value.status == sh.INVALID_ARGUMENT and e.value.n_out == m_exp
        assert np.all(be.download_i32(small[1]) == 0)
        big_n = (1 << 20) + 1
        with pytest.raises(sh.HipError) as e:
            be.build_c2s_map_into(be.upload_i32(np.zeros(4 * big_n, np.int32)), be.alloc(8 * big_n), big_n, *small)
        assert e.value.status == sh.INVALID_ARGUMENT and "1048576" in str(e.value)
        with pytest.raises(sh.HipError) as e:
            be.build_c2s_map_into(cb, be.upload(-np.ones((n, 8), np.float32)), n, *small)
        assert e.value.status == sh.ERROR
        with pytest.raises(sh.HipError) as e:  # logits of the wrong storage type (an int32 buffer)
            be.build_c2s_map_into(cb, cb, n, *small)
        assert e.value.status == sh.INVALID_ARGUMENT
    finally:
        be.destroy()
