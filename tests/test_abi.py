"""C ABI checks that need no GPU: the library loads, exports exactly the entry
points include/trellis_sparse_hip.h declares, and the vtable mirror matches the
reference struct (27 slots in the order of trellis_sparse_backend.h:24-201)."""
import ctypes
import os
import re
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "trellis_sparse_hip.h")


def declared_entry_points():
    text = open(HEADER).read()
    return sorted(set(re.findall(r"\b(trellis_sparse_hip_\w+)\s*\(", text)))


def test_library_exports_every_declared_symbol():
    import sparse_hip

    declared = declared_entry_points()
    assert len(declared) >= 10
    for name in declared:
        assert hasattr(sparse_hip.LIB, name), name
    assert sorted(sparse_hip.ABI) == declared
    out = subprocess.run(["nm", "-D", "--defined-only", sparse_hip.LIB_PATH], capture_output=True, text=True,
                         check=True).stdout
    exported = sorted(line.split()[-1] for line in out.splitlines() if " T " in line)
    assert exported == declared


def test_vtable_mirror_order_and_size():
    import sparse_hip

    names = [f[0] for f in sparse_hip.OPS_FIELDS]
    assert len(names) == 27
    assert names[:6] == ["destroy", "alloc_f32", "upload_f32", "upload_i32", "download_f32", "free_buffer"]
    assert names[12:15] == ["build_rulebook", "sparse_conv3d", "free_rulebook"]
    assert names[-2:] == ["trim", "pixal_naf_attention_project_sparse"]
    assert ctypes.sizeof(sparse_hip.Ops) == 27 * ctypes.sizeof(ctypes.c_void_p)
    # The header's struct lists the same slots in the same order.
    text = open(HEADER).read()
    body = text[text.index("typedef struct trellis_sparse_backend_ops"):text.index("} trellis_sparse_backend_ops;")]
    assert re.findall(r"\(\*(\w+)\)", body) == names


def test_status_and_kind_values_match_reference():
    import sparse_hip

    text = open(HEADER).read()
    for i, name in enumerate(sparse_hip.STATUS_NAMES):
        assert re.search(rf"TRELLIS_STATUS_{name} = {i}\b", text), name
    assert "TRELLIS_SPARSE_BACKEND_VULKAN = 2" in text
    assert sparse_hip.BACKEND_KIND_HIP == 3


def test_policy_struct_matches_header():
    import sparse_hip

    pol = sparse_hip.Policy()
    sparse_hip.LIB.trellis_sparse_hip_policy_init(ctypes.byref(pol))
    assert pol.struct_size == ctypes.sizeof(sparse_hip.Policy) == 24
    assert (pol.compute_dtype, pol.conv_algo, pol.cache_weights, pol.reject_duplicates, pol.linear_algo) == \
        (0, 0, 1, 0, sparse_hip.LINEAR_AUTO)


def test_create_without_device_reports_unavailable():
    import sparse_hip

    if sparse_hip.device_count() > 0:
        pytest.skip("a GPU is visible; covered by the gpu tests")
    out = ctypes.c_void_p(123)
    st = sparse_hip.LIB.trellis_sparse_hip_backend_create(0, ctypes.byref(out))
    assert st == sparse_hip.CUDA_UNAVAILABLE and not out.value
    assert sparse_hip.LIB.trellis_sparse_hip_backend_create(0, None) == sparse_hip.INVALID_ARGUMENT
    bad = sparse_hip.Policy()
    sparse_hip.LIB.trellis_sparse_hip_policy_init(ctypes.byref(bad))
    bad.struct_size = 4
    assert sparse_hip.LIB.trellis_sparse_hip_backend_create_ex(0, ctypes.byref(bad), ctypes.byref(out)) == \
        sparse_hip.INVALID_ARGUMENT
