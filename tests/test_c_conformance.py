"""The compiled C caller of include/trellis_sparse_hip.h (tests/c/
decoder_conformance.c): a two-level sparse decoder driven slot by slot
through backend->ops in the reference executor's order, checked against the
oracle chain, then trimmed and re-run guided by its device C2S map
(src/architectures/sparse_unet_decoder/executor.c:556-819;
tests/test_sparse_decoder_backend.c:69-153, :210-341)."""
import os
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
BIN = os.path.join(ROOT, "tests", "c", "decoder_conformance")


def run(*args, timeout=300):
    if not os.path.exists(BIN):
        raise RuntimeError(f"{BIN} is missing: run __graft_entry__.build() first")
    r = subprocess.run([BIN, *args], capture_output=True, text=True, timeout=timeout)
    print(r.stdout + r.stderr, flush=True)
    sys.stdout.flush()
    return r


def test_binary_links_and_rejects_bad_usage():
    """Built by build(): loads the product library and the oracle, checks its
    arguments before touching a device."""
    r = run("nope", "f32")
    assert r.returncode == 1 and "usage" in r.stderr


def test_binary_skips_without_device():
    import sparse_hip

    if sparse_hip.device_count() > 0:
        pytest.skip("a GPU is visible; covered by the gpu tests")
    assert run("tiny", "f32").returncode == 77


@pytest.mark.gpu
@pytest.mark.parametrize("model,dtype", [("tiny", "f32"), ("medium", "f32"), ("medium", "bf16")])
def test_decoder_conformance_from_c(model, dtype):
    r = run(model, dtype)
    assert r.returncode == 0 and "decoder conformance passed" in r.stdout
