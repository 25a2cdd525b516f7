"""The compiled C callers of include/trellis_sparse_hip.h (tests/c/):

decoder_conformance.c - a two-level sparse decoder driven slot by slot
through backend->ops in the reference executor's order, checked against the
oracle chain, then trimmed and re-run guided by its device C2S map
(src/architectures/sparse_unet_decoder/executor.c:556-819;
tests/test_sparse_decoder_backend.c:69-153, :210-341).

encoder_conformance.c - the sparse encoder through backend->ops and the
device S2C entry points in the reference executor's order
(src/architectures/sparse_unet_encoder/executor.c:160-360, :392-649), checked
against the oracle chain and, for the reference test's tiny encoder, against
that test's known answers (tests/test_sparse_encoder_backend.c:84-161)."""
import os
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
BIN = os.path.join(ROOT, "tests", "c", "decoder_conformance")
ENC_BIN = os.path.join(ROOT, "tests", "c", "encoder_conformance")


def run(*args, timeout=300, binary=BIN):
    if not os.path.exists(binary):
        raise RuntimeError(f"{binary} is missing: run __graft_entry__.build() first")
    r = subprocess.run([binary, *args], capture_output=True, text=True, timeout=timeout)
    print(r.stdout + r.stderr, flush=True)
    sys.stdout.flush()
    return r


@pytest.mark.parametrize("binary", [BIN, ENC_BIN])
def test_binary_links_and_rejects_bad_usage(binary):
    """Built by build(): loads the product library and the oracle, checks its
    arguments before touching a device."""
    r = run("nope", "f32", binary=binary)
    assert r.returncode == 1 and "usage" in r.stderr


@pytest.mark.parametrize("binary", [BIN, ENC_BIN])
def test_binary_skips_without_device(binary):
    import sparse_hip

    if sparse_hip.device_count() > 0:
        pytest.skip("a GPU is visible; covered by the gpu tests")
    assert run("tiny", "f32", binary=binary).returncode == 77


@pytest.mark.parametrize("model,dtype", [("tiny", "f32"), ("tiny", "bf16"), ("medium", "f32")])
def test_encoder_oracle_chain(model, dtype):
    """No device: the encoder's oracle chain (the checker of the GPU run)
    reproduces the reference test's known answers for the tiny encoder -
    coarse voxels, guide, coarse features, closed-form latent - and runs the
    medium model through three levels."""
    r = run(model, dtype, "oracle", binary=ENC_BIN)
    assert r.returncode == 0 and "encoder oracle passed" in r.stdout


@pytest.mark.gpu
@pytest.mark.parametrize("model,dtype", [("tiny", "f32"), ("medium", "f32"), ("medium", "bf16")])
def test_decoder_conformance_from_c(model, dtype):
    r = run(model, dtype)
    assert r.returncode == 0 and "decoder conformance passed" in r.stdout


@pytest.mark.gpu
@pytest.mark.parametrize("model,dtype", [("tiny", "f32"), ("tiny", "bf16"), ("medium", "f32"), ("medium", "bf16")])
def test_encoder_conformance_from_c(model, dtype):
    r = run(model, dtype, binary=ENC_BIN)
    assert r.returncode == 0 and "encoder conformance passed" in r.stdout
