"""bench.py's command-line contract, checked without a GPU: one GPU only
(--gpus above 1 exits with status 2 and says so), and no silent fallback when
no device is visible (status 1, for the configuration step and for every
alternative mode).  Runs only where no GPU driver node exists, so that no
process that has touched a GPU starts another program."""
import os
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
BENCH = os.path.join(ROOT, "bench.py")

pytestmark = pytest.mark.skipif(os.path.exists("/dev/kfd"), reason="a GPU driver node is present")


def run(*args):
    return subprocess.run([sys.executable, BENCH, *args], capture_output=True, text=True, timeout=120)


@pytest.mark.parametrize("n", [2, 8])
def test_more_than_one_gpu_is_refused(n):
    r = run("--gpus", str(n))
    assert r.returncode == 2
    assert "one GPU" in r.stderr and r.stdout == ""


@pytest.mark.parametrize("mode", [[], ["--config", "5"], ["--block", "c2s"], ["--decoder"], ["--encoder"],
                                  ["--calibrate"]])
def test_no_device_is_an_error(mode):
    r = run(*mode)
    assert r.returncode == 1
    assert "no HIP device" in r.stderr and r.stdout == ""
