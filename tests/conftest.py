"""pytest configuration: the `gpu` marker and import paths.

Tests marked `gpu` need an MI355X; everything else runs on the CPU.
"""
import os
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for sub in ("trellis2.c_amd", "tests"):
    path = os.path.join(ROOT, sub)
    if path not in sys.path:
        sys.path.insert(0, path)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: runs on an MI355X through the C ABI")
