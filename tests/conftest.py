"""pytest configuration: the `gpu` marker and import paths.

Tests marked `gpu` need a gfx950 GPU and the built libkd_fa.so; the rest
run on any host (oracle, host logic, C-ABI exports)."""
import os
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for sub in ("", "kandinsky.cpp_amd", "oracle", "tests"):
    p = os.path.join(ROOT, sub)
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a gfx950 GPU and the built HIP library")
