"""Pytest setup: import paths and the `gpu` marker.

`-m "not gpu"` runs the oracle checks, host logic and the C-ABI load checks on
the CPU; `-m gpu` runs the HIP parity tests (they call the kernels through the
C-ABI and need a visible gfx950 device)."""
import os
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG_DIR = os.path.join(ROOT, "hierarchical-block-attention_amd")
for p in (ROOT, PKG_DIR, os.path.join(ROOT, "tests", "golden")):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a gfx950 GPU (HIP kernels)")
