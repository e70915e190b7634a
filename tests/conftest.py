"""Test configuration: import paths and the `gpu` marker.

Tests marked `gpu` need an MI355X and call the HIP kernels through the C-ABI library; the rest
run on any CPU (oracle, host logic, ABI layout, library symbol table).
"""
import os
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(ROOT, "flash-attention-rdna2_amd")
for p in (ROOT, PKG, os.path.join(PKG, "compat")):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a GPU (MI355X); runs the HIP kernels")
