"""Shared pytest setup: import paths and the `gpu` marker.

Tests marked `gpu` need a real MI355X and call the product through its C ABI (librehip.so);
everything else runs on the CPU and checks the oracle, the host logic and that the C-ABI
library loads and exports its symbols.
"""
import os
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(ROOT, "rusty-engine_amd")
for p in (ROOT, PKG):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU and the built librehip.so")
