"""Test configuration: import paths and the `gpu` marker.

Tests marked `gpu` need a real MI355X.  Without a GPU they are skipped, unless
the run explicitly selected them (`-m gpu`): then a missing device is an
error, so a broken GPU box cannot pass the GPU suite vacuously.
"""
import os
import sys

import pytest

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG_ROOT = os.path.join(REPO, "tilelang-fa-v100_amd")
for p in (REPO, PKG_ROOT):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an AMD Instinct GPU (MI355X)")


def _gpu_requested(config) -> bool:
    expr = (config.getoption("-m") or "").replace(" ", "")
    return "gpu" in expr and "notgpu" not in expr


def pytest_runtest_setup(item):
    if item.get_closest_marker("gpu") is None:
        return
    import torch

    if torch.cuda.is_available():
        return
    if _gpu_requested(item.config):
        pytest.fail("GPU tests were selected but no GPU is visible")
    pytest.skip("no GPU visible")
