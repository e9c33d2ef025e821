"""Shared pytest setup.

Markers:
  gpu -- needs a real MI355X (gfx950) device; run with `-m gpu`.
Everything else runs on the CPU (the C oracle, the golden fixtures and the
host-side checks of the C-ABI, which return before touching a device).
"""
import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

GOLDEN = os.path.join(ROOT, "tests", "golden")


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU")


@pytest.fixture(scope="session")
def golden():
    import numpy as np

    def load(name):
        return np.load(os.path.join(GOLDEN, name), allow_pickle=False)

    return load


@pytest.fixture(scope="session")
def cuda():
    """The HIP device; fails (does not skip) when absent, so a GPU run never
    passes without executing the kernels."""
    import torch
    assert torch.cuda.is_available(), "GPU test run without a visible HIP device"
    from ter_amd import _lib
    _lib.lib()
    return torch.device("cuda:0")
