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
    # the tests check the in-tree library and nothing else
    if os.environ.get("TER_HIP_LIB"):
        raise pytest.UsageError("TER_HIP_LIB is set: the tests only load ter_amd/libter_hip.so")
    from ter_amd import _lib
    want = os.path.join(ROOT, "ter_amd", "libter_hip.so")
    if os.path.realpath(_lib.LIB_PATH) != os.path.realpath(want):
        raise pytest.UsageError(f"ter_amd._lib loads {_lib.LIB_PATH}, not the in-tree {want}")


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
