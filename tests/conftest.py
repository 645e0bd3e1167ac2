import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)
TESTS = os.path.dirname(os.path.abspath(__file__))
if TESTS not in sys.path:
    sys.path.insert(0, TESTS)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a gfx950 GPU (runs the HIP library's kernels)")


@pytest.fixture(scope="session")
def orc():
    """The CPU oracle (built on first use)."""
    from oracle import oracle as o
    o.lib()
    return o


@pytest.fixture(scope="session")
def device():
    """One HipComputeDevice for the GPU tests; the native library must load."""
    from aihost_amd.compute import HipComputeDevice
    dev = HipComputeDevice(0)
    yield dev
    dev.dispose()
