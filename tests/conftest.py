"""Shared pytest configuration.

Tests marked ``gpu`` need an MI355X and call the HIP reactor through its C ABI;
everything else runs on the CPU (oracle pinning, host logic, ABI surface).
"""
import sys
from pathlib import Path

import pytest

REPO = Path(__file__).resolve().parent.parent
if str(REPO) not in sys.path:
    sys.path.insert(0, str(REPO))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X GPU and the built HIP reactor")


@pytest.fixture(scope="session")
def gpu_runtime():
    """A runtime on the real device.  Fails (never skips) when the HIP path is absent."""
    from oct_amd import prometheus as p

    rt = p.NativeRuntime()
    assert rt.caps.available == 1, "HIP device unavailable: GPU tests must run on the MI355X box"
    assert rt.caps.backend_type == p.PROM_BACKEND_HARDWARE_GPU
    yield rt
    rt.close()
