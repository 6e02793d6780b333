"""Shared pytest configuration: the `gpu` marker and the GPU device fixture."""
import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a gfx950 GPU (runs through the HIP backend's C ABI)")


@pytest.fixture(scope="session")
def dev():
    """The HIP device.  On a GPU box it must be available: a GPU test never
    passes on a CPU fallback."""
    from zlm_amd.device import Device

    d = Device()
    if not d.available():
        pytest.fail(f"HIP backend unavailable: {d.last_error()}")
    yield d
    d.deinit()
