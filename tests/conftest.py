"""pytest configuration: the `gpu` marker and shared fixtures.

Tests marked `gpu` need an MI355X (they create a device backend); everything else runs on the
CPU: the oracle checks, the C-ABI export check and host-only graph building.
"""
import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X GPU (runs through libmxrt.so on the device)")


@pytest.fixture(scope="session")
def backend():
    """A device backend on GPU 0 (gpu tests only)."""
    import compute_amd as ca

    b = ca.New("mi355x")
    yield b
    b.Finalize()


@pytest.fixture(scope="session")
def host_backend():
    """A host_only backend: graph building and validation, no device work."""
    import compute_amd as ca

    b = ca.New("mi355x:host_only")
    yield b
    b.Finalize()
