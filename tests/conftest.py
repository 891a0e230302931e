"""Test configuration: the `gpu` marker, import paths, and GPU/oracle fixtures.

CPU tests (`-m "not gpu"`) cover the oracle against its pins, the host-side plugin surface
and the C ABI's host checks.  GPU tests (`-m gpu`) call the HIP library through its C ABI
and compare with the oracle; they skip when no GPU is visible, and fail (never fall back)
when the library is missing on a GPU machine.
"""
import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(ROOT, "orcasaq2-kernel_amd")
for p in (ROOT, PKG):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an AMD GPU (MI355X) and the built HIP library")


def _gpu_available() -> bool:
    try:
        import torch
        return torch.cuda.is_available()
    except Exception:
        return False


def pytest_collection_modifyitems(config, items):
    if _gpu_available():
        return
    skip = pytest.mark.skip(reason="no GPU visible")
    for item in items:
        if "gpu" in item.keywords:
            item.add_marker(skip)


@pytest.fixture(scope="session")
def oracle():
    from oracle import oracle as O
    O.lib()
    return O


@pytest.fixture(scope="session")
def native():
    """The HIP library binding; on a GPU machine a missing library is a failure."""
    from orcasaq2 import _native
    _native.lib()
    return _native
