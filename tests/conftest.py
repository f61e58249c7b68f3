"""Test configuration: the ``gpu`` marker and shared fixtures.

``-m "not gpu"`` runs on any host (oracle, host logic, C-ABI loading);
``-m gpu`` tests need an MI355X and compare the HIP path with the CPU oracle.
"""
import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a ROCm GPU (MI355X); compares HIP kernels with the CPU oracle")
    config.addinivalue_line("markers", "slow: long-running")


def _gpu_available() -> bool:
    try:
        import torch
        return torch.cuda.is_available()
    except Exception:
        return False


def pytest_collection_modifyitems(config, items):
    if _gpu_available():
        return
    skip = pytest.mark.skip(reason="no ROCm GPU on this host")
    for item in items:
        if "gpu" in item.keywords:
            item.add_marker(skip)


@pytest.fixture(scope="session")
def dev():
    import torch
    from infurnace_amd import _capi
    _capi.lib()  # fail loudly when the HIP library is missing
    return torch.device("cuda", 0)
