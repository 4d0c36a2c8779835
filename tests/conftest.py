"""Shared pytest configuration.

GPU tests are marked `gpu`; everything else runs on a CPU-only host.  GPU
tests talk to the provider only through its C ABI (neurofabric_amd.plugin).
"""
import os
import sys
from pathlib import Path

import pytest

REPO = Path(__file__).resolve().parents[1]
if str(REPO) not in sys.path:
    sys.path.insert(0, str(REPO))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU")


def _gpu_present() -> bool:
    try:
        import torch  # noqa: F401  (device count only; does not initialise HIP)
        return torch.cuda.device_count() > 0
    except Exception:
        return False


def pytest_collection_modifyitems(config, items):
    if _gpu_present():
        return
    skip = pytest.mark.skip(reason="no GPU visible on this host")
    for it in items:
        if "gpu" in it.keywords:
            it.add_marker(skip)


@pytest.fixture(scope="session")
def provider():
    """An initialised HIP provider (GPU tests only)."""
    from neurofabric_amd.plugin import Provider
    prov = Provider()
    prov.init()
    yield prov
    prov.synchronize()


@pytest.fixture(scope="session")
def oracle_mod():
    from oracle import oracle
    oracle.lib()
    return oracle


def pytest_report_header(config):
    return f"neurofabric_amd repo: {REPO}"
