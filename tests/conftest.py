"""Shared pytest configuration: the `gpu` marker, import paths, fixtures."""
from __future__ import annotations

import sys
from pathlib import Path

import pytest

REPO = Path(__file__).resolve().parent.parent
sys.path.insert(0, str(REPO / "tiny-metal-nn_amd"))
sys.path.insert(0, str(REPO / "tests"))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (run with -m gpu)")


@pytest.fixture(scope="session", autouse=True)
def _torch_device_first(request):
    """Sessions with GPU tests: torch's own HIP runtime (bundled with torch)
    sets up its device context before the library's first call, the order
    bench.py and smoke() use; torch's first device call made after a run of
    library-only tests has failed to find the device."""
    if not any(item.get_closest_marker("gpu") for item in request.session.items):
        return
    try:
        import torch
    except ImportError:
        return
    if torch.cuda.is_available():
        torch.zeros(1, device="cuda:0")
        torch.cuda.synchronize()


@pytest.fixture(scope="session")
def oracle():
    from oracle_binding import Oracle
    return Oracle()


@pytest.fixture(scope="session")
def reflib():
    from oracle_binding import REF_SO, RefLib
    if not REF_SO.exists():
        pytest.skip("oracle/_ref not built (reference checkout absent when built)")
    return RefLib()
