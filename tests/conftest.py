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
