"""Shared fixtures: the `gpu` marker, the package loader and a HIP context."""
from __future__ import annotations

import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))

import __graft_entry__  # noqa: E402


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU")


@pytest.fixture(scope="session")
def axc():
    """The axiom-compute_amd package (fails if libaxh.so is not built)."""
    return __graft_entry__.load_package()


@pytest.fixture(scope="session")
def ctx(axc):
    c = axc.HipContext.new()
    yield c
    c.close()
