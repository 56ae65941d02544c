"""Shared pytest setup: import paths, the `gpu` marker, common fixtures."""

from __future__ import annotations

import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
PKG_PARENT = ROOT / "router-ia_amd"
for p in (str(ROOT), str(PKG_PARENT)):
    if p not in sys.path:
        sys.path.insert(0, p)

GOLDEN = ROOT / "tests" / "golden"


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a ROCm GPU and the built HIP library")


@pytest.fixture(scope="session")
def gpu():
    import torch

    if not torch.cuda.is_available():
        pytest.skip("no ROCm GPU visible")
    from router_ia import _native

    _native.load()  # with a GPU present, a missing library is an error, not a skip
    return torch.device("cuda:0")


def announce(msg: str) -> None:
    """Print and flush a line naming the case before GPU work starts."""
    print(msg, flush=True)
