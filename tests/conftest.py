"""Shared pytest configuration: the `gpu` marker and library/oracle set-up."""
from __future__ import annotations

import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a HIP device (MI355X / gfx950)")


def _has_gpu() -> bool:
    try:
        import torch
        return torch.cuda.is_available()
    except Exception:
        return False


def pytest_collection_modifyitems(config, items):
    if _has_gpu():
        return
    skip = pytest.mark.skip(reason="no HIP device")
    for item in items:
        if "gpu" in item.keywords:
            item.add_marker(skip)


@pytest.fixture(scope="session")
def oracle_lib():
    import oracle
    if not oracle.LIB_PATH.exists():
        oracle.build()
    return oracle


@pytest.fixture(scope="session")
def d3d_lib():
    """The built libd3d_hip.so; built here only when it is missing."""
    from d3d_amd import _lib
    if not _lib.LIB_PATH.exists():
        from d3d_amd import build
        build.build()
    return _lib.load()
