import os
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU and the built HIP library")


def _has_gpu() -> bool:
    try:
        import torch

        return torch.cuda.is_available()
    except Exception:
        return False


def pytest_collection_modifyitems(config, items):
    if _has_gpu():
        return
    skip = pytest.mark.skip(reason="no GPU visible")
    for item in items:
        if "gpu" in item.keywords:
            item.add_marker(skip)


@pytest.fixture(autouse=True)
def _aklr_env(monkeypatch):
    """Every AKLR_* variable unset (the reference's aklr_env fixture, tests/conftest.py:48-54)."""
    for name in list(os.environ):
        if name.startswith("AKLR_"):
            monkeypatch.delenv(name, raising=False)
    yield


@pytest.fixture(scope="session")
def native_lib():
    """The built C-ABI library (built here when missing; loading needs no GPU)."""
    from aklr_amd import _build, _lib

    if not _build.LIB_PATH.exists():
        _build.build()
    return _lib.lib()
