import os
import sys
from pathlib import Path

import pytest

REPO = Path(__file__).resolve().parents[1]
sys.path.insert(0, str(REPO))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU and libmbhip.so")


def _gpu_present() -> bool:
    try:
        import torch
        return torch.cuda.is_available()
    except Exception:
        return False


def pytest_collection_modifyitems(config, items):
    # GPU tests are selected with -m gpu on the GPU box.  Where no GPU exists at
    # all they are skipped; where one exists they run and fail loudly if the
    # native library is missing (there is no CPU fallback).
    if _gpu_present():
        return
    skip = pytest.mark.skip(reason="no GPU in this environment")
    for item in items:
        if "gpu" in item.keywords:
            item.add_marker(skip)


@pytest.fixture(scope="session")
def mb():
    """The native library, initialised on device 0."""
    from metalbench_amd import native
    native.init(0)
    yield native


@pytest.fixture(scope="session")
def dev():
    import torch
    return torch.device("cuda", 0)
