"""Shared fixtures: repository import path, the ``gpu`` marker and the package loader."""

from __future__ import annotations

import importlib
import sys
from pathlib import Path

import pytest

REPO = Path(__file__).resolve().parent.parent
if str(REPO) not in sys.path:
    sys.path.insert(0, str(REPO))
GOLDEN = REPO / "tests" / "golden"


def pytest_configure(config: pytest.Config) -> None:
    config.addinivalue_line("markers", "gpu: needs an MI355X GPU (HIP); run with -m gpu on the GPU host")


@pytest.fixture(scope="session")
def ctmr():
    """The product package (directory ``mlx-generate-ctmr_amd``)."""
    return importlib.import_module("mlx-generate-ctmr_amd")


@pytest.fixture(scope="session")
def dev():
    """The GPU; GPU tests fail (never skip) without one."""
    import torch

    assert torch.cuda.is_available(), "GPU tests need a HIP device"
    return torch.device("cuda:0")


@pytest.fixture(scope="session")
def native_loaded(ctmr):
    """Load libctmr_hip.so; fails loudly when it is not built."""
    return ctmr._lib.lib()
