"""Test configuration: the ``gpu`` marker, the repository on ``sys.path`` and the package fixture."""

from __future__ import annotations

import importlib
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU and the built HIP library")


@pytest.fixture(scope="session")
def gdn():
    """The ``zonos3-mini_amd`` package (its directory name is not an identifier, so import it by name)."""
    return importlib.import_module("zonos3-mini_amd")


@pytest.fixture(scope="session")
def cuda():
    import torch

    if not torch.cuda.is_available():
        raise RuntimeError("GPU tests need a visible GPU (select them with -m gpu only on a GPU host)")
    return torch.device("cuda:0")
