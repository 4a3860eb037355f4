from __future__ import annotations

import os
import sys
from pathlib import Path

import pytest
import torch

ROOT = Path(__file__).resolve().parents[1]
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a ROCm GPU (MI355X) and the built HIP library")


def gpu_available() -> bool:
    return torch.cuda.is_available()


@pytest.fixture
def device():
    if not gpu_available():
        pytest.skip("no ROCm GPU in this environment")
    return torch.device("cuda", 0)


@pytest.fixture(autouse=True)
def _seed():
    torch.manual_seed(0)


def pytest_collection_modifyitems(config, items):
    if gpu_available():
        return
    skip = pytest.mark.skip(reason="no ROCm GPU in this environment")
    for item in items:
        if "gpu" in item.keywords:
            item.add_marker(skip)


os.environ.setdefault("PYTHONHASHSEED", "0")
