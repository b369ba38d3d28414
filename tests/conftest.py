"""Shared test configuration: the ``gpu`` marker and the repository root on sys.path."""

import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU and the built HIP library")


@pytest.fixture(scope="session")
def gpu_device():
    import torch

    if not torch.cuda.is_available():
        pytest.fail("GPU test selected but no GPU is visible")
    name = torch.cuda.get_device_properties(0).gcnArchName
    if "gfx950" not in name:
        pytest.fail(f"GPU tests need gfx950, found {name}")
    return torch.device("cuda", 0)
