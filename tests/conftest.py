"""pytest set-up: the package root (tensix-kernels_amd/) and the repository root (oracle/) on sys.path, the `gpu`
marker, and the session device (the reference's conftest.py:13-19 opens one device for the session)."""

import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
for p in (ROOT / "tensix-kernels_amd", ROOT):
    if str(p) not in sys.path:
        sys.path.insert(0, str(p))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a ROCm GPU (MI355X) and the built HIP library")


@pytest.fixture(scope="session")
def device():
    import torch

    from common import device as cdev

    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    d = cdev.open_device(0)
    yield d
    cdev.close_device(d)
