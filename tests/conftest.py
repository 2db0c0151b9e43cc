"""Shared test setup: repo root on sys.path, the `gpu` marker, GPU fixtures."""
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (HIP device); run with -m gpu")


@pytest.fixture(scope="session")
def lib():
    import cubutterfly_amd as cb
    return cb.Native()


@pytest.fixture(scope="session")
def torch_gpu():
    """torch with a visible HIP device; GPU tests fail (not skip) without one."""
    import torch
    assert torch.cuda.is_available(), "GPU tests need a HIP device"
    return torch


@pytest.fixture(scope="session")
def stream(torch_gpu):
    return torch_gpu.cuda.current_stream().cuda_stream
