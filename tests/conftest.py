"""pytest configuration: `gpu` marker, repo root on sys.path, shared helpers."""
from __future__ import annotations

import os
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

import pytest  # noqa: E402


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (HIP device) and the built library")


@pytest.fixture(scope="session")
def gpu_device():
    import torch

    if not torch.cuda.is_available():
        pytest.skip("no HIP device")
    import ops3d_amd

    if ops3d_amd._C is None:
        pytest.fail("libops3d_fda.so is not built: run __graft_entry__.build() first")
    return torch.device("cuda:0")
