"""Shared pytest configuration: the ``gpu`` marker and repository paths."""
from __future__ import annotations

import os
import sys

import pytest

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if REPO not in sys.path:
    sys.path.insert(0, REPO)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs the HIP kernels)")


def gpu_available() -> bool:
    import torch

    return torch.cuda.is_available()


@pytest.fixture(scope="session")
def cuda():
    import torch

    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    return torch.device("cuda", 0)


def rel_err(actual, expected) -> float:
    """max |actual - expected| / max |expected| (the reference's precision metric,
    tests/test_scan_chunk.py:125-138)."""
    import torch

    a = actual.detach().to("cpu", torch.float64)
    e = expected.detach().to("cpu", torch.float64)
    scale = e.abs().max().clamp_min(1e-30)
    return float((a - e).abs().max() / scale)
