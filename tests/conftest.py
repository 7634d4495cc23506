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


# With THETASCAN_ERROR_LOG=<path>, every rel_err value is recorded per test
# (the largest one) and written to <path> as JSON at the end of the session:
# the measured floors that the tests' bars are set against.
# (pytest loads this file as its own plugin module while the tests import it as
# tests.conftest: the record lives in one object both copies share)
_SHARED = sys.__dict__.setdefault("_thetascan_test_errors", {"errors": {}, "current": [None]})
_ERRORS: dict = _SHARED["errors"]
_CURRENT: list = _SHARED["current"]


@pytest.fixture(autouse=True)
def _name_the_test(request):
    _CURRENT[0] = request.node.nodeid
    yield
    _CURRENT[0] = None


def pytest_sessionfinish(session, exitstatus):
    path = os.environ.get("THETASCAN_ERROR_LOG")
    if path and _ERRORS:
        import json

        with open(path, "w") as f:
            json.dump(_ERRORS, f, indent=0, sort_keys=True)


def rel_err(actual, expected) -> float:
    """max |actual - expected| / max |expected| (the reference's precision metric,
    tests/test_scan_chunk.py:125-138)."""
    import torch

    a = actual.detach().to("cpu", torch.float64)
    e = expected.detach().to("cpu", torch.float64)
    scale = e.abs().max().clamp_min(1e-30)
    err = float((a - e).abs().max() / scale)
    if _CURRENT[0] is not None:
        _ERRORS[_CURRENT[0]] = max(_ERRORS.get(_CURRENT[0], 0.0), err)
    return err
