"""Shared test setup: import paths, the `gpu` marker, oracle and C-ABI handles."""

import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PYDIR = os.path.join(ROOT, "fast-polynomial-transcendentals_amd", "python")
for p in (PYDIR, os.path.join(ROOT, "oracle"), os.path.join(ROOT, "tests")):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (HIP device) to run")


@pytest.fixture(scope="session")
def oracle():
    import oracle as orc  # oracle/oracle.py (test infrastructure)

    orc.lib()
    return orc


@pytest.fixture(scope="session")
def cuda():
    import torch

    if not torch.cuda.is_available():
        pytest.fail("GPU test started without a HIP device")
    return torch.device("cuda:0")


@pytest.fixture(scope="session")
def spline_ops(cuda):
    import spline_ops as ext  # the in-tree HIP extension; no fallback exists

    return ext


@pytest.fixture(scope="session")
def capi(cuda):
    import capi_helpers

    return capi_helpers.CApi()
