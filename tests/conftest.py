"""Shared fixtures: the built package (kvb_amd) and the CPU oracle. Builds first only when nothing
is built yet; GPU tests are marked `gpu` and fail (not skip) when the device is missing."""
import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

import __graft_entry__ as graft  # noqa: E402

if not graft.built():
    graft.build()


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a GPU (MI355X); run with -m gpu")


@pytest.fixture(scope="session")
def kvb():
    return graft.load_package()


@pytest.fixture(scope="session")
def oracle():
    return graft.load_oracle()


@pytest.fixture(scope="session")
def gpu(kvb):
    if not kvb.gpu_available():
        pytest.fail("GPU test run without a GPU")
    return kvb


def progress(msg):
    """A progress line that reaches the log even under pytest's capture."""
    print(msg, file=sys.__stderr__, flush=True)
