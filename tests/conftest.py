"""Shared test setup.

Markers: `gpu` tests run the HIP kernels and need an MI355X; everything else runs on CPU.
On a machine without a GPU (/dev/kfd absent) gpu tests are skipped unless they were
selected explicitly with `-m gpu`, in which case they run and fail loudly.
"""
import os
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for p in (ROOT, os.path.join(ROOT, "turing-sm75_amd")):
    if p not in sys.path:
        sys.path.insert(0, p)

GOLDEN = os.path.join(ROOT, "tests", "golden")


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: runs HIP kernels on an MI355X")


def pytest_collection_modifyitems(config, items):
    if os.path.exists("/dev/kfd") or "gpu" in (config.getoption("-m") or ""):
        return
    skip = pytest.mark.skip(reason="no GPU on this machine (/dev/kfd absent)")
    for item in items:
        if "gpu" in item.keywords:
            item.add_marker(skip)


@pytest.fixture(scope="session")
def golden():
    def _load(name):
        with np.load(os.path.join(GOLDEN, name)) as z:  # allow_pickle=False
            return {k: z[k] for k in z.files}
    return _load


@pytest.fixture(scope="session")
def orc():
    import oracle
    oracle.load()
    return oracle


@pytest.fixture(scope="session")
def dev():
    import torch
    assert torch.cuda.is_available(), "gpu test selected but no HIP device is visible"
    import tsa
    tsa.load()
    return torch.device("cuda:0")
