import os
import sys
from pathlib import Path

import numpy as np
import pytest

ROOT = Path(__file__).resolve().parent.parent
sys.path.insert(0, str(ROOT))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs through libvgemm.so on cuda:0)")


@pytest.fixture(scope="session")
def gpu():
    """The GPU tests run only where a GPU is visible; there the HIP library must load (no fallback)."""
    import torch

    if not torch.cuda.is_available():
        pytest.skip("no GPU visible")
    from vela_amd import _lib

    _lib.load()
    return torch.device("cuda:0")


@pytest.fixture(autouse=True)
def _announce(request):
    # name the case before any GPU work so a fault that ends the process still identifies it
    if request.node.get_closest_marker("gpu"):
        print(f"\n[case] {request.node.nodeid}", flush=True)
    yield


def to_np(t):
    return t.detach().cpu().numpy()


def assert_equal(got, want, what=""):
    got = np.asarray(got)
    want = np.asarray(want)
    assert got.shape == want.shape, f"{what}: shape {got.shape} != {want.shape}"
    if not np.array_equal(got, want):
        bad = np.argwhere(got != want)
        i = tuple(bad[0])
        raise AssertionError(f"{what}: {len(bad)} mismatches; first at {i}: got {got[i]} want {want[i]}")
