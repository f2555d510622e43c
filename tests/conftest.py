"""Test configuration: import paths and the ``gpu`` marker."""
from __future__ import annotations

import os
import sys
from pathlib import Path

import pytest

REPO = Path(__file__).resolve().parents[1]
PKG_ROOT = REPO / "k8v4-xpu_amd"
for p in (str(PKG_ROOT), str(REPO)):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU and the built HIP library")


@pytest.fixture(scope="session")
def gpu_ops():
    """The ctypes op table on a real GPU; fails (not skips) when the library is missing."""
    import torch

    if not torch.cuda.is_available():
        pytest.fail("GPU test collected on a machine without a GPU")
    from k8v4_v030.ops_api import ops

    return ops()


@pytest.fixture(autouse=True)
def _no_decode_wait_gave_up(request):
    """Every GPU test: no in-kernel wait of the decode kernels (the handshakes
    of the paired halves and of the row split) gave up while it ran; a wait
    that gives up lets its wave go on, so it could hide in a tolerance."""
    if request.node.get_closest_marker("gpu") is None:
        yield
        return
    from k8v4_v030 import ops_api

    lib = ops_api.load_library()
    before = lib.k8v4_decode_fault_count()
    yield
    after = lib.k8v4_decode_fault_count()
    assert after == before, "%d in-kernel decode waits gave up during the test" % (after - before)
