"""Test configuration: import paths and the `gpu` marker.

`-m "not gpu"` tests run on any host (oracle vs golden vectors, host logic, C
ABI symbols).  `-m gpu` tests need a ROCm GPU and call the HIP library.
"""
import os
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
for p in (ROOT, ROOT / "ravel-lm_amd"):
    if str(p) not in sys.path:
        sys.path.insert(0, str(p))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a ROCm GPU (MI355X) and the built HIP library")


@pytest.fixture(autouse=True)
def _check_status_words(request):
    """GPU tests read back the status word of every sorting call (see
    ravel_em._native.after_call): a bounded device wait that gave up fails the
    test with DeviceWaitError instead of passing with wrong outputs."""
    if request.node.get_closest_marker("gpu") is None:
        yield
        return
    from ravel_em import _native as nat

    prev = nat.set_status_check(True)
    try:
        yield
    finally:
        nat.set_status_check(prev)


@pytest.fixture(scope="session")
def device():
    import torch

    assert torch.cuda.is_available(), "gpu tests need a ROCm device"
    return torch.device("cuda", 0)
