"""Shared fixtures. GPU tests are marked ``gpu`` and need a HIP device (MI355X)."""

from __future__ import annotations

import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a HIP device (MI355X); calls the C-ABI library")
    config.addinivalue_line("markers", "slow: long-running")


@pytest.fixture(scope="session")
def device():
    import torch

    if not torch.cuda.is_available():
        pytest.fail("GPU test run without a HIP device")
    from slipstream_amd import _ffi

    _ffi.lib()  # the HIP library must load: no silent fallback
    return torch.device("cuda:0")
