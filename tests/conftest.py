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


def pytest_terminal_summary(terminalreporter, exitstatus, config):
    """Max-abs and max-rel error of every attention parity check, worst first per test."""
    try:
        from tests._helpers import ERRORS
    except ImportError:
        return
    if not ERRORS:
        return
    tr = terminalreporter
    tr.section("attention parity errors (max_abs, max_rel where |ref| >= 0.2)")
    worst: dict[str, tuple[str, float, float, int]] = {}
    for test, what, a, r, n in ERRORS:
        w = worst.get(test)
        if w is None or a > w[1]:
            worst[test] = (what, a, max(r, w[2]) if w else r, n + (w[3] if w else 0))
        else:
            worst[test] = (w[0], w[1], max(r, w[2]), w[3] + n)
    for test, (what, a, r, n) in sorted(worst.items()):
        tr.write_line(f"{test:70s} max_abs {a:.2e}  max_rel {r:.2e}  ({n} elements; worst: {what})")
    tr.write_line(f"overall: max_abs {max(e[2] for e in ERRORS):.2e}  max_rel {max(e[3] for e in ERRORS):.2e}  "
                  f"over {len(ERRORS)} checks")
