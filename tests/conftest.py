"""Test configuration: CPU tests run anywhere; `-m gpu` tests need an MI355X
and the built libttrl_hip.so (they fail, not skip, when the library is
missing, so a GPU run can never pass on a fallback)."""

from __future__ import annotations

import os
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
for p in (ROOT, ROOT / "tt-rl_amd"):
    if str(p) not in sys.path:
        sys.path.insert(0, str(p))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X GPU and the built libttrl_hip.so")


@pytest.fixture(scope="session")
def device():
    from ttrl_amd.engine.device import device_count, open_device

    if device_count() < 1:
        pytest.fail("no GPU visible: -m gpu tests must run on a GPU box")
    dev = open_device(0)
    yield dev


def pytest_runtest_logstart(nodeid, location):
    # Name each case before it touches the GPU, so a fault report names it.
    if os.environ.get("TTRL_TRACE_TESTS"):
        print(f"\n[start] {nodeid}", flush=True)
