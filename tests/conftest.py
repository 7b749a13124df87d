"""Test configuration: import paths, the `gpu` marker, shared fixtures.

CPU tests (`-m "not gpu"`) pin the oracle against the reference's golden
vectors and check the host logic and the C-ABI library's exports.  GPU tests
(`-m gpu`) call the HIP backend through its C ABI and compare with the oracle.
"""
from __future__ import annotations

import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
for sub in ("", "oracle", "minxfmr.cpp_amd", "tests"):
    p = str(ROOT / sub) if sub else str(ROOT)
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU; runs the HIP backend")


@pytest.fixture(scope="session")
def mxh():
    """The HIP backend, initialised on device 0 (fails loudly if unavailable)."""
    import mxhip

    mxhip.init(0)
    return mxhip
