"""Shared pytest setup: repo paths and the ``gpu`` marker.

``-m "not gpu"`` runs the oracle, host-logic and ABI-export tests on any host;
``-m gpu`` runs the parity tests, which call the HIP library through its C ABI
and need an MI355X (gfx950) device.
"""
import os
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
PACKAGE_ROOT = ROOT / "strix-trellis_amd"
for entry in (str(ROOT), str(PACKAGE_ROOT)):
    if entry not in sys.path:
        sys.path.insert(0, entry)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU and the built HIP library")
    config.addinivalue_line("markers", "slow: long-running CPU check")


@pytest.fixture(scope="session")
def repo_root():
    return ROOT
