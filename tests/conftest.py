"""Test configuration: the `gpu` marker, import paths and shared fixtures.

CPU tests (`-m "not gpu"`) pin the oracle against golden vectors and closed forms, check the host logic, and
check that libsc_handoff.so loads and exports what include/sc_handoff.h declares.  GPU tests (`-m gpu`) are the
parity tests proper: they call the HIP path through the C-ABI and compare it with the oracle.
"""
import os
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
sys.path.insert(0, str(ROOT / "strata-concurrent_amd"))
sys.path.insert(0, str(ROOT))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (run with -m gpu on the GPU box)")


def gpu_available() -> bool:
    import sc_handoff
    return sc_handoff.device_count() > 0


@pytest.fixture(scope="session")
def sc():
    import sc_handoff
    return sc_handoff


@pytest.fixture(scope="session")
def oracle():
    from oracle import sc_oracle
    return sc_oracle


@pytest.fixture(scope="session")
def cuda():
    if not gpu_available():
        pytest.fail("GPU test collected on a machine without a GPU (run -m 'not gpu' here)")
    return 0
