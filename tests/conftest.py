"""pytest configuration: markers and shared fixtures.

``-m "not gpu"`` runs the oracle checks, host logic and C-ABI export checks
on CPU; ``-m gpu`` runs the HIP parity tests on an MI355X.
"""
import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (HIP) device")
    config.addinivalue_line("markers", "slow: long-running CPU test")


@pytest.fixture(scope="session")
def orc():
    import oracle

    oracle.lib()
    return oracle
