"""Test configuration: the `gpu` marker and import paths.

CPU tests (`-m "not gpu"`) check the oracle against the reference's golden
vectors, the layout and host logic, and that the C-ABI library loads and exports
its symbols. GPU tests (`-m gpu`) are the parity tests proper: HIP kernels
through the C ABI against the oracle.
"""
import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs the HIP kernels)")


@pytest.fixture(scope="session")
def exact():
    from oracle.oracle import Exact

    return Exact()
