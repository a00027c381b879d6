"""Shared pytest configuration.

GPU tests are marked ``gpu`` and need a HIP device (the driver runs them on
an MI355X with ``-m gpu``); everything else runs on the CPU.
"""
import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a HIP GPU (MI355X); run with -m gpu")


@pytest.fixture(scope="session")
def ctx():
    import godwit_amd as gw
    if gw.device_count() == 0:
        pytest.fail("gpu test selected but no HIP device is visible")
    c = gw.Context(0)
    yield c
    c.close()
