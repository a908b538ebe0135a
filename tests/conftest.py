import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, ROOT)
sys.path.insert(0, os.path.dirname(os.path.abspath(__file__)))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) and libbybyhip.so")


@pytest.fixture(scope="session")
def hip():
    """The HIP device through libbybyhip.so; GPU tests fail (not skip) when it is unavailable."""
    from bybylang_amd import device
    device.init(0)
    return device


@pytest.fixture(scope="session")
def oracle():
    from oracle_lib import Oracle
    return Oracle()
