import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line(
        "markers", "gpu: needs a real MI355X (run with -m gpu on the GPU box)")


@pytest.fixture(scope="session")
def device():
    from lcd_amd import hip_runtime
    return hip_runtime.default_device()


@pytest.fixture(scope="session")
def oracle():
    from oracle import lcd_oracle
    lcd_oracle.lib()
    return lcd_oracle
