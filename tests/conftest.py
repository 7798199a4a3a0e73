import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(ROOT, "reciprocating-engine_amd")
for p in (ROOT, os.path.join(ROOT, "oracle"), PKG):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs through libreng_hip.so)")


@pytest.fixture(scope="session")
def golden_path():
    return os.path.join(ROOT, "tests", "golden", "fp8_cast.json")
