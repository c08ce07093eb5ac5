import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)
HERE = os.path.dirname(os.path.abspath(__file__))
if HERE not in sys.path:
    sys.path.insert(0, HERE)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs through libfa_rocm.so on the device)")
    config.addinivalue_line("markers", "slow: full-size model runs (minutes on CPU)")


@pytest.fixture(scope="session")
def ctx():
    from ai_amd import _native as N
    c = N.Context(0)
    yield c
    c.close()
