import os
import sys

import pytest

sys.path.insert(0, os.path.dirname(os.path.abspath(__file__)))
from _pkg import load_pkg  # noqa: E402


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) and the built libdj.so")


@pytest.fixture(scope="session")
def pkg():
    return load_pkg()


@pytest.fixture(scope="session")
def ctx(pkg):
    from decision_js_amd import _dj
    c = _dj.Context(0)
    print(f"device: {c.info()}", flush=True)
    yield c
    c.close()
