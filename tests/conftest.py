import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, ROOT)

import __graft_entry__ as ge  # noqa: E402


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU; runs through the C ABI")


@pytest.fixture(scope="session")
def fa():
    return ge.load_package()


@pytest.fixture(scope="session")
def orc():
    o = ge.load_oracle()
    o.set_threads(min(16, os.cpu_count() or 1))
    return o


@pytest.fixture(scope="session")
def ctx(fa):
    c = fa.createContext("hip")
    yield c
    c.destroy()
