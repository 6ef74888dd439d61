import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, ROOT)

import __graft_entry__ as ge  # noqa: E402


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs through the HIP library)")


@pytest.fixture(scope="session")
def eff():
    return ge.package()


@pytest.fixture(scope="session")
def orc():
    return ge.oracle()


@pytest.fixture(scope="session")
def ctx(eff):
    c = eff.Context(0)
    yield c
    c.close()
