import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an AMD Instinct GPU (runs on the MI355X box)")


@pytest.fixture(scope="session")
def rt():
    from malus_amd import Runtime

    return Runtime()


@pytest.fixture(scope="session")
def L(rt):
    return rt.L
