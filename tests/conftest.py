"""Shared test setup.

`gpu` tests call liblgx on a real MI355X and compare against the CPU oracle;
everything else (oracle pinning, host logic, ABI loading) runs without a GPU.
"""
import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) and the built liblgx")


@pytest.fixture(scope="session")
def orc():
    from oracle import oracle

    return oracle


@pytest.fixture(scope="session")
def golden():
    import numpy as np

    return np.load(os.path.join(ROOT, "tests", "golden", "q8_golden.npz"))


@pytest.fixture(scope="session")
def ctx():
    """The product path.  No skip: a GPU test without liblgx or a device fails."""
    import logicaffeine_amd as lgx

    c = lgx.Context(0)
    yield c
    c.close()
