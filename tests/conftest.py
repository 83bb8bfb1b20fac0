import importlib
import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU")


def load_pkg():
    return importlib.import_module("cannbench-operator-solutions_amd")


@pytest.fixture(scope="session")
def cb():
    return load_pkg()


@pytest.fixture(scope="session")
def orc():
    from oracle import oracle
    oracle.lib()
    return oracle


@pytest.fixture
def overrides():
    """Sets the library's per-thread test overrides (persistent grid, exchange poll limit,
    GroupedMatmul tile) for one test and restores the defaults afterwards."""
    lib = load_pkg()._lib.load()

    def set_(persistent_grid=0, exchange_spin_limit=0, gmm_tile=0):
        lib.cb_set_test_overrides(persistent_grid, exchange_spin_limit, gmm_tile)

    yield set_
    lib.cb_set_test_overrides(0, 0, 0)
