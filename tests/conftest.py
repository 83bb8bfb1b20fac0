import importlib
import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
# GroupedMatmulSwigluQuant calls in the tests read back the persistent kernel's status word
os.environ.setdefault("CANNBENCH_AMD_CHECK", "1")
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
