"""Runs the CPU test suite against the host-sanitized builds (ASan + UBSan) of the operator library
and of the oracle.  Started by tests/test_sanitize.py in a child process whose environment preloads
the clang ASan runtime; not meant to be run by hand.

usage: run_cpu_tests.py SAN_LIB SAN_ORACLE TEST_FILE...
"""
import importlib
import os
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, ROOT)

san_lib, san_oracle, files = sys.argv[1], sys.argv[2], sys.argv[3:]
L = importlib.import_module("cannbench-operator-solutions_amd._lib")
L.LIB_PATH = san_lib  # before anything loads the library
from oracle import oracle  # noqa: E402

oracle.LIB = san_oracle

import pytest  # noqa: E402

rc = pytest.main(["-x", "-q", "-m", "not gpu", "-p", "no:cacheprovider", *files])
# the modules must really have used the sanitized builds
loaded = open("/proc/self/maps").read()
assert os.path.basename(san_lib) in loaded and os.path.basename(san_oracle) in loaded, "sanitized builds not loaded"
sys.exit(int(rc))
