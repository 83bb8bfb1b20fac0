"""The CPU tests under AddressSanitizer + UndefinedBehaviorSanitizer.

The operator library is rebuilt with the host passes sanitized (build.build_sanitized: the C ABI's
validation, group-table and launch-selection code; the device code is unchanged) and the oracle with
clang's ASan + UBSan (oracle/Makefile, target sanitize).  A child process that preloads the clang
ASan runtime then runs every other CPU test file against those two builds: every status branch of
the C ABI (tests/test_abi.py, tests/test_ops_host.py) and every oracle function on its pinning
vectors (tests/test_oracle*.py).  A sanitizer report aborts the child, and the test fails.
"""
import glob
import importlib
import os
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _asan_runtime():
    hits = sorted(glob.glob("/opt/rocm/llvm/lib/clang/*/lib/linux/libclang_rt.asan-x86_64.so"))
    return hits[-1] if hits else None


def test_cpu_suite_under_asan_ubsan():
    rt = _asan_runtime()
    if rt is None:
        pytest.skip("clang ASan runtime not found under /opt/rocm/llvm")
    build = importlib.import_module("cannbench-operator-solutions_amd.build")
    san_lib = build.build_sanitized()
    subprocess.run(["make", "-s", "-C", os.path.join(ROOT, "oracle"), "sanitize"], check=True)
    san_oracle = os.path.join(ROOT, "oracle", "_build", "libcb_oracle_san.so")
    files = sorted(f for f in glob.glob(os.path.join(ROOT, "tests", "test_*.py"))
                   if not f.endswith("test_sanitize.py"))
    env = dict(os.environ)
    env["LD_PRELOAD"] = rt
    # leaks: the interpreter and torch keep allocations until exit by design; the rest stays on
    env["ASAN_OPTIONS"] = "detect_leaks=0:abort_on_error=1:alloc_dealloc_mismatch=0:detect_odr_violation=0"
    env["UBSAN_OPTIONS"] = "halt_on_error=1:print_stacktrace=1"
    r = subprocess.run([sys.executable, os.path.join(ROOT, "tests", "sanitize", "run_cpu_tests.py"), san_lib,
                        san_oracle, *files], cwd=ROOT, env=env, capture_output=True, text=True, timeout=1200)
    out = r.stdout + r.stderr
    assert "ERROR: AddressSanitizer" not in out and "runtime error:" not in out, out[-6000:]
    assert r.returncode == 0, out[-6000:]
