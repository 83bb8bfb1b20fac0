"""C ABI checks that need no GPU: the library loads, exports every symbol include/cannbench_amd.h
declares, and each entry point rejects bad arguments with the right status before touching a
device (validation runs before any HIP call)."""
import ctypes
import os
import re

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "cannbench_amd.h")


def declared_symbols():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(cb_[a-z0-9_]+)\s*\(", text)))


@pytest.fixture(scope="module")
def lib(cb):
    from importlib import import_module
    L = import_module("cannbench-operator-solutions_amd._lib")
    return L, L.load()


def test_header_symbols_exported(lib):
    L, so = lib
    syms = declared_symbols()
    assert len(syms) >= 8
    for s in syms:
        assert hasattr(so, s), f"{s} declared in the header but not exported"
        assert s in L.SIGNATURES, f"{s} has no ctypes signature"


def test_version_and_status_strings(lib):
    L, so = lib
    assert b"gfx950" in so.cb_version()
    assert L.status_string(L.CB_ERR_N_ODD) == "N must be even"
    assert L.status_string(L.CB_ERR_GROUP_TOTAL) == "group_list[-1] must equal M"
    assert L.status_string(999) == "unknown status"


def _gl(vals):
    return (ctypes.c_int64 * max(1, len(vals)))(*vals)


FAKE = 0x1000  # a non-NULL pointer value; never dereferenced because validation fails first


@pytest.mark.parametrize("gl,E,M,N,expect", [
    ([4, 8], 2, 8, 7, "CB_ERR_N_ODD"),
    ([4, 8], 3, 8, 8, "CB_ERR_GROUP_LEN"),
    ([4, 3], 2, 8, 8, "CB_ERR_GROUP_ORDER"),
    ([4, 9], 2, 8, 8, "CB_ERR_GROUP_ORDER"),
    ([4, 7], 2, 8, 8, "CB_ERR_GROUP_TOTAL"),
    ([1] * 257, 257, 1, 8, "CB_ERR_GROUP_COUNT"),
    ([4, 8], 2, 0, 8, "CB_OK"),          # M == 0: early return, nothing launched
])
def test_gmsq_validation(lib, gl, E, M, N, expect):
    L, so = lib
    rc = so.cb_grouped_matmul_swiglu_quant(FAKE, FAKE, FAKE, FAKE, _gl(gl), len(gl), M, 64, N, E,
                                           FAKE, FAKE, FAKE, 1 << 40, None)
    assert rc == getattr(L, expect)


def test_gmsq_workspace_checked(lib):
    L, so = lib
    M, K, N, E = 8, 64, 32, 2
    need = so.cb_grouped_matmul_swiglu_quant_workspace_size(M, K, N, E)
    assert need >= M * (N // 2) * 4 + M * 4
    rc = so.cb_grouped_matmul_swiglu_quant(FAKE, FAKE, FAKE, FAKE, _gl([4, 8]), 2, M, K, N, E,
                                           FAKE, FAKE, FAKE, need - 1, None)
    assert rc == L.CB_ERR_WORKSPACE
    rc = so.cb_grouped_matmul_swiglu_quant(FAKE, FAKE, FAKE, FAKE, _gl([4, 8]), 2, M, K, N, E,
                                           FAKE, FAKE, None, need, None)
    assert rc == L.CB_ERR_WORKSPACE


def test_gmsq_null_pointer(lib):
    L, so = lib
    rc = so.cb_grouped_matmul_swiglu_quant(None, FAKE, FAKE, FAKE, _gl([8]), 1, 8, 64, 32, 1,
                                           FAKE, FAKE, FAKE, 1 << 30, None)
    assert rc == L.CB_ERR_NULL_POINTER


@pytest.mark.parametrize("kw,expect", [
    (dict(scale_dtype=5), "CB_ERR_DTYPE"),
    (dict(out_dtype=3), "CB_ERR_DTYPE"),
    (dict(K=0), "CB_ERR_EMPTY"),
    (dict(scale_numel=7), "CB_ERR_SCALE_LEN"),
    (dict(offset_numel=3), "CB_ERR_SCALE_LEN"),
    (dict(pertoken_numel=5), "CB_ERR_SCALE_LEN"),
    (dict(bias_numel=3, bias_dtype=3), "CB_ERR_SCALE_LEN"),
    (dict(bias_numel=32, bias_dtype=4), "CB_ERR_DTYPE"),
    (dict(bias_numel=64, bias_dtype=3, bias_batched=1, batch=1), "CB_ERR_SCALE_LEN"),
])
def test_quant_matmul_validation(lib, kw, expect):
    L, so = lib
    a = dict(scale_dtype=3, scale_numel=32, offset_numel=0, pertoken_numel=0, bias_numel=0, bias_dtype=3,
             bias_batched=0, batch=1, M=16, K=64, N=32, out_dtype=2)
    a.update(kw)
    rc = so.cb_quant_matmul(FAKE, FAKE, FAKE, a["scale_dtype"], a["scale_numel"], FAKE, a["offset_numel"],
                            FAKE, a["pertoken_numel"], FAKE, a["bias_dtype"], a["bias_numel"], a["bias_batched"],
                            a["batch"], a["M"], a["K"], a["N"], a["out_dtype"], FAKE, None)
    assert rc == getattr(L, expect)


def test_grouped_matmul_quant_validation(lib):
    L, so = lib
    assert so.cb_grouped_matmul_quant(FAKE, FAKE, FAKE, FAKE, _gl([3, 2]), 2, 3, 64, 32, 2, FAKE, None) \
        == L.CB_ERR_GROUP_ORDER
    assert so.cb_grouped_matmul_quant(FAKE, FAKE, FAKE, FAKE, _gl([3]), 1, 3, 64, 32, 0, FAKE, None) \
        == L.CB_ERR_GROUP_COUNT


def test_norm_quant_validation(lib):
    L, so = lib
    assert so.cb_add_rms_norm_dynamic_quant(FAKE, FAKE, FAKE, 3, 4, 64, 1e-6, FAKE, FAKE, FAKE, None) == L.CB_ERR_DTYPE
    assert so.cb_add_rms_norm_dynamic_quant(FAKE, FAKE, FAKE, 2, 4, 16385, 1e-6, FAKE, FAKE, FAKE, None) \
        == L.CB_ERR_ROW_TOO_LONG
    assert so.cb_add_rms_norm_dynamic_quant(FAKE, FAKE, FAKE, 2, 0, 64, 1e-6, FAKE, FAKE, FAKE, None) == L.CB_OK
    assert so.cb_dynamic_quant(FAKE, 4, 4, 64, FAKE, FAKE, None) == L.CB_ERR_DTYPE
    assert so.cb_dynamic_quant(FAKE, 1, 4, 0, FAKE, FAKE, None) == L.CB_ERR_EMPTY


def test_routing_validation(lib):
    L, so = lib
    # MoeReRouting: zero dimensions return before any dtype check (reference plugin order)
    assert so.cb_moe_re_routing(FAKE, 9, 0, 16, FAKE, 9, 2, 2, None, FAKE, FAKE, FAKE, FAKE, None, 0, None) == L.CB_OK
    assert so.cb_moe_re_routing(FAKE, 3, 4, 16, FAKE, 5, 2, 2, None, FAKE, FAKE, FAKE, FAKE, FAKE, 1 << 20, None) \
        == L.CB_ERR_DTYPE
    assert so.cb_moe_re_routing(FAKE, 2, 4, 16, FAKE, 4, 2, 2, None, FAKE, FAKE, FAKE, FAKE, FAKE, 1 << 20, None) \
        == L.CB_ERR_DTYPE
    assert so.cb_moe_re_routing(FAKE, 2, 4, 16, FAKE, 6, 2, 2, None, FAKE, FAKE, FAKE, FAKE, FAKE, 8, None) \
        == L.CB_ERR_WORKSPACE
    assert so.cb_moe_re_routing_workspace_size(2, 2) >= 2 * 2 * 4 * 2 + 3 * 4
    assert so.cb_moe_re_routing_workspace_size(0, 2) == 0
    # MoeFinalizeRouting
    assert so.cb_moe_finalize_routing(FAKE, 4, 4, 8, FAKE, 2, 1, None, None, None, 0, None, 0, None, 0, FAKE, None) \
        == L.CB_ERR_DTYPE
    assert so.cb_moe_finalize_routing(FAKE, 2, 4, 8, FAKE, 2, 0, None, None, None, 0, None, 0, None, 0, FAKE, None) \
        == L.CB_ERR_SHAPE
    assert so.cb_moe_finalize_routing(FAKE, 2, 4, 8, FAKE, 0, 1, None, None, None, 0, None, 0, None, 0, FAKE, None) \
        == L.CB_OK
    # DequantSwigluQuant
    assert so.cb_dequant_swiglu_quant(FAKE, 2, 4, 7, None, None, None, 0, FAKE, FAKE, None) == L.CB_ERR_N_ODD
    assert so.cb_dequant_swiglu_quant(FAKE, 5, 4, 8, None, FAKE, None, 0, FAKE, FAKE, None) == L.CB_ERR_NULL_POINTER
    assert so.cb_dequant_swiglu_quant(FAKE, 2, 4, 8, FAKE, None, None, 0, FAKE, FAKE, None) == L.CB_ERR_SCALE_LEN
    assert so.cb_dequant_swiglu_quant(FAKE, 3, 4, 8, None, None, None, 0, FAKE, FAKE, None) == L.CB_ERR_DTYPE
    # MoeGatingTopKSoftmax
    assert so.cb_moe_gating_top_k_softmax(FAKE, 4, 4, 8, None, 2, FAKE, FAKE, FAKE, None) == L.CB_ERR_DTYPE
    assert so.cb_moe_gating_top_k_softmax(FAKE, 3, 4, 8, None, 9, FAKE, FAKE, FAKE, None) == L.CB_ERR_SHAPE
    assert so.cb_moe_gating_top_k_softmax(FAKE, 3, 4, 4096, None, 2, FAKE, FAKE, FAKE, None) == L.CB_ERR_SHAPE
    assert so.cb_moe_gating_top_k_softmax(FAKE, 3, 0, 8, None, 2, FAKE, FAKE, FAKE, None) == L.CB_ERR_EMPTY


def test_grouped_matmul_validation(lib):
    L, so = lib
    gl = lambda v: L.int64_array(v)
    # E outside [1, 64], dtype, group_list checks, then empty shapes return before any device use
    assert so.cb_grouped_matmul(FAKE, FAKE, None, 3, 0, gl([]), 0, 4, 8, 8, 0, 0, FAKE, None) == L.CB_ERR_GROUP_COUNT
    assert so.cb_grouped_matmul(FAKE, FAKE, None, 3, 0, gl([4] * 65), 65, 4, 8, 8, 65, 0, FAKE, None) \
        == L.CB_ERR_GROUP_COUNT
    assert so.cb_grouped_matmul(FAKE, FAKE, None, 4, 0, gl([4]), 1, 4, 8, 8, 1, 0, FAKE, None) == L.CB_ERR_DTYPE
    assert so.cb_grouped_matmul(FAKE, FAKE, FAKE, 2, 5, gl([4]), 1, 4, 8, 8, 1, 0, FAKE, None) == L.CB_ERR_DTYPE
    assert so.cb_grouped_matmul(FAKE, FAKE, None, 2, 0, gl([4]), 1, 4, 8, 8, 2, 0, FAKE, None) == L.CB_ERR_GROUP_LEN
    assert so.cb_grouped_matmul(FAKE, FAKE, None, 2, 0, gl([3, 2]), 2, 4, 8, 8, 2, 0, FAKE, None) \
        == L.CB_ERR_GROUP_ORDER
    assert so.cb_grouped_matmul(FAKE, FAKE, None, 2, 0, gl([1, 3]), 2, 4, 8, 8, 2, 0, FAKE, None) \
        == L.CB_ERR_GROUP_TOTAL
    assert so.cb_grouped_matmul(None, None, None, 1, 0, gl([0]), 1, 0, 8, 8, 1, 0, None, None) == L.CB_OK
    assert so.cb_grouped_matmul(FAKE, FAKE, None, 1, 0, gl([4]), 1, 4, 8, 8, 1, 0, None, None) == L.CB_ERR_NULL_POINTER


def test_launch_grid_limits(lib):
    """Row counts whose one-block-per-row launch would exceed the dispatch's 32-bit work-item count
    are rejected before any device call; the same operators accept them below the limit (checked on
    the GPU by the parity suites)."""
    L, so = lib
    big = (1 << 31) - 1
    assert so.cb_dynamic_quant(FAKE, 1, 1 << 23, 64, FAKE, FAKE, None) == L.CB_ERR_SHAPE
    assert so.cb_add_rms_norm_dynamic_quant(FAKE, FAKE, FAKE, 2, big, 64, 1e-6, FAKE, FAKE, FAKE, None) \
        == L.CB_ERR_SHAPE
    # H = 6 is off the vector path (whose persistent grid is bounded): one block per row
    assert so.cb_dequant_swiglu_quant(FAKE, 1, big, 12, None, None, None, 0, FAKE, FAKE, None) == L.CB_ERR_SHAPE
    assert so.cb_moe_gating_top_k_softmax(FAKE, 3, big, 8, None, 2, FAKE, FAKE, FAKE, None) == L.CB_ERR_SHAPE


def test_gmsq_status_query_host_paths(lib):
    """The status query rejects NULL arguments and reports 0 for empty shapes, both before any
    device access."""
    L, so = lib
    st = ctypes.c_uint32(7)
    assert so.cb_grouped_matmul_swiglu_quant_status(None, 16, 64, 2, ctypes.byref(st), None) == L.CB_ERR_NULL_POINTER
    buf = (ctypes.c_uint8 * 16)()
    assert so.cb_grouped_matmul_swiglu_quant_status(ctypes.addressof(buf), 16, 64, 2, None, None) == L.CB_ERR_NULL_POINTER
    assert so.cb_grouped_matmul_swiglu_quant_status(ctypes.addressof(buf), 0, 64, 2, ctypes.byref(st), None) == L.CB_OK
    assert st.value == 0


def test_abi_from_c(lib, tmp_path):
    """The header compiles as C99 under -Wall -Wextra -pedantic -Werror, and a C program linked
    against the library gets each validation status back (tests/abi_c/abi_from_c.c)."""
    import shutil
    import subprocess
    L, _ = lib
    cc = shutil.which("gcc") or shutil.which("cc")
    if cc is None:
        pytest.skip("no C compiler")
    so = L.LIB_PATH
    if os.path.basename(so) != "libcannbench_amd.so":
        pytest.skip("a sanitized build needs the clang sanitizer runtimes to link; the plain build is checked")
    src = os.path.join(ROOT, "tests", "abi_c", "abi_from_c.c")
    exe = str(tmp_path / "abi_from_c")
    libdir, libfile = os.path.split(os.path.abspath(so))
    cmd = [cc, "-std=c99", "-Wall", "-Wextra", "-pedantic", "-Werror", "-I", os.path.join(ROOT, "include"), src,
           os.path.join(libdir, libfile), "-Wl,-rpath," + libdir, "-o", exe]
    r = subprocess.run(cmd, capture_output=True, text=True)
    assert r.returncode == 0, r.stderr
    r = subprocess.run([exe], capture_output=True, text=True, timeout=120)
    assert r.returncode == 0 and r.stdout.strip().endswith("ok"), r.stdout + r.stderr
