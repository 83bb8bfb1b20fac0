"""ctypes binding of libcannbench_amd.so (the C ABI declared in include/cannbench_amd.h).

The library is built in-tree by build.py.  Loading fails loudly when it is missing: there is no
fallback implementation behind these entry points.
"""
import ctypes
import os

PKG_DIR = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(PKG_DIR, "libcannbench_amd.so")

# Status codes (cb_status in include/cannbench_amd.h).
CB_OK = 0
CB_ERR_NULL_POINTER = 1
CB_ERR_DTYPE = 2
CB_ERR_SHAPE = 3
CB_ERR_K_MISMATCH = 4
CB_ERR_N_ODD = 5
CB_ERR_GROUP_LEN = 6
CB_ERR_GROUP_COUNT = 7
CB_ERR_GROUP_ORDER = 8
CB_ERR_GROUP_TOTAL = 9
CB_ERR_SCALE_LEN = 10
CB_ERR_ROW_TOO_LONG = 11
CB_ERR_WORKSPACE = 12
CB_ERR_EMPTY = 13
CB_ERR_LAUNCH = 14
CB_ERR_NO_DEVICE = 15
CB_ERR_SCRATCH_LIMIT = 16

# dtype codes (cb_dtype)
CB_DT_FLOAT16 = 1
CB_DT_BFLOAT16 = 2
CB_DT_FLOAT32 = 3
CB_DT_INT8 = 4
CB_DT_INT32 = 5
CB_DT_INT64 = 6

CB_MAX_EXPERTS = 256
CB_GMM_MAX_EXPERTS = 64  # GroupedMatmul (GMM_MAX_E)
CB_ARDQ_MAX_ROW = 16384

_P = ctypes.c_void_p
_I64 = ctypes.c_int64
_I = ctypes.c_int
_F = ctypes.c_float

# name -> (restype, argtypes); every symbol include/cannbench_amd.h declares.
SIGNATURES = {
    "cb_status_string": (ctypes.c_char_p, [_I]),
    "cb_version": (ctypes.c_char_p, []),
    "cb_set_kernel_timing": (None, [_P, _P]),
    "cb_probe_mfma_i8": (_I, [_I64, _P, _I64, _P, _P]),
    "cb_add_rms_norm_dynamic_quant": (_I, [_P, _P, _P, _I, _I64, _I64, _F, _P, _P, _P, _P]),
    "cb_dynamic_quant": (_I, [_P, _I, _I64, _I64, _P, _P, _P]),
    "cb_grouped_matmul_swiglu_quant_workspace_size": (_I64, [_I64, _I64, _I64, _I64]),
    "cb_grouped_matmul_swiglu_quant": (_I, [_P, _P, _P, _P, _P, _I64, _I64, _I64, _I64, _I64, _P, _P, _P, _I64, _P]),
    "cb_grouped_matmul_swiglu_quant_status": (_I, [_P, _I64, _I64, _I64, _P, _P]),
    "cb_set_test_overrides": (None, [_I, _I, _I]),
    "cb_grouped_matmul_swiglu_quant_noalloc": (_I, [_P, _P, _P, _P, _P, _I64, _I64, _I64, _I64, _I64, _P, _P, _P]),
    "cb_grouped_matmul_swiglu_quant_gather": (_I, [_P, _I64, _P, _P, _P, _P, _P, _I64, _I64, _I64, _I64, _I64, _P, _P, _P, _I64, _P]),
    "cb_quant_matmul": (_I, [_P, _P, _P, _I, _I64, _P, _I64, _P, _I64, _P, _I, _I64, _I, _I64, _I64, _I64, _I64, _I, _P, _P]),
    "cb_grouped_matmul_quant": (_I, [_P, _P, _P, _P, _P, _I64, _I64, _I64, _I64, _I64, _P, _P]),
    "cb_grouped_matmul_int32": (_I, [_P, _P, _P, _I64, _I64, _I64, _I64, _I64, _P, _P]),
    "cb_grouped_matmul": (_I, [_P, _P, _P, _I, _I, _P, _I64, _I64, _I64, _I64, _I64, _I, _P, _P]),
    "cb_moe_re_routing_workspace_size": (_I64, [_I64, _I64]),
    "cb_moe_re_routing": (_I, [_P, _I, _I64, _I64, _P, _I, _I64, _I64, _P, _P, _P, _P, _P, _P, _I64, _P]),
    "cb_moe_finalize_routing": (_I, [_P, _I, _I64, _I64, _P, _I64, _I64, _P, _P, _P, _I64, _P, _I, _P, _I, _P, _P]),
    "cb_dequant_swiglu_quant": (_I, [_P, _I, _I64, _I64, _P, _P, _P, _I, _P, _P, _P]),
    "cb_moe_gating_top_k_softmax": (_I, [_P, _I, _I64, _I64, _P, _I64, _P, _P, _P, _P]),
}

_lib = None


def load():
    """Load the in-tree library (once).  Raises if it has not been built."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(
                f"cannbench_amd: {LIB_PATH} is missing; build it with "
                "`python __graft_entry__.py` or `python cannbench-operator-solutions_amd/build.py`")
        lib = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = args
        _lib = lib
    return _lib


def status_string(code):
    return load().cb_status_string(int(code)).decode()


def int64_array(values):
    """Host int64 array for group_list (kept alive by the caller)."""
    arr = (ctypes.c_int64 * len(values))(*[int(v) for v in values])
    return arr
