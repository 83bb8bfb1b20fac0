"""numpy front end of the CPU oracle (oracle/cb_oracle.c).  TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and the cpu_baseline leg of bench.py may use this module, and
only as the checker.  Arrays are numpy; 16-bit floats travel as uint16 bit patterns (dtype code
'bf16' or 'f16').  Every function restates the reference semantics cited in cb_oracle.c.
"""
import ctypes
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB = os.path.join(HERE, "_build", "libcb_oracle.so")

DT = {"f16": 1, "bf16": 2, "f32": 3, "i8": 4, "i32": 5, "i64": 6}

_lib = None


def build():
    subprocess.run(["make", "-s", "-C", HERE], check=True)
    return LIB


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB):
            build()
        L = ctypes.CDLL(LIB)
        P, I64, I, F = ctypes.c_void_p, ctypes.c_int64, ctypes.c_int, ctypes.c_float
        L.or_dynamic_quant.argtypes = [P, I, I64, I64, P, P]
        L.or_ardq.argtypes = [P, P, P, I, I64, I64, F, P, P, P]
        L.or_i8_gemm.argtypes = [P, I64, P, I64, P, I64, I64, I64, I64]
        L.or_gmsq.argtypes = [P, P, P, P, P, I64, I64, I64, I64, I64, I64, P, P]
        L.or_quant_matmul.argtypes = [P, P, P, I, I64, P, I64, P, I64, P, I, I64, I, I64, I64, I64, I64, I, P, I64, I64]
        L.or_grouped_matmul_quant.argtypes = [P, P, P, P, P, I64, I64, I64, I64, I64, I64, P]
        L.or_grouped_matmul.argtypes = [P, P, P, I, I, P, I64, I64, I64, I64, I, P]
        L.or_moe_re_routing.argtypes = [P, I64, I64, P, I64, I64, P, P, P, P, P]
        L.or_moe_re_routing.restype = I64
        L.or_moe_finalize_routing.argtypes = [P, I, I64, I64, P, I64, I64, P, P, P, I64, P, I, P, I, P]
        L.or_dequant_swiglu_quant.argtypes = [P, I, I64, I64, P, P, P, I, P, P]
        L.or_moe_gating_top_k_softmax.argtypes = [P, I, I64, I64, P, I64, P, P, P]
        L.or_rint16.argtypes = [F]
        L.or_rint16.restype = ctypes.c_int8
        L.or_f32_to_f16.argtypes = [F]
        L.or_f32_to_f16.restype = ctypes.c_uint16
        L.or_f32_to_bf16.argtypes = [F]
        L.or_f32_to_bf16.restype = ctypes.c_uint16
        _lib = L
    return _lib


def _p(a):
    return None if a is None else a.ctypes.data_as(ctypes.c_void_p)


def _c(a, dtype):
    return np.ascontiguousarray(a, dtype=dtype)


# ---- scalar conversions (exposed for the pinning tests) ---------------------------------------
def f32_to_f16_bits(v):
    L = lib()
    return np.array([L.or_f32_to_f16(float(x)) for x in np.asarray(v, np.float32).ravel()], np.uint16)


def f32_to_bf16_bits(v):
    L = lib()
    return np.array([L.or_f32_to_bf16(float(x)) for x in np.asarray(v, np.float32).ravel()], np.uint16)


def rint16(v):
    L = lib()
    return np.array([L.or_rint16(float(x)) for x in np.asarray(v, np.float32).ravel()], np.int8)


# ---- operators ---------------------------------------------------------------------------------
def dynamic_quant(x_bits, dtype):
    x = _c(x_bits, np.uint16)
    rows, n = x.reshape(-1, x.shape[-1]).shape
    y = np.empty(x.shape, np.int8)
    s = np.empty(x.shape[:-1], np.float32)
    lib().or_dynamic_quant(_p(x), DT[dtype], rows, n, _p(y), _p(s))
    return y, s


def ardq(x1_bits, x2_bits, gamma_bits, dtype, eps):
    x1 = _c(x1_bits, np.uint16)
    x2 = _c(x2_bits, np.uint16)
    g = _c(gamma_bits, np.uint16)
    n = x1.shape[-1]
    rows = x1.size // n
    y = np.empty(x1.shape, np.int8)
    xo = np.empty(x1.shape, np.uint16)
    s = np.empty(x1.shape[:-1], np.float32)
    lib().or_ardq(_p(x1), _p(x2), _p(g), DT[dtype], rows, n, float(eps), _p(y), _p(xo), _p(s))
    return y, xo, s


def i8_gemm(a, b):
    a = _c(a, np.int8)
    b = _c(b, np.int8)
    m, k = a.shape
    n = b.shape[1]
    c = np.empty((m, n), np.int32)
    lib().or_i8_gemm(_p(a), k, _p(b), n, _p(c), n, m, k, n)
    return c


def gmsq(x, w, ws, xs, group_list, row_begin=0, row_end=None):
    """GroupedMatmulSwigluQuant; only rows [row_begin, row_end) of y / y_scale are computed."""
    x = _c(x, np.int8)
    w = _c(w, np.int8)
    ws = _c(ws, np.float32)
    xs = _c(xs, np.float32)
    gl = _c(group_list, np.int64)
    M, K = x.shape
    E, _, N = w.shape
    row_end = M if row_end is None else row_end
    y = np.zeros((M, N // 2), np.int8)
    ys = np.zeros((M,), np.float32)
    lib().or_gmsq(_p(x), _p(w), _p(ws), _p(xs), _p(gl), E, M, K, N, row_begin, row_end, _p(y), _p(ys))
    return y, ys


def quant_matmul(x1, x2, scale, scale_dtype="f32", offset=None, pertoken=None, bias=None, bias_dtype="f32",
                 bias_batched=False, out_dtype="bf16", row_begin=0, row_end=None):
    """QuantMatmul; x1 [B, M, K] or [M, K], x2 [B, K, N] or [K, N].  16-bit scale / bias as uint16 bits."""
    x1 = _c(x1, np.int8)
    x2 = _c(x2, np.int8)
    batch = int(np.prod(x1.shape[:-2])) if x1.ndim > 2 else 1
    M, K = x1.shape[-2:]
    N = x2.shape[-1]
    sc = _c(scale, np.uint16 if scale_dtype == "bf16" else np.float32)
    off = None if offset is None else _c(offset, np.float32)
    pt = None if pertoken is None else _c(pertoken, np.float32)
    bdt = {"i32": np.int32, "f16": np.uint16, "bf16": np.uint16, "f32": np.float32}[bias_dtype]
    bi = None if bias is None else _c(bias, bdt)
    row_end = M if row_end is None else row_end
    out = np.zeros(x1.shape[:-1] + (N,), np.uint16)
    lib().or_quant_matmul(_p(x1), _p(x2), _p(sc), DT[scale_dtype], sc.size, _p(off), 0 if off is None else off.size,
                          _p(pt), 0 if pt is None else pt.size, _p(bi), DT[bias_dtype], 0 if bi is None else bi.size,
                          int(bias_batched), batch, M, K, N, DT[out_dtype], _p(out), row_begin, row_end)
    return out


def grouped_matmul(x, w, group_list, bias=None, dtype="bf16", bias_dtype=None, trans=False):
    """GroupedMatmul.  x [M, K], w [E, K, N] (or [E, N, K] with trans), bias [E, N]; 16-bit arrays as
    uint16 bits (dtype 'bf16' / 'f16'), fp32 as float32.  Returns y [M, N] in the same form."""
    et = np.float32 if dtype == "f32" else np.uint16
    x = _c(x, et)
    w = _c(w, et)
    M, K = x.shape
    E = w.shape[0]
    N = w.shape[1] if trans else w.shape[2]
    bdt = bias_dtype or dtype
    b = None if bias is None else _c(bias, np.float32 if bdt == "f32" else np.uint16)
    gl = _c(group_list, np.int64)
    y = np.zeros((M, N), et)
    lib().or_grouped_matmul(_p(x), _p(w), _p(b), DT[dtype], DT[bdt], _p(gl), E, M, K, N, 1 if trans else 0, _p(y))
    return y


def grouped_matmul_quant(x, w, ws, xs, group_list, row_begin=0, row_end=None):
    x = _c(x, np.int8)
    w = _c(w, np.int8)
    ws = _c(ws, np.float32)
    xs = _c(xs, np.float32)
    gl = _c(group_list, np.int64)
    M, K = x.shape
    E, _, N = w.shape
    row_end = M if row_end is None else row_end
    out = np.zeros((M, N), np.uint16)
    lib().or_grouped_matmul_quant(_p(x), _p(w), _p(ws), _p(xs), _p(gl), E, M, K, N, row_begin, row_end, _p(out))
    return out


# ---- routing operators -------------------------------------------------------------------------
_NP = {"f16": np.uint16, "bf16": np.uint16, "f32": np.float32, "i32": np.int32, "i8": np.int8}


def moe_re_routing(tokens, counts, scales=None):
    """tokens [A, H] any 1/2-byte dtype (raw bytes are moved); counts [N, E] int.  Returns
    (permute_tokens, permute_scales, permute_idx, expert_token_num, routed_total).  Rows past the
    routed total are zero here (the operator leaves them unwritten)."""
    t = np.ascontiguousarray(tokens)
    A, H = t.shape
    cnt = _c(counts, np.int64)
    n, e = cnt.shape
    sc = None if scales is None else _c(scales, np.float32)
    out = np.zeros_like(t)
    osc = np.zeros((A,), np.float32)
    oidx = np.zeros((A,), np.int32)
    etn = np.zeros((e,), np.int64)
    total = lib().or_moe_re_routing(_p(t), A, H * t.itemsize, _p(cnt), n, e, _p(sc), _p(out), _p(osc), _p(oidx),
                                    _p(etn))
    return out, osc, oidx, etn, int(total)


def moe_finalize_routing(epr, dtype, esdr, K, skip1=None, skip2=None, bias=None, scales=None, scales_dtype=None,
                         expert=None, drop_pad_mode=0):
    """epr [num_dst, H] (uint16 bits for f16/bf16, float32 for f32); esdr int32 [num_rows * K]."""
    epr = _c(epr, _NP[dtype])
    H = epr.shape[-1]
    num_dst = epr.size // H
    esdr = _c(esdr, np.int32)
    num_rows = esdr.size // K
    sk1 = None if skip1 is None else _c(skip1, _NP[dtype])
    sk2 = None if skip2 is None else _c(skip2, _NP[dtype])
    bi = None if bias is None else _c(bias, _NP[dtype])
    sdt = scales_dtype or dtype
    sc = None if scales is None else _c(scales, _NP[sdt])
    ex = None if expert is None else _c(expert, np.int32)
    out = np.zeros((num_rows, H), _NP[dtype])
    lib().or_moe_finalize_routing(_p(epr), DT[dtype], num_dst, H, _p(esdr), num_rows, K, _p(sk1), _p(sk2), _p(bi),
                                  0 if bi is None else bi.shape[0], _p(sc), DT[sdt], _p(ex), int(drop_pad_mode),
                                  _p(out))
    return out


def dequant_swiglu_quant(x, x_dtype, weight_scale=None, activation_scale=None, quant_scale=None,
                         activate_left=False):
    x = _c(x, _NP[x_dtype])
    M, N2 = x.shape
    H = N2 // 2
    ws = None if weight_scale is None else _c(weight_scale, np.float32)
    asc = None if activation_scale is None else _c(activation_scale, np.float32)
    qs = None if quant_scale is None else _c(quant_scale, np.float32)
    y = np.zeros((M, H), np.int8)
    s = np.zeros((M,), np.float32)
    lib().or_dequant_swiglu_quant(_p(x), DT[x_dtype], M, H, _p(ws), _p(asc), _p(qs), int(bool(activate_left)),
                                  _p(y), _p(s))
    return y, s


def moe_gating_top_k_softmax(x, dtype, k, finished=None):
    x = _c(x, _NP[dtype])
    E = x.shape[-1]
    rows = x.size // E
    fin = None if finished is None else _c(finished, np.uint8)
    y = np.zeros((rows, k), _NP[dtype])
    ei = np.zeros((rows, k), np.int32)
    ri = np.zeros((rows, k), np.int32)
    lib().or_moe_gating_top_k_softmax(_p(x), DT[dtype], rows, E, _p(fin), k, _p(y), _p(ei), _p(ri))
    return y, ei, ri


# ---- 16-bit helpers ----------------------------------------------------------------------------
def bf16_bits_to_f32(b):
    return (np.asarray(b, np.uint16).astype(np.uint32) << 16).view(np.float32)


def f16_bits_to_f32(b):
    return np.asarray(b, np.uint16).view(np.float16).astype(np.float32)
