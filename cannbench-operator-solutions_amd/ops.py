"""Host-side mirror of the reference's `cann_bench` operator plugins, on ROCm torch tensors.

Each function keeps the reference schema (argument order, defaults, output dtypes and shapes) and
its TORCH_CHECK validations with the same messages, allocates the outputs (and workspace) with the
torch caching allocator like the reference plugins do, and enqueues the HIP kernels through the C
ABI on torch's current stream.  There is no CPU fallback: inputs must live on a ROCm device and the
library must be built.

Reference plugins mirrored (paths under operators/):
  add_rms_norm_dynamic_quant   addrmsnormdynamicquant/csrc/ops/add_rms_norm_dynamic_quant/op_plugin/add_rms_norm_dynamic_quant_plugin.cpp:32-115
  dynamic_quant                dynamicquant/csrc/ops/dynamic_quant/op_plugin/dynamic_quant_plugin.cpp:30-87
  grouped_matmul_swiglu_quant  groupedmatmulswigluquant/csrc/ops/grouped_matmul_swiglu_quant/op_plugin/gmsq_plugin.cpp:40-145
  quant_matmul                 quantmatmul/csrc/ops/quant_matmul/op_plugin/quant_matmul_plugin.cpp:48-267
  grouped_matmul_quant         (no reference op) group semantics of groupedmatmul/csrc/ops/grouped_matmul/op_plugin/grouped_matmul_plugin.cpp:42-185
"""
import torch

from . import _lib as L


def _check(cond, msg):
    if not cond:
        raise RuntimeError(msg)


def _stream():
    return ctypes_ptr(torch.cuda.current_stream().cuda_stream)


def ctypes_ptr(v):
    return int(v) if v is not None else None


def _ptr(t):
    return t.data_ptr() if t is not None and t.numel() > 0 else None


def _on_device(name, *ts):
    for t in ts:
        if t is not None:
            _check(t.is_cuda, f"{name}: tensors must be on a ROCm device (there is no CPU path)")


def _raise_status(name, code):
    if code != L.CB_OK:
        raise RuntimeError(f"{name}: {L.status_string(code)} (status {code})")


def _dtype_code(dt):
    return {torch.float16: L.CB_DT_FLOAT16, torch.bfloat16: L.CB_DT_BFLOAT16,
            torch.float32: L.CB_DT_FLOAT32, torch.int8: L.CB_DT_INT8,
            torch.int32: L.CB_DT_INT32}.get(dt, -1)


# ------------------------------------------------------------------------------------------------
# AddRmsNormDynamicQuant
# ------------------------------------------------------------------------------------------------
def add_rms_norm_dynamic_quant_meta(x1, x2, gamma, epsilon):
    _check(x1.dim() >= 1, "add_rms_norm_dynamic_quant: x1 must have at least one dimension.")
    _check(x1.shape == x2.shape, "add_rms_norm_dynamic_quant: x1 and x2 must share a shape.")
    _check(gamma.dim() == 1 and gamma.size(0) == x1.size(-1),
           "add_rms_norm_dynamic_quant: gamma must be 1-D with size == x1.size(-1).")
    _check(gamma.dtype == x1.dtype, "add_rms_norm_dynamic_quant: gamma dtype must match x1 dtype.")
    y = torch.empty(x1.shape, dtype=torch.int8, device=x1.device)
    x_out = torch.empty_like(x1)
    scale = torch.empty(x1.shape[:-1], dtype=torch.float32, device=x1.device)
    return y, x_out, scale


def add_rms_norm_dynamic_quant(x1, x2, gamma, epsilon):
    """(y int8, xOut, scaleOut fp32) = AddRmsNormDynamicQuant(x1, x2, gamma, epsilon)."""
    x1 = x1.contiguous()
    x2 = x2.contiguous()
    gamma = gamma.contiguous()
    y, x_out, scale = add_rms_norm_dynamic_quant_meta(x1, x2, gamma, epsilon)
    row_len = x1.size(-1)
    total = x1.numel()
    if total == 0 or row_len <= 0:
        return y, x_out, scale
    rows = total // row_len
    _check(x1.dtype in (torch.float16, torch.bfloat16),
           "add_rms_norm_dynamic_quant: only float16/bfloat16 inputs are supported.")
    _check(row_len <= L.CB_ARDQ_MAX_ROW, "add_rms_norm_dynamic_quant: row length must not exceed 16384.")
    _on_device("add_rms_norm_dynamic_quant", x1, x2, gamma)
    rc = L.load().cb_add_rms_norm_dynamic_quant(
        _ptr(x1), _ptr(x2), _ptr(gamma), _dtype_code(x1.dtype), rows, row_len, float(epsilon),
        _ptr(y), _ptr(x_out), _ptr(scale), _stream())
    _raise_status("add_rms_norm_dynamic_quant", rc)
    return y, x_out, scale


# ------------------------------------------------------------------------------------------------
# DynamicQuant
# ------------------------------------------------------------------------------------------------
def dynamic_quant_meta(x):
    _check(x.dim() >= 2, "dynamic_quant requires a tensor with rank >= 2.")
    _check(x.dtype in (torch.float16, torch.bfloat16),
           "dynamic_quant only supports float16 / bfloat16 inputs.")
    y = torch.empty(x.shape, dtype=torch.int8, device=x.device)
    scale = torch.empty(x.shape[:-1], dtype=torch.float32, device=x.device)
    return y, scale


def dynamic_quant(x):
    """(y int8, scale fp32) = DynamicQuant(x), per-token symmetric."""
    x = x.contiguous()
    y, scale = dynamic_quant_meta(x)
    n = x.size(-1)
    _check(n > 0, "dynamic_quant requires a non-zero last dimension.")
    rows = x.numel() // n
    if rows <= 0:
        return y, scale
    _on_device("dynamic_quant", x)
    rc = L.load().cb_dynamic_quant(_ptr(x), _dtype_code(x.dtype), rows, n, _ptr(y), _ptr(scale), _stream())
    _raise_status("dynamic_quant", rc)
    return y, scale


# ------------------------------------------------------------------------------------------------
# GroupedMatmulSwigluQuant
# ------------------------------------------------------------------------------------------------
def grouped_matmul_swiglu_quant_meta(x, weight, weight_scale, x_scale, group_list):
    _check(x.dim() == 2, "grouped_matmul_swiglu_quant: x must be 2D [M, K]")
    _check(weight.dim() == 3, "grouped_matmul_swiglu_quant: weight must be 3D [E, K, N]")
    M, N = x.size(0), weight.size(2)
    _check(N % 2 == 0, "grouped_matmul_swiglu_quant: N must be even")
    y = torch.empty((M, N // 2), dtype=torch.int8, device=x.device)
    y_scale = torch.empty((M,), dtype=torch.float32, device=x.device)
    return y, y_scale


def _validate_group_list(prefix, group_list, E, M, max_e):
    gl = [int(v) for v in group_list]
    _check(len(gl) == E, f"{prefix}: group_list length must equal the expert count")
    _check(1 <= len(gl) <= max_e, f"{prefix}: unsupported expert count")
    prev = 0
    for v in gl:
        _check(prev <= v <= M, f"{prefix}: group_list must be a cumsum <= M")
        prev = v
    _check(prev == M, f"{prefix}: group_list[-1] must equal M")
    return gl


def grouped_matmul_swiglu_quant(x, weight, weight_scale, x_scale, group_list):
    """(y int8 [M, N/2], y_scale fp32 [M]) = GroupedMatmulSwigluQuant(...).

    group_list: python list / tensor of E int64 cumulative row counts (a host attribute).
    """
    name = "grouped_matmul_swiglu_quant"
    _check(x.dtype == torch.int8, f"{name}: x must be int8")
    _check(weight.dtype == torch.int8, f"{name}: weight must be int8")
    _check(weight_scale.dtype == torch.float32, f"{name}: weight_scale must be float32")
    _check(x_scale.dtype == torch.float32, f"{name}: x_scale must be float32")
    x = x.contiguous()
    weight = weight.contiguous()
    weight_scale = weight_scale.contiguous()
    x_scale = x_scale.contiguous()
    y, y_scale = grouped_matmul_swiglu_quant_meta(x, weight, weight_scale, x_scale, group_list)
    M, K = x.shape
    E, N = weight.size(0), weight.size(2)
    if M == 0 or N == 0 or E == 0:
        return y, y_scale
    _check(weight.size(1) == K, f"{name}: K mismatch between x and weight")
    _check(x_scale.numel() == M, f"{name}: x_scale must have M elements")
    _check(weight_scale.dim() == 2 and weight_scale.size(0) == E and weight_scale.size(1) == N,
           f"{name}: weight_scale must be [E, N]")
    gl = _validate_group_list(name, group_list, E, M, L.CB_MAX_EXPERTS)
    _on_device(name, x, weight, weight_scale, x_scale)
    lib = L.load()
    ws_bytes = lib.cb_grouped_matmul_swiglu_quant_workspace_size(M, K, N, E)
    ws = torch.empty((ws_bytes,), dtype=torch.uint8, device=x.device)
    gla = L.int64_array(gl)
    rc = lib.cb_grouped_matmul_swiglu_quant(
        _ptr(x), _ptr(weight), _ptr(weight_scale), _ptr(x_scale), gla, len(gl), M, K, N, E,
        _ptr(y), _ptr(y_scale), _ptr(ws), ws_bytes, _stream())
    _raise_status(name, rc)
    return y, y_scale


# ------------------------------------------------------------------------------------------------
# QuantMatmul
# ------------------------------------------------------------------------------------------------
def quant_matmul_meta(x1, x2, scale, offset=None, pertoken_scale=None, bias=None, output_dtype=None):
    _check(x1.dim() >= 2 and x2.dim() >= 2, "quant_matmul requires inputs of rank >= 2.")
    _check(x1.size(-1) == x2.size(-2), "quant_matmul requires x1.size(-1) == x2.size(-2).")
    dt = torch.bfloat16 if output_dtype == "bfloat16" else torch.float16
    shape = list(x1.shape[:-1]) + [x2.size(-1)]
    return torch.empty(shape, dtype=dt, device=x1.device)


def quant_matmul(x1, x2, scale, *, offset=None, pertoken_scale=None, bias=None, output_dtype=None):
    """out = QuantMatmul(x1, x2, scale, offset, pertoken_scale, bias, output_dtype)."""
    name = "quant_matmul"
    _check(x1.dtype == torch.int8 and x2.dtype == torch.int8, "quant_matmul requires int8 x1 and x2.")
    _check(x1.is_contiguous() and x2.is_contiguous() and scale.is_contiguous(),
           "quant_matmul requires contiguous x1/x2/scale.")
    _check(scale.dtype in (torch.float32, torch.bfloat16), "quant_matmul requires float32 or bfloat16 scale.")
    _check(x1.dim() >= 2 and x2.dim() >= 2 and x1.dim() == x2.dim(), "quant_matmul expects equal ranks >= 2.")
    _check(x1.size(-1) == x2.size(-2), "quant_matmul requires x1.size(-1) == x2.size(-2).")
    K, M, N = x1.size(-1), x1.size(-2), x2.size(-1)
    _check(K > 0 and M > 0 and N > 0, "quant_matmul requires non-empty shapes.")
    batch = 1
    for d in range(x1.dim() - 2):
        _check(x1.size(d) == x2.size(d), "quant_matmul expects matching leading batch dimensions.")
        batch *= x1.size(d)
    out = quant_matmul_meta(x1, x2, scale, offset, pertoken_scale, bias, output_dtype)
    _check(scale.numel() in (1, N), "quant_matmul expects scale length 1 or n.")
    off_n = 0
    if offset is not None:
        _check(offset.dtype == torch.float32 and offset.is_contiguous(),
               "quant_matmul requires float32 contiguous offset.")
        _check(offset.numel() in (1, N), "quant_matmul expects offset length 1 or n.")
        off_n = offset.numel()
    pt_n = 0
    if pertoken_scale is not None:
        _check(pertoken_scale.dtype == torch.float32 and pertoken_scale.is_contiguous(),
               "quant_matmul requires float32 contiguous pertoken_scale.")
        _check(pertoken_scale.numel() == M, "quant_matmul expects pertoken_scale length m.")
        pt_n = M
    bias_n, bias_dt, bias_batched = 0, 0, 0
    if bias is not None:
        _check(bias.is_contiguous(), "quant_matmul requires contiguous bias.")
        bias_dt = {torch.int32: L.CB_DT_INT32, torch.float16: L.CB_DT_FLOAT16,
                   torch.bfloat16: L.CB_DT_BFLOAT16, torch.float32: L.CB_DT_FLOAT32}.get(bias.dtype)
        _check(bias_dt is not None, f"quant_matmul unsupported bias dtype: {bias.dtype}")
        if bias.dim() == 3 and bias.size(1) == 1 and bias.size(2) == N and batch > 1 and bias.size(0) == batch:
            bias_batched = 1
        else:
            _check(bias.numel() in (1, N), "quant_matmul expects bias length 1 or n.")
        bias_n = bias.numel()
    _on_device(name, x1, x2, scale, offset, pertoken_scale, bias)
    rc = L.load().cb_quant_matmul(
        _ptr(x1), _ptr(x2), _ptr(scale), _dtype_code(scale.dtype), scale.numel(),
        _ptr(offset), off_n, _ptr(pertoken_scale), pt_n, _ptr(bias), bias_dt, bias_n, bias_batched,
        batch, M, K, N, _dtype_code(out.dtype), _ptr(out), _stream())
    _raise_status(name, rc)
    return out


# ------------------------------------------------------------------------------------------------
# int8 grouped down-projection
# ------------------------------------------------------------------------------------------------
def grouped_matmul_quant_meta(x, weight, weight_scale, x_scale, group_list):
    _check(x.dim() == 2, "grouped_matmul: x must be 2D [M, K]")
    _check(weight.dim() == 3, "grouped_matmul: weight must be 3D [E, K, N] or [E, N, K]")
    return torch.empty((x.size(0), weight.size(2)), dtype=torch.bfloat16, device=x.device)


def grouped_matmul_quant(x, weight, weight_scale, x_scale, group_list):
    """out bf16 [M, N] = W8A8 grouped matmul: per expert g, x[rows_g] @ weight[g], dequantised by
    weight_scale[g, n] then x_scale[row] (QuantMatmul's epilogue order).  The reference has no int8
    grouped matmul; group_list follows grouped_matmul's cumsum rules (split_item = 2: one output).
    """
    name = "grouped_matmul"
    _check(x.dtype == torch.int8 and weight.dtype == torch.int8, f"{name}: x and weight must be int8")
    _check(weight_scale.dtype == torch.float32 and x_scale.dtype == torch.float32,
           f"{name}: weight_scale and x_scale must be float32")
    x = x.contiguous()
    weight = weight.contiguous()
    weight_scale = weight_scale.contiguous()
    x_scale = x_scale.contiguous()
    out = grouped_matmul_quant_meta(x, weight, weight_scale, x_scale, group_list)
    M, K = x.shape
    E, N = weight.size(0), weight.size(2)
    _check(E >= 1, f"{name}: weight must contain at least one expert")
    _check(E <= L.CB_MAX_EXPERTS, f"{name}: at most {L.CB_MAX_EXPERTS} experts are supported")
    _check(weight.size(1) == K, f"{name}: K dimension mismatch between x and weight")
    _check(x_scale.numel() == M, f"{name}: x_scale must have M elements")
    _check(weight_scale.dim() == 2 and weight_scale.size(0) == E and weight_scale.size(1) == N,
           f"{name}: weight_scale must be [E, N]")
    gl = [int(v) for v in group_list]
    _check(len(gl) == E, f"{name}: group_list length must equal the number of experts")
    prev = 0
    for v in gl:
        _check(v >= prev, f"{name}: group_list must be a non-decreasing cumsum")
        _check(v <= M, f"{name}: group_list values must not exceed M")
        prev = v
    _check(prev == M, f"{name}: group_list[-1] must equal M")
    if M == 0 or N == 0:
        return out
    _on_device(name, x, weight, weight_scale, x_scale)
    gla = L.int64_array(gl)
    rc = L.load().cb_grouped_matmul_quant(
        _ptr(x), _ptr(weight), _ptr(weight_scale), _ptr(x_scale), gla, len(gl), M, K, N, E,
        _ptr(out), _stream())
    _raise_status(name, rc)
    return out


# ------------------------------------------------------------------------------------------------
# raw grouped int8 GEMM (the reference's launch_gmsq_cube stage)
# ------------------------------------------------------------------------------------------------
def grouped_matmul_int32(x, weight, group_list):
    """c int32 [M, N] = x[rows_g] @ weight[g] per expert, exact int32 accumulation."""
    name = "grouped_matmul_int32"
    _check(x.dtype == torch.int8 and weight.dtype == torch.int8, f"{name}: x and weight must be int8")
    _check(x.dim() == 2 and weight.dim() == 3, f"{name}: x must be [M, K] and weight [E, K, N]")
    x = x.contiguous()
    weight = weight.contiguous()
    M, K = x.shape
    E, N = weight.size(0), weight.size(2)
    _check(weight.size(1) == K, f"{name}: K mismatch between x and weight")
    gl = _validate_group_list(name, group_list, E, M, L.CB_MAX_EXPERTS)
    c = torch.empty((M, N), dtype=torch.int32, device=x.device)
    if M == 0 or N == 0:
        return c
    _on_device(name, x, weight)
    gla = L.int64_array(gl)
    rc = L.load().cb_grouped_matmul_int32(_ptr(x), _ptr(weight), gla, len(gl), M, K, N, E, _ptr(c), _stream())
    _raise_status(name, rc)
    return c
