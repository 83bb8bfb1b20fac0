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
  grouped_matmul               groupedmatmul/csrc/ops/grouped_matmul/op_plugin/grouped_matmul_plugin.cpp:38-185
  grouped_matmul_quant         (no reference op) group semantics of groupedmatmul/csrc/ops/grouped_matmul/op_plugin/grouped_matmul_plugin.cpp:42-185
  moe_re_routing               moererouting/csrc/ops/moe_re_routing/op_plugin/moe_re_routing_plugin.cpp:33-161
  moe_finalize_routing         moefinalizerouting/csrc/ops/moe_finalize_routing/op_plugin/moe_finalize_routing_plugin.cpp:31-230
  dequant_swiglu_quant         dequantswigluquant/csrc/ops/dequant_swiglu_quant/op_plugin/dqsq_plugin.cpp:32-151
  moe_gating_top_k_softmax     moegatingtopksoftmax/csrc/ops/moe_gating_top_k_softmax/op_plugin/moe_gating_plugin.cpp:28-118
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
            torch.int32: L.CB_DT_INT32, torch.int64: L.CB_DT_INT64}.get(dt, -1)


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


def _gmsq(name, x, row_index, weight, weight_scale, x_scale, group_list):
    _check(x.dtype == torch.int8, f"{name}: x must be int8")
    _check(weight.dtype == torch.int8, f"{name}: weight must be int8")
    _check(weight_scale.dtype == torch.float32, f"{name}: weight_scale must be float32")
    _check(x_scale.dtype == torch.float32, f"{name}: x_scale must be float32")
    if row_index is not None:
        _check(row_index.dtype == torch.int32 and row_index.dim() == 1, f"{name}: row_index must be 1D int32")
        row_index = row_index.contiguous()
    x = x.contiguous()
    weight = weight.contiguous()
    weight_scale = weight_scale.contiguous()
    x_scale = x_scale.contiguous()
    _check(x.dim() == 2, f"{name}: x must be 2D [M, K]")
    _check(weight.dim() == 3, f"{name}: weight must be 3D [E, K, N]")
    M = x.size(0) if row_index is None else row_index.numel()
    _check(weight.size(2) % 2 == 0, f"{name}: N must be even")
    y = torch.empty((M, weight.size(2) // 2), dtype=torch.int8, device=x.device)
    y_scale = torch.empty((M,), dtype=torch.float32, device=x.device)
    K = x.size(1)
    E, N = weight.size(0), weight.size(2)
    if M == 0 or N == 0 or E == 0:
        return y, y_scale
    _check(weight.size(1) == K, f"{name}: K mismatch between x and weight")
    _check(x_scale.numel() == x.size(0), f"{name}: x_scale must have M elements" if row_index is None
           else f"{name}: x_scale must have one element per row of x")
    _check(weight_scale.dim() == 2 and weight_scale.size(0) == E and weight_scale.size(1) == N,
           f"{name}: weight_scale must be [E, N]")
    gl = _validate_group_list(name, group_list, E, M, L.CB_MAX_EXPERTS)
    _on_device(name, x, weight, weight_scale, x_scale, row_index)
    lib = L.load()
    ws_bytes = lib.cb_grouped_matmul_swiglu_quant_workspace_size(M, K, N, E)
    ws = torch.empty((ws_bytes,), dtype=torch.uint8, device=x.device)
    gla = L.int64_array(gl)
    if row_index is None:
        rc = lib.cb_grouped_matmul_swiglu_quant(
            _ptr(x), _ptr(weight), _ptr(weight_scale), _ptr(x_scale), gla, len(gl), M, K, N, E,
            _ptr(y), _ptr(y_scale), _ptr(ws), ws_bytes, _stream())
    else:
        rc = lib.cb_grouped_matmul_swiglu_quant_gather(
            _ptr(x), x.size(0), _ptr(row_index), _ptr(weight), _ptr(weight_scale), _ptr(x_scale), gla, len(gl),
            M, K, N, E, _ptr(y), _ptr(y_scale), _ptr(ws), ws_bytes, _stream())
    _raise_status(name, rc)
    return y, y_scale


def grouped_matmul_swiglu_quant(x, weight, weight_scale, x_scale, group_list):
    """(y int8 [M, N/2], y_scale fp32 [M]) = GroupedMatmulSwigluQuant(...).

    group_list: python list / tensor of E int64 cumulative row counts (a host attribute).
    """
    return _gmsq("grouped_matmul_swiglu_quant", x, None, weight, weight_scale, x_scale, group_list)


def grouped_matmul_swiglu_quant_gather(x, row_index, weight, weight_scale, x_scale, group_list):
    """GroupedMatmulSwigluQuant on gathered rows, without writing them: equal to
    grouped_matmul_swiglu_quant(x[row_index], weight, weight_scale, x_scale[row_index], group_list).

    x int8 [T, K] (e.g. one row per token), x_scale fp32 [T], row_index int32 [M] (the source row of
    each routed row, e.g. MoeReRouting's permutation); outputs have M rows.  An index outside
    [0, T) reads a zero row with scale 0.  No single reference op: it folds moe_re_routing's token
    permutation (moe_re_routing_plugin.cpp:35-38) into the GEMM's activation loads.
    """
    return _gmsq("grouped_matmul_swiglu_quant_gather", x, row_index, weight, weight_scale, x_scale, group_list)


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
# GroupedMatmul (float)
# ------------------------------------------------------------------------------------------------
_GMM_DTYPES = (torch.float16, torch.bfloat16, torch.float32)


def _gmm_ends(group_list, E, M):
    ends = [int(v) for v in group_list]
    prev = 0
    for v in ends:
        _check(v >= prev, "grouped_matmul: group_list must be a non-decreasing cumsum")
        _check(v <= M, "grouped_matmul: group_list values must not exceed M")
        prev = v
    _check(prev == M, "grouped_matmul: group_list[-1] must equal M")
    return ends


def _gmm_outputs(y, ends, split_item):
    """split_item 0/1: one view per expert along M; 2/3: the joined [M, N] tensor
    (grouped_matmul_plugin.cpp:61-77)."""
    if split_item in (0, 1):
        out, s = [], 0
        for e in ends:
            out.append(y.narrow(0, s, e - s))
            s = e
        return out
    return [y]


def grouped_matmul_meta(x, weight, group_list, bias=None, split_item=0, transpose_weight=False):
    _check(x.dim() == 2, "grouped_matmul: x must be 2D [M, K]")
    _check(weight.dim() == 3, "grouped_matmul: weight must be 3D [E, K, N] or [E, N, K]")
    M, E = x.size(0), weight.size(0)
    N = weight.size(1) if transpose_weight else weight.size(2)
    _check(len(group_list) == E, "grouped_matmul: group_list length must equal the number of experts")
    ends = _gmm_ends(group_list, E, M)
    y = torch.empty((M, N), dtype=x.dtype, device=x.device)
    return _gmm_outputs(y, ends, split_item)


def grouped_matmul(x, weight, group_list, bias=None, split_item=0, transpose_weight=False):
    """y[rows_g] = x[rows_g] @ weight[g] (+ bias[g]) per expert g, in the dtype of x (fp16, bf16 or
    fp32); weight [E, K, N], or [E, N, K] with transpose_weight.  Returns a list: one view per expert
    (split_item 0 / 1) or the joined [M, N] tensor (2 / 3)."""
    name = "grouped_matmul"
    _check(x.dim() == 2, f"{name}: x must be 2D [M, K]")
    _check(weight.dim() == 3, f"{name}: weight must be 3D [E, K, N] or [E, N, K]")
    x = x.contiguous()
    weight = weight.contiguous()
    M, K = x.shape
    E = weight.size(0)
    _check(E >= 1, f"{name}: weight must contain at least one expert")
    _check(E <= L.CB_GMM_MAX_EXPERTS, f"{name}: at most {L.CB_GMM_MAX_EXPERTS} experts are supported")
    _check(len(group_list) == E, f"{name}: group_list length must equal the number of experts")
    N = weight.size(1) if transpose_weight else weight.size(2)
    k_stored = weight.size(2) if transpose_weight else weight.size(1)
    _check(k_stored == K, f"{name}: K dimension mismatch between x and weight")
    ends = _gmm_ends(group_list, E, M)
    if bias is not None:
        bias = bias.contiguous()
        _check(bias.numel() == E * N, f"{name}: bias must have shape [E, N]")
    _check(x.dtype in _GMM_DTYPES and weight.dtype == x.dtype, f"{name}: unsupported dtype")
    _check(bias is None or bias.dtype in _GMM_DTYPES, f"{name}: unsupported dtype")
    y = torch.empty((M, N), dtype=x.dtype, device=x.device)
    out = _gmm_outputs(y, ends, split_item)
    if M == 0 or N == 0:
        return out
    _on_device(name, x, weight, bias)
    gla = L.int64_array(ends)
    rc = L.load().cb_grouped_matmul(
        _ptr(x), _ptr(weight), _ptr(bias), _dtype_code(x.dtype), _dtype_code(bias.dtype) if bias is not None else 0,
        gla, len(ends), M, K, N, E, 1 if transpose_weight else 0, _ptr(y), _stream())
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


# ------------------------------------------------------------------------------------------------
# MoeReRouting
# ------------------------------------------------------------------------------------------------
def moe_re_routing_meta(tokens, expert_token_num_per_rank, per_token_scales=None, expert_token_num_type=1,
                        idx_type=0):
    _check(tokens.dim() == 2, "moe_re_routing: tokens must be 2D (A, H).")
    _check(expert_token_num_per_rank.dim() == 2, "moe_re_routing: expert_token_num_per_rank must be 2D (N, E).")
    a, h = tokens.shape
    e = expert_token_num_per_rank.size(1)
    dev = tokens.device
    return (torch.empty((a, h), dtype=tokens.dtype, device=dev),
            torch.empty((a,), dtype=torch.float32, device=dev),
            torch.empty((a,), dtype=torch.int32, device=dev),
            torch.empty((e,), dtype=expert_token_num_per_rank.dtype, device=expert_token_num_per_rank.device))


def moe_re_routing(tokens, expert_token_num_per_rank, per_token_scales=None, expert_token_num_type=1, idx_type=0):
    """(permute_tokens, permute_per_token_scales, permute_token_idx, expert_token_num): rank-major tokens
    re-ordered expert-major.  expert_token_num_type is accepted and ignored, as in the reference."""
    _check(idx_type == 0, "moe_re_routing: only gather index mode (idx_type == 0) is supported.")
    tokens = tokens.contiguous()
    counts = expert_token_num_per_rank.contiguous()
    has_scales = per_token_scales is not None
    if has_scales:
        per_token_scales = per_token_scales.contiguous()
        _check(per_token_scales.dtype == torch.float32, "moe_re_routing: per_token_scales must be float32.")
    outs = moe_re_routing_meta(tokens, counts, per_token_scales, expert_token_num_type, idx_type)
    a, h = tokens.shape
    n, e = counts.shape
    if a <= 0 or h <= 0 or n <= 0 or e <= 0:
        return outs
    _check(tokens.dtype in (torch.float16, torch.bfloat16, torch.int8), "moe_re_routing: unsupported tokens dtype.")
    _check(counts.dtype in (torch.int32, torch.int64),
           "moe_re_routing: unsupported expert_token_num_per_rank dtype.")
    if has_scales:
        _check(per_token_scales.numel() == a, "moe_re_routing: per_token_scales must have A elements.")
    _on_device("moe_re_routing", tokens, counts, per_token_scales)
    pt, ps, pi, etn = outs
    lib = L.load()
    wsb = lib.cb_moe_re_routing_workspace_size(n, e)
    ws = torch.empty((max(wsb, 1),), dtype=torch.uint8, device=tokens.device)
    rc = lib.cb_moe_re_routing(_ptr(tokens), _dtype_code(tokens.dtype), a, h, _ptr(counts), _dtype_code(counts.dtype),
                               n, e, _ptr(per_token_scales), _ptr(pt), _ptr(ps), _ptr(pi), _ptr(etn), _ptr(ws), wsb,
                               _stream())
    _raise_status("moe_re_routing", rc)
    return outs


# ------------------------------------------------------------------------------------------------
# MoeFinalizeRouting
# ------------------------------------------------------------------------------------------------
def _mfr_resolve(epr, esdr, scales):
    _check(epr.dim() >= 2, "moe_finalize_routing: expanded_permuted_rows must have rank >= 2.")
    _check(esdr.dtype == torch.int32, "moe_finalize_routing: expanded_src_to_dst_row must be int32.")
    H = epr.size(-1)
    nk = esdr.numel()
    K = 1
    if scales is not None:
        _check(scales.dim() == 2, "moe_finalize_routing: scales must be 2-D (NUM_ROWS, K).")
        K = scales.size(1)
    _check(K > 0, "moe_finalize_routing: K must be positive.")
    _check(nk % K == 0, "moe_finalize_routing: expanded_src_to_dst_row length must be K*NUM_ROWS.")
    return nk // K, K, H


def moe_finalize_routing_meta(expanded_permuted_rows, expanded_src_to_dst_row, skip1=None, skip2=None, bias=None,
                              scales=None, expert_for_source_row=None, drop_pad_mode=0):
    num_rows, _, H = _mfr_resolve(expanded_permuted_rows, expanded_src_to_dst_row, scales)
    return torch.empty((num_rows, H), dtype=expanded_permuted_rows.dtype, device=expanded_permuted_rows.device)


_FLOATS = (torch.float16, torch.float32, torch.bfloat16)


def moe_finalize_routing(expanded_permuted_rows, expanded_src_to_dst_row, skip1=None, skip2=None, bias=None,
                         scales=None, expert_for_source_row=None, drop_pad_mode=0):
    """out [NUM_ROWS, H] = skip1 + skip2 + sum_k scales[:, k] * (epr[p(i, k)] + bias[expert[i, k]])."""
    name = "moe_finalize_routing"
    _check(expanded_permuted_rows.dtype in _FLOATS,
           f"{name}: expanded_permuted_rows must be float16 / float32 / bfloat16.")
    epr = expanded_permuted_rows.contiguous()
    esdr = expanded_src_to_dst_row.contiguous()
    num_rows, K, H = _mfr_resolve(epr, esdr, scales)
    out = torch.empty((num_rows, H), dtype=epr.dtype, device=epr.device)
    if num_rows <= 0 or H <= 0 or K <= 0:
        return out
    num_dst = epr.numel() // H
    has_bias = bias is not None and expert_for_source_row is not None
    if has_bias:
        _check(bias.size(1) == H, f"{name}: bias head dim must equal H.")
    _check(scales is None or scales.dtype in _FLOATS,
           f"{name}: unsupported dtype combination for expanded_permuted_rows / scales.")
    sk1 = None if skip1 is None else skip1.contiguous()
    sk2 = None if skip2 is None else skip2.contiguous()
    bs = bias.contiguous() if has_bias else None
    sc = None if scales is None else scales.contiguous()
    ex = None if expert_for_source_row is None else expert_for_source_row.contiguous()
    for t, what in ((sk1, "skip1"), (sk2, "skip2"), (bs, "bias")):
        if t is not None:
            _check(t.dtype == epr.dtype, f"{name}: {what} must have the dtype of expanded_permuted_rows.")
    if sk1 is not None:
        _check(sk1.numel() >= num_rows * H, f"{name}: skip1 must hold NUM_ROWS * H elements.")
    if sk2 is not None:
        _check(sk2.numel() >= num_rows * H, f"{name}: skip2 must hold NUM_ROWS * H elements.")
    if ex is not None:
        _check(ex.dtype == torch.int32, f"{name}: expert_for_source_row must be int32.")
        _check(ex.numel() >= num_rows * K, f"{name}: expert_for_source_row must hold NUM_ROWS * K elements.")
    _on_device(name, epr, esdr, sk1, sk2, bs, sc, ex)
    rc = L.load().cb_moe_finalize_routing(
        _ptr(epr), _dtype_code(epr.dtype), num_dst, H, _ptr(esdr), num_rows, K, _ptr(sk1), _ptr(sk2), _ptr(bs),
        bs.size(0) if bs is not None else 0, _ptr(sc), _dtype_code(sc.dtype) if sc is not None else 0, _ptr(ex),
        int(drop_pad_mode), _ptr(out), _stream())
    _raise_status(name, rc)
    return out


# ------------------------------------------------------------------------------------------------
# DequantSwigluQuant
# ------------------------------------------------------------------------------------------------
def dequant_swiglu_quant_meta(x, weight_scale=None, activation_scale=None, quant_scale=None, activate_left=False):
    _check(x.dim() == 2, "dequant_swiglu_quant requires a 2D input [TokensNum, 2H].")
    M, N2 = x.shape
    _check(N2 % 2 == 0, "dequant_swiglu_quant requires an even last dimension.")
    return (torch.empty((M, N2 // 2), dtype=torch.int8, device=x.device),
            torch.empty((M,), dtype=torch.float32, device=x.device))


def dequant_swiglu_quant(x, weight_scale=None, activation_scale=None, quant_scale=None, activate_left=False):
    """(y int8 [M, H], scale fp32 [M]) = per-token quant of SwiGLU(dequant(x))."""
    _check(x.dim() == 2, "dequant_swiglu_quant requires a 2D input [TokensNum, 2H].")
    _check(x.is_contiguous(), "dequant_swiglu_quant requires a contiguous input.")
    y, scale = dequant_swiglu_quant_meta(x, weight_scale, activation_scale, quant_scale, activate_left)
    M, N2 = x.shape
    if M <= 0 or N2 <= 0:
        return y, scale
    H = N2 // 2
    if x.dtype == torch.int32:
        _check(weight_scale is not None, "weight_scale is required when x is int32.")
        _check(activation_scale is not None, "activation_scale is required when x is int32.")
        _check(weight_scale.dtype == torch.float32, "weight_scale must be float32.")
        _check(activation_scale.dtype == torch.float32, "activation_scale must be float32.")
        _check(weight_scale.is_contiguous() and activation_scale.is_contiguous(),
               "weight_scale / activation_scale must be contiguous.")
        _check(weight_scale.numel() == N2, "weight_scale must have 2H elements.")
        _check(activation_scale.numel() == M, "activation_scale must have TokensNum elements.")
    else:
        _check(x.dtype in (torch.float16, torch.bfloat16),
               "dequant_swiglu_quant supports int32 / float16 / bfloat16 inputs.")
        _check(weight_scale is None, "weight_scale must be None for float16 / bfloat16 inputs.")
        _check(activation_scale is None, "activation_scale must be None for float16 / bfloat16 inputs.")
    if quant_scale is not None:
        _check(quant_scale.dtype == torch.float32, "quant_scale must be float32.")
        _check(quant_scale.is_contiguous(), "quant_scale must be contiguous.")
        _check(quant_scale.numel() == H, "quant_scale must have H elements.")
    _on_device("dequant_swiglu_quant", x, weight_scale, activation_scale, quant_scale)
    rc = L.load().cb_dequant_swiglu_quant(_ptr(x), _dtype_code(x.dtype), M, N2, _ptr(weight_scale),
                                          _ptr(activation_scale), _ptr(quant_scale), int(bool(activate_left)),
                                          _ptr(y), _ptr(scale), _stream())
    _raise_status("dequant_swiglu_quant", rc)
    return y, scale


# ------------------------------------------------------------------------------------------------
# MoeGatingTopKSoftmax
# ------------------------------------------------------------------------------------------------
_MGT = "cann_bench.moe_gating_top_k_softmax"


def moe_gating_top_k_softmax_meta(x, finished=None, k=1):
    _check(x.dtype in (torch.float32, torch.float16, torch.bfloat16),
           f"{_MGT} only supports float32, float16 and bfloat16 inputs.")
    _check(x.dim() >= 2, f"{_MGT} requires a tensor with rank >= 2.")
    inner = x.size(-1)
    _check(inner > 0, f"{_MGT} requires a non-empty last dimension.")
    _check(0 < k <= inner, f"{_MGT} requires 0 < k <= x.size(-1).")
    if finished is not None:
        _check(finished.dtype == torch.bool, f"{_MGT} requires a bool 'finished' tensor.")
    shape = tuple(x.shape[:-1]) + (k,)
    return (torch.empty(shape, dtype=x.dtype, device=x.device),
            torch.empty(shape, dtype=torch.int32, device=x.device),
            torch.empty(shape, dtype=torch.int32, device=x.device))


def moe_gating_top_k_softmax(x, finished=None, k=1):
    """(y, expert_idx int32, row_idx int32) = top-k of softmax(x, -1); finished rows get expert E."""
    xc = x.contiguous()
    y, ei, ri = moe_gating_top_k_softmax_meta(xc, finished, k)
    inner = xc.size(-1)
    rows = xc.numel() // inner
    _check(rows > 0, f"{_MGT} requires at least one row.")
    fin = None
    if finished is not None:
        fin = finished.contiguous()
        _check(fin.numel() == rows, f"{_MGT}: finished must have numel == rows.")
    _check(inner <= 2048, f"{_MGT}: the last dimension must not exceed 2048 on this device.")
    _on_device("moe_gating_top_k_softmax", xc, fin)
    rc = L.load().cb_moe_gating_top_k_softmax(_ptr(xc), _dtype_code(xc.dtype), rows, inner, _ptr(fin), k, _ptr(y),
                                              _ptr(ei), _ptr(ri), _stream())
    _raise_status("moe_gating_top_k_softmax", rc)
    return y, ei, ri
