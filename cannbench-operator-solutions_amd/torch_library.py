"""Registers the operators as torch.ops.cann_bench.* with the reference's schema strings.

The reference registers these schemas with TORCH_LIBRARY_FRAGMENT(cann_bench, m) and provides a
Meta (shape inference) and a PrivateUse1 (NPU) implementation per op, e.g.
operators/groupedmatmulswigluquant/csrc/ops/grouped_matmul_swiglu_quant/op_plugin/gmsq_plugin.cpp:38-65,147-150.
Here the device implementation is registered for the CUDA dispatch key, which is the ROCm device
key in PyTorch-ROCm.  `grouped_matmul_quant` is this library's int8 down-projection (no reference
counterpart).
"""
import torch

from . import ops

SCHEMAS = {
    "add_rms_norm_dynamic_quant":
        "add_rms_norm_dynamic_quant(Tensor x1, Tensor x2, Tensor gamma, float epsilon) -> (Tensor y, Tensor xOut, Tensor scaleOut)",
    "dynamic_quant":
        "dynamic_quant(Tensor x) -> (Tensor y, Tensor scale)",
    "grouped_matmul_swiglu_quant":
        "grouped_matmul_swiglu_quant(Tensor x, Tensor weight, Tensor weight_scale, Tensor x_scale, int[] group_list) -> (Tensor y, Tensor y_scale)",
    "quant_matmul":
        "quant_matmul(Tensor x1, Tensor x2, Tensor scale, *, Tensor? offset=None, Tensor? pertoken_scale=None, Tensor? bias=None, str? output_dtype=None) -> Tensor",
    "grouped_matmul":
        "grouped_matmul(Tensor x, Tensor weight, int[] group_list, Tensor? bias=None, int split_item=0, bool transpose_weight=False) -> Tensor[]",
    "grouped_matmul_quant":
        "grouped_matmul_quant(Tensor x, Tensor weight, Tensor weight_scale, Tensor x_scale, int[] group_list) -> Tensor",
    "moe_re_routing":
        "moe_re_routing(Tensor tokens, Tensor expert_token_num_per_rank, Tensor? per_token_scales=None, int expert_token_num_type=1, int idx_type=0) -> (Tensor, Tensor, Tensor, Tensor)",
    "moe_finalize_routing":
        "moe_finalize_routing(Tensor expanded_permuted_rows, Tensor expanded_src_to_dst_row, Tensor? skip1=None, Tensor? skip2=None, Tensor? bias=None, Tensor? scales=None, Tensor? expert_for_source_row=None, int drop_pad_mode=0) -> Tensor out",
    "dequant_swiglu_quant":
        "dequant_swiglu_quant(Tensor x, Tensor? weight_scale=None, Tensor? activation_scale=None, Tensor? quant_scale=None, bool activate_left=False) -> (Tensor y, Tensor scale)",
    "moe_gating_top_k_softmax":
        "moe_gating_top_k_softmax(Tensor x, Tensor? finished=None, int k=1) -> (Tensor y, Tensor expert_idx, Tensor row_idx)",
}

_IMPLS = {
    "add_rms_norm_dynamic_quant": (ops.add_rms_norm_dynamic_quant, ops.add_rms_norm_dynamic_quant_meta),
    "dynamic_quant": (ops.dynamic_quant, ops.dynamic_quant_meta),
    "grouped_matmul_swiglu_quant": (ops.grouped_matmul_swiglu_quant, ops.grouped_matmul_swiglu_quant_meta),
    "quant_matmul": (ops.quant_matmul,
                     lambda x1, x2, scale, *, offset=None, pertoken_scale=None, bias=None, output_dtype=None:
                     ops.quant_matmul_meta(x1, x2, scale, offset, pertoken_scale, bias, output_dtype)),
    "grouped_matmul": (ops.grouped_matmul, ops.grouped_matmul_meta),
    "grouped_matmul_quant": (ops.grouped_matmul_quant, ops.grouped_matmul_quant_meta),
    "moe_re_routing": (ops.moe_re_routing, ops.moe_re_routing_meta),
    "moe_finalize_routing": (ops.moe_finalize_routing, ops.moe_finalize_routing_meta),
    "dequant_swiglu_quant": (ops.dequant_swiglu_quant, ops.dequant_swiglu_quant_meta),
    "moe_gating_top_k_softmax": (ops.moe_gating_top_k_softmax, ops.moe_gating_top_k_softmax_meta),
}

_lib_def = None


def register():
    """Idempotently define torch.ops.cann_bench.* (CUDA/ROCm + Meta implementations)."""
    global _lib_def
    if _lib_def is not None:
        return
    lib = torch.library.Library("cann_bench", "DEF")
    for name, schema in SCHEMAS.items():
        lib.define(schema)
        dev, meta = _IMPLS[name]
        lib.impl(name, dev, "CUDA")
        lib.impl(name, meta, "Meta")
    _lib_def = lib
