"""MI355X (gfx950) W8A8 MoE-FFN operators with the reference's `cann_bench` operator surface.

    AddRmsNormDynamicQuant -> GroupedMatmulSwigluQuant -> QuantMatmul / int8 grouped down-projection
    (+ DynamicQuant, and the float GroupedMatmul), with the routing operators on either side of the experts:
    MoeGatingTopKSoftmax, MoeReRouting, DequantSwigluQuant, MoeFinalizeRouting

Python entry points mirror the reference torch ops (same names, argument order and dtypes); the
compute runs in hand-written HIP kernels behind the C ABI of include/cannbench_amd.h.
`register_torch_ops()` additionally exposes them as torch.ops.cann_bench.*.
"""
from .ops import (add_rms_norm_dynamic_quant, dynamic_quant, grouped_matmul, grouped_matmul_int32, grouped_matmul_quant,
                  grouped_matmul_swiglu_quant, grouped_matmul_swiglu_quant_gather, quant_matmul, moe_re_routing, moe_finalize_routing,
                  dequant_swiglu_quant, moe_gating_top_k_softmax)
from . import _lib


def register_torch_ops():
    from . import torch_library
    torch_library.register()


def library_path():
    return _lib.LIB_PATH


__all__ = ["add_rms_norm_dynamic_quant", "dynamic_quant", "grouped_matmul_swiglu_quant",
           "grouped_matmul_swiglu_quant_gather", "quant_matmul",
           "grouped_matmul", "grouped_matmul_quant", "grouped_matmul_int32", "moe_re_routing", "moe_finalize_routing", "dequant_swiglu_quant",
           "moe_gating_top_k_softmax", "register_torch_ops", "library_path"]
