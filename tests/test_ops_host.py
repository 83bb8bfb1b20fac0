"""Host-side mirror of the reference plugins, without a GPU: argument validation (same checks and
messages as the reference's TORCH_CHECKs), output shapes / dtypes through the Meta implementations
registered as torch.ops.cann_bench.*, and the absence of any CPU fallback."""
import pytest
import torch


def i8(*s):
    return torch.zeros(*s, dtype=torch.int8)


def f32(*s):
    return torch.zeros(*s, dtype=torch.float32)


@pytest.mark.parametrize("args,msg", [
    ((torch.zeros(4, 8, dtype=torch.int32), i8(2, 8, 16), f32(2, 16), f32(4), [2, 4]), "x must be int8"),
    ((i8(4, 8), i8(2, 8, 16).float(), f32(2, 16), f32(4), [2, 4]), "weight must be int8"),
    ((i8(4, 8), i8(2, 8, 16), f32(2, 16).half(), f32(4), [2, 4]), "weight_scale must be float32"),
    ((i8(4, 8), i8(2, 8, 15), f32(2, 15), f32(4), [2, 4]), "N must be even"),
    ((i8(4, 8), i8(2, 9, 16), f32(2, 16), f32(4), [2, 4]), "K mismatch"),
    ((i8(4, 8), i8(2, 8, 16), f32(2, 16), f32(3), [2, 4]), "x_scale must have M elements"),
    ((i8(4, 8), i8(2, 8, 16), f32(3, 16), f32(4), [2, 4]), "weight_scale must be [E, N]"),
    ((i8(4, 8), i8(2, 8, 16), f32(2, 16), f32(4), [4]), "group_list length must equal the expert count"),
    ((i8(4, 8), i8(2, 8, 16), f32(2, 16), f32(4), [3, 2]), "group_list must be a cumsum <= M"),
    ((i8(4, 8), i8(2, 8, 16), f32(2, 16), f32(4), [1, 3]), "group_list[-1] must equal M"),
])
def test_gmsq_checks(cb, args, msg):
    with pytest.raises(RuntimeError, match=msg.replace("[", r"\[").replace("]", r"\]")):
        cb.grouped_matmul_swiglu_quant(*args)


def test_gmsq_empty_returns_without_device(cb):
    y, ys = cb.grouped_matmul_swiglu_quant(i8(0, 8), i8(2, 8, 16), f32(2, 16), f32(0), [0, 0])
    assert y.shape == (0, 8) and ys.shape == (0,)


def test_gmsq_no_cpu_fallback(cb):
    with pytest.raises(RuntimeError, match="ROCm device"):
        cb.grouped_matmul_swiglu_quant(i8(4, 8), i8(2, 8, 16), f32(2, 16), f32(4), [2, 4])


def test_quant_matmul_checks(cb):
    with pytest.raises(RuntimeError, match="int8 x1 and x2"):
        cb.quant_matmul(f32(4, 8), i8(8, 16), f32(16))
    with pytest.raises(RuntimeError, match="scale length 1 or n"):
        cb.quant_matmul(i8(4, 8), i8(8, 16), f32(3))
    with pytest.raises(RuntimeError, match="pertoken_scale length m"):
        cb.quant_matmul(i8(4, 8), i8(8, 16), f32(16), pertoken_scale=f32(5))
    with pytest.raises(RuntimeError, match="unsupported bias dtype"):
        cb.quant_matmul(i8(4, 8), i8(8, 16), f32(16), bias=torch.zeros(16, dtype=torch.int64))
    with pytest.raises(RuntimeError, match="x1.size\\(-1\\) == x2.size\\(-2\\)"):
        cb.quant_matmul(i8(4, 8), i8(9, 16), f32(16))


def test_norm_quant_checks(cb):
    x = torch.zeros(4, 8, dtype=torch.bfloat16)
    with pytest.raises(RuntimeError, match="gamma dtype must match"):
        cb.add_rms_norm_dynamic_quant(x, x, torch.zeros(8, dtype=torch.float16), 1e-6)
    with pytest.raises(RuntimeError, match="only float16/bfloat16"):
        cb.add_rms_norm_dynamic_quant(x.float(), x.float(), torch.zeros(8), 1e-6)
    with pytest.raises(RuntimeError, match="must not exceed 16384"):
        big = torch.zeros(1, 16385, dtype=torch.bfloat16)
        cb.add_rms_norm_dynamic_quant(big, big, torch.zeros(16385, dtype=torch.bfloat16), 1e-6)
    with pytest.raises(RuntimeError, match="rank >= 2"):
        cb.dynamic_quant(torch.zeros(8, dtype=torch.float16))


def test_torch_ops_meta_shapes(cb):
    cb.register_torch_ops()
    m = torch.device("meta")
    y, ys = torch.ops.cann_bench.grouped_matmul_swiglu_quant(
        torch.empty(10, 64, dtype=torch.int8, device=m), torch.empty(3, 64, 96, dtype=torch.int8, device=m),
        torch.empty(3, 96, device=m), torch.empty(10, device=m), [3, 7, 10])
    assert y.shape == (10, 48) and y.dtype == torch.int8 and ys.shape == (10,) and ys.dtype == torch.float32
    out = torch.ops.cann_bench.quant_matmul(torch.empty(2, 5, 64, dtype=torch.int8, device=m),
                                            torch.empty(2, 64, 32, dtype=torch.int8, device=m),
                                            torch.empty(32, device=m), output_dtype="bfloat16")
    assert out.shape == (2, 5, 32) and out.dtype == torch.bfloat16
    out = torch.ops.cann_bench.quant_matmul(torch.empty(5, 64, dtype=torch.int8, device=m),
                                            torch.empty(64, 32, dtype=torch.int8, device=m), torch.empty(1, device=m))
    assert out.dtype == torch.float16
    y, xo, s = torch.ops.cann_bench.add_rms_norm_dynamic_quant(
        torch.empty(2, 3, 128, dtype=torch.bfloat16, device=m), torch.empty(2, 3, 128, dtype=torch.bfloat16, device=m),
        torch.empty(128, dtype=torch.bfloat16, device=m), 1e-6)
    assert y.shape == (2, 3, 128) and xo.dtype == torch.bfloat16 and s.shape == (2, 3)
    y, s = torch.ops.cann_bench.dynamic_quant(torch.empty(7, 256, dtype=torch.float16, device=m))
    assert y.dtype == torch.int8 and s.shape == (7,)
    out = torch.ops.cann_bench.grouped_matmul_quant(torch.empty(6, 32, dtype=torch.int8, device=m),
                                                    torch.empty(2, 32, 48, dtype=torch.int8, device=m),
                                                    torch.empty(2, 48, device=m), torch.empty(6, device=m), [2, 6])
    assert out.shape == (6, 48) and out.dtype == torch.bfloat16


def test_routing_checks_and_meta(cb):
    with pytest.raises(RuntimeError, match="only gather index mode"):
        cb.moe_re_routing(torch.zeros(4, 8, dtype=torch.bfloat16), torch.ones(2, 2, dtype=torch.int32), idx_type=1)
    with pytest.raises(RuntimeError, match="tokens must be 2D"):
        cb.moe_re_routing(torch.zeros(4, dtype=torch.bfloat16), torch.ones(2, 2, dtype=torch.int32))
    with pytest.raises(RuntimeError, match="per_token_scales must be float32"):
        cb.moe_re_routing(torch.zeros(4, 8, dtype=torch.bfloat16), torch.ones(2, 2, dtype=torch.int32),
                          torch.zeros(4, dtype=torch.float16))
    with pytest.raises(RuntimeError, match="ROCm device"):
        cb.moe_re_routing(torch.zeros(4, 8, dtype=torch.bfloat16), torch.ones(2, 2, dtype=torch.int32))
    with pytest.raises(RuntimeError, match="must be int32"):
        cb.moe_finalize_routing(torch.zeros(4, 8), torch.zeros(4, dtype=torch.int64))
    with pytest.raises(RuntimeError, match="length must be K\\*NUM_ROWS"):
        cb.moe_finalize_routing(torch.zeros(4, 8), torch.zeros(5, dtype=torch.int32), scales=torch.zeros(2, 2))
    with pytest.raises(RuntimeError, match="float16 / float32 / bfloat16"):
        cb.moe_finalize_routing(torch.zeros(4, 8, dtype=torch.int32), torch.zeros(4, dtype=torch.int32))
    with pytest.raises(RuntimeError, match="activation_scale is required"):
        cb.dequant_swiglu_quant(torch.zeros(2, 8, dtype=torch.int32), torch.zeros(8))
    with pytest.raises(RuntimeError, match="weight_scale must be None"):
        cb.dequant_swiglu_quant(torch.zeros(2, 8, dtype=torch.bfloat16), torch.zeros(8))
    with pytest.raises(RuntimeError, match="quant_scale must have H elements"):
        cb.dequant_swiglu_quant(torch.zeros(2, 8, dtype=torch.bfloat16), quant_scale=torch.zeros(3))
    with pytest.raises(RuntimeError, match="0 < k <= x.size"):
        cb.moe_gating_top_k_softmax(torch.zeros(2, 8), None, 9)
    with pytest.raises(RuntimeError, match="bool 'finished'"):
        cb.moe_gating_top_k_softmax(torch.zeros(2, 8), torch.zeros(2), 1)
    with pytest.raises(RuntimeError, match="rank >= 2"):
        cb.moe_gating_top_k_softmax(torch.zeros(8), None, 1)
    cb.register_torch_ops()
    m = torch.device("meta")
    outs = torch.ops.cann_bench.moe_re_routing(torch.empty(10, 32, dtype=torch.int8, device=m),
                                               torch.empty(4, 6, dtype=torch.int64, device=m))
    assert [tuple(o.shape) for o in outs] == [(10, 32), (10,), (10,), (6,)]
    assert outs[3].dtype == torch.int64 and outs[2].dtype == torch.int32
    out = torch.ops.cann_bench.moe_finalize_routing(torch.empty(24, 16, dtype=torch.bfloat16, device=m),
                                                    torch.empty(24, dtype=torch.int32, device=m),
                                                    scales=torch.empty(3, 8, device=m))
    assert out.shape == (3, 16) and out.dtype == torch.bfloat16
    y, s = torch.ops.cann_bench.dequant_swiglu_quant(torch.empty(5, 64, dtype=torch.int32, device=m))
    assert y.shape == (5, 32) and y.dtype == torch.int8 and s.shape == (5,)
    y, ei, ri = torch.ops.cann_bench.moe_gating_top_k_softmax(torch.empty(2, 7, 64, device=m), None, 8)
    assert y.shape == (2, 7, 8) and ei.dtype == torch.int32 and ri.dtype == torch.int32


def test_grouped_matmul_checks_and_outputs(cb):
    """The float GroupedMatmul mirror: the plugin's checks with its messages, split_item views, and
    no CPU fallback once the checks pass (grouped_matmul_plugin.cpp:61-77, 127-157)."""
    f = torch.float32
    x, w = torch.zeros(5, 8, dtype=f), torch.zeros(2, 8, 3, dtype=f)
    with pytest.raises(RuntimeError, match="at least one expert"):
        cb.grouped_matmul(x, torch.zeros(0, 8, 3, dtype=f), [])
    with pytest.raises(RuntimeError, match="at most 64 experts"):
        cb.grouped_matmul(x, torch.zeros(65, 8, 3, dtype=f), [5] * 65)
    with pytest.raises(RuntimeError, match="group_list length must equal"):
        cb.grouped_matmul(x, w, [5])
    with pytest.raises(RuntimeError, match="K dimension mismatch"):
        cb.grouped_matmul(x, torch.zeros(2, 7, 3, dtype=f), [2, 5])
    with pytest.raises(RuntimeError, match="non-decreasing"):
        cb.grouped_matmul(x, w, [3, 2])
    with pytest.raises(RuntimeError, match=r"group_list\[-1\] must equal M"):
        cb.grouped_matmul(x, w, [2, 4])
    with pytest.raises(RuntimeError, match=r"bias must have shape \[E, N\]"):
        cb.grouped_matmul(x, w, [2, 5], bias=torch.zeros(5))
    with pytest.raises(RuntimeError, match="unsupported dtype"):
        cb.grouped_matmul(x.to(torch.int8), w.to(torch.int8), [2, 5])
    with pytest.raises(RuntimeError, match="no CPU path"):
        cb.grouped_matmul(x, w, [2, 5])
    # empty outputs return before any device access; split_item 0/1 give per-expert views
    outs = cb.grouped_matmul(torch.zeros(0, 8, dtype=f), w, [0, 0])
    assert len(outs) == 2 and all(o.shape == (0, 3) for o in outs)
    outs = cb.grouped_matmul(torch.zeros(0, 8, dtype=f), w, [0, 0], split_item=2)
    assert len(outs) == 1 and outs[0].shape == (0, 3)
    views = cb.ops.grouped_matmul_meta(x, torch.zeros(2, 3, 8, dtype=f), [2, 5], transpose_weight=True)
    assert [v.shape for v in views] == [(2, 3), (3, 3)]
