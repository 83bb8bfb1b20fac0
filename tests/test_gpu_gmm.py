"""GPU parity of GroupedMatmul, the float grouped GEMM (cb_grouped_matmul), against the oracle.

The bar for floating point: the GPU accumulates in fp32 in its own order and the oracle in float64.
The fp32 sum's error is bounded by a multiple of sum_k |x_k w_k| (allowed: 1e-6 of it, about
sqrt(K) x 2^-24 for these K), which near cancellations can span a few 16-bit ulps, plus the output
rounding itself: every element within one output ulp + 1e-6 x sum |x_k w_k|, and under 1% of the
16-bit outputs differing at all.  fp32 outputs: within 1e-5 relative + 1e-6 x sum |x_k w_k|.
Shapes cover the MFMA path (K and N multiples of 8: K tails inside a 32-deep stage, partial
column and row tiles, empty and single-row groups, both weight layouts, every bias dtype) and the
fp32 loop (fp32 inputs, K or N off the multiple of 8).  The MFMA cases run on both tile kernels.
"""
import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu

DEV = "cuda"
TD = {"bf16": torch.bfloat16, "f16": torch.float16, "f32": torch.float32}


def bits(t):
    return t.contiguous().view(torch.int16).cpu().numpy().view(np.uint16)


def host(t, dtype):
    return t.cpu().numpy() if dtype == "f32" else bits(t)


def _inputs(counts, K, N, dtype, trans, bias_dtype, seed):
    g = torch.Generator()
    g.manual_seed(seed)
    E, M = len(counts), sum(counts)
    x = torch.randn(M, K, generator=g).to(TD[dtype])
    w = torch.randn((E, N, K) if trans else (E, K, N), generator=g).to(TD[dtype])
    b = None if bias_dtype is None else torch.randn(E, N, generator=g).to(TD[bias_dtype])
    return x, w, b, np.cumsum(counts).tolist()


def _check(y, ref, dtype, x, w, ends, trans):
    # error bound scale: sum_k |x_k| |w_k| per output
    xa, wa = x.abs().double().numpy(), w.abs().double().numpy()
    bound = np.zeros((x.shape[0], y.shape[1]))
    s = 0
    for gi, e in enumerate(ends):
        bound[s:e] = xa[s:e] @ (wa[gi].T if trans else wa[gi])
        s = e
    got = y.float().cpu().numpy().astype(np.float64)
    if dtype == "f32":
        np.testing.assert_array_less(np.abs(got - ref), 1e-5 * np.abs(ref) + 1e-6 * bound + 1e-30)
    else:
        as_val = lambda b: torch.from_numpy(b.astype(np.uint16).view(np.int16)).view(TD[dtype]).double().numpy()
        rv = as_val(ref)
        ulp = np.abs(as_val(ref + 1) - rv)  # the next representable magnitude above |ref|
        np.testing.assert_array_less(np.abs(got - rv), ulp + 1e-6 * bound + 1e-30)
        d = bits(y) != ref
        assert d.size == 0 or d.mean() < 0.01, f"{dtype}: {d.mean():.3%} of outputs differ"


CASES = [
    # (counts, K, N)
    ([300, 0, 45, 1], 256, 384),      # MFMA: empty and single-row groups, two row tiles
    ([130, 7], 40, 136),              # MFMA: K tail inside a stage, partial column tile
    ([520], 64, 128),                 # MFMA: one group, whole tiles
    ([33, 0, 18], 20, 24),            # fp32 loop: K % 8 != 0
]


@pytest.fixture(params=["256", "128"])
def gmm_tile(request, overrides):
    """The 256 x 256 LDS-DMA kernel (default) and the 128 x 128 register-staged one."""
    if request.param == "128":
        overrides(gmm_tile=128)
    return request.param


@pytest.mark.parametrize("counts,K,N", CASES)
@pytest.mark.parametrize("dtype", ["bf16", "f16", "f32"])
@pytest.mark.parametrize("trans", [False, True])
def test_grouped_matmul(cb, orc, gmm_tile, counts, K, N, dtype, trans):
    bias_dtype = {"bf16": "f32", "f16": "f16", "f32": "bf16"}[dtype]
    x, w, b, ends = _inputs(counts, K, N, dtype, trans, bias_dtype, K + N + len(counts))
    ys = cb.grouped_matmul(x.to(DEV), w.to(DEV), ends, bias=b.to(DEV), split_item=2, transpose_weight=trans)
    assert len(ys) == 1 and ys[0].dtype == x.dtype and ys[0].shape == (sum(counts), N)
    ref = orc.grouped_matmul(host(x, dtype), host(w, dtype), ends, host(b, bias_dtype), dtype=dtype,
                             bias_dtype=bias_dtype, trans=trans)
    _check(ys[0], ref, dtype, x.float(), w.float(), ends, trans)


@pytest.mark.parametrize("dtype", ["bf16", "f16"])
def test_grouped_matmul_no_bias_and_split_views(cb, orc, dtype):
    counts = [64, 0, 200]
    x, w, _, ends = _inputs(counts, 128, 256, dtype, False, None, 5)
    outs = cb.grouped_matmul(x.to(DEV), w.to(DEV), ends)  # split_item 0: one view per expert
    assert [o.shape[0] for o in outs] == counts
    y = torch.cat(outs)
    ref = orc.grouped_matmul(host(x, dtype), host(w, dtype), ends, None, dtype=dtype)
    _check(y, ref, dtype, x.float(), w.float(), ends, False)
    # the views share one joined tensor, as the reference's narrow() outputs do
    assert outs[2].data_ptr() == outs[0].data_ptr() + 64 * 256 * 2


def test_grouped_matmul_layouts_agree(cb, gmm_tile):
    """[E, K, N] and [E, N, K] storage of the same weights give bit-identical results on the MFMA
    path (the same fp32 operation order)."""
    x, w, b, ends = _inputs([90, 170], 96, 256, "bf16", False, "f32", 11)
    y1 = cb.grouped_matmul(x.to(DEV), w.to(DEV), ends, bias=b.to(DEV), split_item=3)[0]
    wt = w.transpose(1, 2).contiguous()
    y2 = cb.grouped_matmul(x.to(DEV), wt.to(DEV), ends, bias=b.to(DEV), split_item=3, transpose_weight=True)[0]
    assert torch.equal(y1.view(torch.int16), y2.view(torch.int16))


def test_grouped_matmul_torch_op(cb):
    cb.register_torch_ops()
    x, w, b, ends = _inputs([12, 20], 64, 64, "f16", False, "f16", 13)
    y1 = torch.ops.cann_bench.grouped_matmul(x.to(DEV), w.to(DEV), ends, b.to(DEV), 2, False)
    y2 = cb.grouped_matmul(x.to(DEV), w.to(DEV), ends, bias=b.to(DEV), split_item=2)
    assert torch.equal(y1[0], y2[0])


@pytest.mark.parametrize("dtype,trans", [("bf16", False), ("bf16", True), ("f16", False)])
def test_grouped_matmul_many_tiles(cb, orc, gmm_tile, dtype, trans):
    """A larger ragged problem: 29 row tiles of 128 (partial ones included) x 32 column tiles, a K
    tail inside a stage."""
    counts = [300, 0, 45, 700, 1, 2000, 130]
    K, N = 264, 4096
    x, w, b, ends = _inputs(counts, K, N, dtype, trans, "f32", 77)
    y = cb.grouped_matmul(x.to(DEV), w.to(DEV), ends, bias=b.to(DEV), split_item=2, transpose_weight=trans)[0]
    ref = orc.grouped_matmul(host(x, dtype), host(w, dtype), ends, b.numpy(), dtype=dtype, bias_dtype="f32",
                             trans=trans)
    _check(y, ref, dtype, x.float(), w.float(), ends, trans)


def test_grouped_matmul_golden_fixture(cb):
    """The committed fixture (tests/golden/grouped_matmul.npz, bf16 with a bf16 bias and an empty
    group), within the same bar."""
    import os
    g = np.load(os.path.join(os.path.dirname(__file__), "golden", "grouped_matmul.npz"), allow_pickle=False)
    as_t = lambda a: torch.from_numpy(a.view(np.int16)).view(torch.bfloat16)
    x, w, b = as_t(g["x"]), as_t(g["w"]), as_t(g["bias"])
    ends = g["group_list"].tolist()
    y = cb.grouped_matmul(x.to(DEV), w.to(DEV), ends, bias=b.to(DEV), split_item=2)[0]
    _check(y, g["y"], "bf16", x.float(), w.float(), ends, False)


@pytest.mark.parametrize("N", [(1 << 22) - 8, 1 << 22])
def test_grouped_matmul_wide_n_dispatch(cb, orc, N):
    """N at the LDS kernel's limit: a 256-row block of y stays under 2 GiB at N = 2^22 - 8 (LDS-DMA
    kernel) and reaches it at N = 2^22 (128 x 128 kernel); both against the oracle."""
    counts = [2, 0, 1]
    x, w, b, ends = _inputs(counts, 8, N, "bf16", False, "f32", 23)
    y = cb.grouped_matmul(x.to(DEV), w.to(DEV), ends, bias=b.to(DEV), split_item=2)[0]
    ref = orc.grouped_matmul(host(x, "bf16"), host(w, "bf16"), ends, b.numpy(), dtype="bf16", bias_dtype="f32")
    _check(y, ref, "bf16", x.float(), w.float(), ends, False)
