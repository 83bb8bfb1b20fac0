"""GPU parity of the persistent dequant / int32 GEMM (one continuous DMA stage stream per workgroup).

These tests force a small grid with the library's test override, so every workgroup walks many
tiles (the dequant GEMM on the ring core and the 8-wave int32 GEMM).  Together the cases cover an odd number of K stages (the ring rotates between tiles), both launch orders of the ring core (row tile runs; 4 x 8 tile blocks per XCD), K of
exactly the ring's depth, K shorter than the ring (launched one tile per workgroup instead), ragged
and empty groups, partial row and column tiles, every dequant flag, and the last tile's stages that
fetch nothing.  The bar is the same as the non-persistent path: bit-exact against the oracle.
"""
import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu

DEV = "cuda"


def bits16(t):
    return t.contiguous().view(torch.int16).cpu().numpy().view(np.uint16)


def rand_i8(shape, g):
    return torch.randint(-127, 128, shape, dtype=torch.int8, generator=g).to(DEV)


def cpu_gen(seed):
    g = torch.Generator()
    g.manual_seed(seed)
    return g


@pytest.fixture(params=[3, 5])
def small_grid(request, overrides):
    overrides(persistent_grid=request.param)
    return request.param


GMQ_CASES = [
    # (counts, K, N): 64-deep stages of the ring-core dequant kernel -> 6, 7 (odd: the ring slot
    # rotates by 3 per tile), 4 (exactly its prologue depth), 2 (below it: the 8-wave kernel)
    ([300, 0, 45, 600, 1, 0, 33], 384, 784),
    ([270, 40], 400, 784),
    ([520, 17, 0], 256, 512),
    ([520, 17, 0], 96, 512),
    # 8 column tiles (the last one 248 wide) and at least 4 row tiles: the block launch order (4 row
    # tiles x 8 column tiles per XCD and round), with a partial last band of row tiles
    ([520, 17, 0, 700], 256, 2040),
    ([300, 0, 45, 600, 1, 0, 33, 256, 90], 448, 4096),
    # N % 8 == 4 with K of at least 4 stages: the ring core's 16-byte stores need N % 8 == 0, so
    # these take the 8-wave persistent kernel
    ([300, 0, 45, 600], 384, 772),
]


@pytest.mark.parametrize("counts,K,N", GMQ_CASES)
def test_persistent_grouped_matmul_quant(cb, orc, small_grid, counts, K, N):
    g = cpu_gen(K + N + len(counts))
    E, M = len(counts), sum(counts)
    x = rand_i8((M, K), g)
    w = rand_i8((E, K, N), g)
    ws = (torch.rand(E, N, generator=g) * 0.009 + 0.001).to(DEV)
    xs = (torch.rand(M, generator=g) * 0.015 + 0.005).to(DEV)
    gl = np.cumsum(counts).tolist()
    out = cb.grouped_matmul_quant(x, w, ws, xs, gl)
    ref = orc.grouped_matmul_quant(x.cpu().numpy(), w.cpu().numpy(), ws.cpu().numpy(), xs.cpu().numpy(),
                                   np.array(gl))
    np.testing.assert_array_equal(bits16(out), ref)


@pytest.mark.parametrize("counts,K,N", [([40, 0, 129, 7, 256], 1024, 768), ([300, 77], 384, 272)])
def test_persistent_grouped_matmul_int32(cb, orc, small_grid, counts, K, N):
    g = cpu_gen(K * 3 + N)
    E = len(counts)
    x = rand_i8((sum(counts), K), g)
    w = rand_i8((E, K, N), g)
    c = cb.grouped_matmul_int32(x, w, np.cumsum(counts).tolist()).cpu().numpy()
    xn, wn = x.cpu().numpy(), w.cpu().numpy()
    s = 0
    for e, cnt in enumerate(counts):
        if cnt:
            np.testing.assert_array_equal(c[s:s + cnt], orc.i8_gemm(xn[s:s + cnt], wn[e]), err_msg=f"group {e}")
        s += cnt


@pytest.mark.parametrize("variant", ["pertoken_bf16", "offset_bias_f32", "bias_i32_scalar_scale",
                                     "bf16_scale_f16_out", "default_fp16"])
def test_persistent_quant_matmul_flags(cb, orc, small_grid, variant):
    g = cpu_gen(91)
    M, K, N = 600, 384, 528  # 3 x 3 tiles, the last column tile 16 wide
    x1 = rand_i8((M, K), g)
    x2 = rand_i8((K, N), g)
    scale = torch.rand(N, generator=g) * 0.009 + 0.001
    pt = torch.rand(M, generator=g) * 0.015 + 0.005
    kw, okw = {"pertoken_scale": pt.to(DEV), "output_dtype": "bfloat16"}, {"pertoken": pt.numpy(), "out_dtype": "bf16"}
    if variant == "offset_bias_f32":
        off = torch.rand(N, generator=g) - 0.5
        bias = torch.rand(N, generator=g) * 4 - 2
        kw.update(offset=off.to(DEV), bias=bias.to(DEV))
        okw.update(offset=off.numpy(), bias=bias.numpy(), bias_dtype="f32")
    elif variant == "bias_i32_scalar_scale":
        scale = scale[:1]
        bias = torch.randint(-1000, 1000, (N,), dtype=torch.int32, generator=g)
        kw.update(bias=bias.to(DEV))
        okw.update(bias=bias.numpy(), bias_dtype="i32")
    elif variant == "bf16_scale_f16_out":
        scale = scale.to(torch.bfloat16)
        kw["output_dtype"] = "float16"
        okw.update(scale_dtype="bf16", out_dtype="f16")
    elif variant == "default_fp16":
        kw, okw = {}, {"out_dtype": "f16"}
    out = cb.quant_matmul(x1, x2, scale.to(DEV), **kw)
    sc_np = bits16(scale) if scale.dtype == torch.bfloat16 else scale.numpy()
    ref = orc.quant_matmul(x1.cpu().numpy(), x2.cpu().numpy(), sc_np, **okw)
    np.testing.assert_array_equal(bits16(out).reshape(ref.shape), ref)


@pytest.mark.parametrize("N", [772, 100])
def test_quant_matmul_n_mod8_4(cb, orc, small_grid, N):
    """QuantMatmul with N % 8 == 4 and K >= 256 (outside the ring core's 16-byte store gate):
    bit-exact against the oracle on the kernel these shapes take."""
    g = cpu_gen(N)
    M, K = 300, 512
    x1 = rand_i8((M, K), g)
    x2 = rand_i8((K, N), g)
    scale = torch.rand(N, generator=g) * 0.009 + 0.001
    pt = torch.rand(M, generator=g) * 0.015 + 0.005
    out = cb.quant_matmul(x1, x2, scale.to(DEV), pertoken_scale=pt.to(DEV), output_dtype="bfloat16")
    ref = orc.quant_matmul(x1.cpu().numpy(), x2.cpu().numpy(), scale.numpy(), pertoken=pt.numpy(), out_dtype="bf16")
    np.testing.assert_array_equal(bits16(out).reshape(ref.shape), ref)


def test_persistent_default_grid_matches_one_tile_per_workgroup(cb, overrides):
    """More tiles than CUs: the default launch is persistent; bit-identical to the launch with one
    tile per workgroup (persistent launch off) and to the oracle's int32 products on a sample."""
    g = cpu_gen(5)
    counts = [600, 13, 0, 700, 256, 640, 1, 550, 900]  # 19 row tiles x 16 column tiles > 256
    K, N = 256, 4096
    E, M = len(counts), sum(counts)
    x = rand_i8((M, K), g)
    w = rand_i8((E, K, N), g)
    ws = (torch.rand(E, N, generator=g) * 0.009 + 0.001).to(DEV)
    xs = (torch.rand(M, generator=g) * 0.015 + 0.005).to(DEV)
    gl = np.cumsum(counts).tolist()
    a = cb.grouped_matmul_quant(x, w, ws, xs, gl)
    c = cb.grouped_matmul_int32(x, w, gl)
    overrides(persistent_grid=-1)  # persistent launch off: one tile per workgroup
    b = cb.grouped_matmul_quant(x, w, ws, xs, gl)
    d = cb.grouped_matmul_int32(x, w, gl)
    assert torch.equal(a.view(torch.int16), b.view(torch.int16))
    assert torch.equal(c, d)
    # int32 products of every group's first and last rows against a CPU int64 product
    xn, wn, cn = x.cpu().numpy().astype(np.int64), w.cpu().numpy().astype(np.int64), c.cpu().numpy()
    s = 0
    for e, cnt in enumerate(counts):
        for r in {s, s + cnt - 1} if cnt else ():
            np.testing.assert_array_equal(cn[r], xn[r] @ wn[e], err_msg=f"group {e} row {r}")
        s += cnt


@pytest.mark.parametrize("counts,K,N", [
    ([100, 300, 37], 400, 896),              # prefill-shaped groups, K tail, half-full last column tile
    ([260, 0, 33], 7184, 4128),              # prefill-shaped, 17 column tiles
    ([3, 0, 5, 1, 16, 0, 2, 8], 7168, 4096),  # decode-shaped groups
])
def test_gmsq_two_pass_path_on_fused_shapes(cb, orc, overrides, counts, K, N):
    """GroupedMatmulSwigluQuant's two-pass path, the one a call takes when its fused kernel's grid
    cannot all be resident, on the shapes that normally take the fused prefill and decode kernels:
    against the oracle to the fused path's bar (scales 1e-5 relative, int8 within one step on at
    most 1% of elements)."""
    g = cpu_gen(K + N)
    E, M = len(counts), sum(counts)
    x = rand_i8((M, K), g)
    w = rand_i8((E, K, N), g)
    ws = (torch.rand(E, N, generator=g) * 0.009 + 0.001).to(DEV)
    xs = (torch.rand(M, generator=g) * 0.015 + 0.005).to(DEV)
    gl = np.cumsum(counts).tolist()
    overrides(persistent_grid=-1)  # fused launches off
    y, ys = cb.grouped_matmul_swiglu_quant(x, w, ws, xs, gl)
    torch.cuda.synchronize()
    yr, ysr = orc.gmsq(x.cpu().numpy(), w.cpu().numpy(), ws.cpu().numpy(), xs.cpu().numpy(), np.array(gl))
    np.testing.assert_allclose(ys.cpu().numpy(), ysr, rtol=1e-5)
    d = np.abs(y.cpu().numpy().astype(np.int32) - yr.astype(np.int32))
    assert d.max() <= 1, f"int8 diff {d.max()}"
    assert (d > 0).mean() <= 0.01, f"{(d > 0).mean():.4%} differ by one step"
