"""GPU parity: every HIP path against the CPU oracle on identical seeded inputs.

Bars: int32 accumulators and routing bit-exact; int8 outputs within +-1 LSB
(the reference's fp32 -> fp16 -> int8 double rounding and exp/division ulps can move a value across
a rounding boundary); fp32 scales within 1e-5 relative (stated bar 1e-3); bf16 / fp16 QuantMatmul
and down-projection outputs bit-exact (same fp32 operation order, no FMA contraction).
Shapes cover every dispatch path: skinny (<= 32 rows per group), tiled (LDS / 32x32x32 MFMA) and
the generic byte-load path (K % 16 != 0 or N not a multiple of 16/32), plus the reference's edge
cases (empty groups, single-row groups, all rows in one expert, M < 16, K tails, all-zero rows).
"""
import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu

DEV = "cuda"


def bits16(t):
    return t.contiguous().view(torch.int16).cpu().numpy().view(np.uint16)


def np_i8(t):
    return t.cpu().numpy()


def assert_int8_close(got, ref, max_frac=0.01, label=""):
    d = np.abs(got.astype(np.int32) - ref.astype(np.int32))
    frac = float((d > 0).mean()) if d.size else 0.0
    assert d.size == 0 or d.max() <= 1, f"{label}: int8 diff {d.max()} > 1 LSB"
    assert frac <= max_frac, f"{label}: {frac:.4%} of int8 outputs differ by 1 LSB"


def rand_i8(shape, g):
    return torch.randint(-127, 128, shape, dtype=torch.int8, generator=g).to(DEV)


def cpu_gen(seed):
    g = torch.Generator()
    g.manual_seed(seed)
    return g


# ---------------------------------------------------------------------------------------------
# AddRmsNormDynamicQuant / DynamicQuant
# ---------------------------------------------------------------------------------------------
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("rows,n", [(64, 7168), (37, 4096), (5, 33), (3, 16384), (1, 1)])
def test_ardq(cb, orc, dtype, rows, n):
    g = cpu_gen(rows * 7 + n)
    x1 = torch.randn(rows, n, generator=g).to(dtype)
    x2 = torch.randn(rows, n, generator=g).to(dtype)
    gamma = (torch.rand(n, generator=g) + 0.5).to(dtype)
    if rows > 2:
        x1[1] = 0
        x2[1] = 0
    y, xo, s = cb.add_rms_norm_dynamic_quant(x1.to(DEV), x2.to(DEV), gamma.to(DEV), 1e-6)
    torch.cuda.synchronize()
    dt = "bf16" if dtype == torch.bfloat16 else "f16"
    yr, xor_, sr = orc.ardq(bits16(x1), bits16(x2), bits16(gamma), dt, 1e-6)
    np.testing.assert_array_equal(bits16(xo), xor_)
    np.testing.assert_allclose(s.cpu().numpy(), sr, rtol=1e-5)
    assert_int8_close(np_i8(y), yr, label="ardq y")


def test_ardq_3d_input(cb, orc):
    g = cpu_gen(3)
    x1 = torch.randn(2, 3, 256, generator=g).to(torch.bfloat16)
    x2 = torch.randn(2, 3, 256, generator=g).to(torch.bfloat16)
    gamma = torch.ones(256).to(torch.bfloat16)
    y, xo, s = cb.add_rms_norm_dynamic_quant(x1.to(DEV), x2.to(DEV), gamma.to(DEV), 1e-6)
    assert y.shape == (2, 3, 256) and s.shape == (2, 3) and xo.dtype == torch.bfloat16
    yr, _, sr = orc.ardq(bits16(x1), bits16(x2), bits16(gamma), "bf16", 1e-6)
    assert_int8_close(np_i8(y), yr)
    np.testing.assert_allclose(s.cpu().numpy(), sr, rtol=1e-5)


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("rows,n", [(1024, 4096), (7, 1000), (3, 12288), (2, 20000)])
def test_dynamic_quant(cb, orc, dtype, rows, n):
    g = cpu_gen(rows + n)
    x = torch.randn(rows, n, generator=g)
    idx = torch.randperm(x.numel(), generator=g)[: max(1, x.numel() // 1000)]
    x.view(-1)[idx] *= 50
    x[0] = 0
    x = x.to(dtype)
    y, s = cb.dynamic_quant(x.to(DEV))
    torch.cuda.synchronize()
    yr, sr = orc.dynamic_quant(bits16(x), "bf16" if dtype == torch.bfloat16 else "f16")
    np.testing.assert_allclose(s.cpu().numpy(), sr, rtol=1e-6)
    assert_int8_close(np_i8(y), yr, label="dq y")


# ---------------------------------------------------------------------------------------------
# raw int32 grouped GEMM: exact
# ---------------------------------------------------------------------------------------------
GEMM_CASES = [
    # (counts, K, N)  -- path exercised
    ([3, 0, 5, 1, 16], 7168, 512),            # skinny, empty group, single-row group
    ([1], 64, 16),                            # M < 16, minimal
    ([40, 0, 129, 7, 256], 1024, 768),        # tiled, ragged row blocks
    ([300], 96, 272),                         # tiled, K tail (96 = 64 + 32), N tail
    ([9, 4], 200, 48),                        # K % 16 != 0 -> generic
    ([50, 3], 64, 40),                        # N % 16 != 0 -> generic
]


@pytest.mark.parametrize("counts,K,N", GEMM_CASES)
def test_grouped_matmul_int32_exact(cb, orc, counts, K, N):
    g = cpu_gen(K + N + len(counts))
    E, M = len(counts), sum(counts)
    x = rand_i8((M, K), g)
    w = rand_i8((E, K, N), g)
    gl = np.cumsum(counts).tolist()
    c = cb.grouped_matmul_int32(x, w, gl).cpu().numpy()
    xn, wn = np_i8(x), np_i8(w)
    s = 0
    for e, cnt in enumerate(counts):
        if cnt:
            np.testing.assert_array_equal(c[s:s + cnt], orc.i8_gemm(xn[s:s + cnt], wn[e]), err_msg=f"group {e}")
        s += cnt


def test_int32_extreme_values(cb):
    """|c| = 127 * 128 * K at the int32 edge region: no overflow, exact."""
    K, N = 7168, 256
    x = torch.full((4, K), -128, dtype=torch.int8, device=DEV)
    w = torch.full((1, K, N), -128, dtype=torch.int8, device=DEV)
    c = cb.grouped_matmul_int32(x, w, [4])
    assert (c == 128 * 128 * K).all()


# ---------------------------------------------------------------------------------------------
# GroupedMatmulSwigluQuant
# ---------------------------------------------------------------------------------------------
GMSQ_CASES = [
    ([3, 0, 5, 1, 16, 0, 2, 8], 7168, 4096),   # decode-like, skinny
    ([1], 512, 256),                           # single row, E = 1
    ([200, 0, 37, 129, 1], 1024, 512),         # tiled, ragged
    ([640], 256, 1024),                        # all rows in one expert, E = 1
    ([100, 300, 37], 400, 896),                # fused persistent path: K tail (400 = 3 x 128 + 16), H = 448 (last column tile half full)
    ([260, 0, 33], 7184, 4128),                # fused path: K = 7168 + 16, H = 2064 (17 column tiles, the last 16 columns wide)
    ([100, 300, 37], 192, 1024),               # fused path, K of 3 stages: lock-step requant (no stage stream across tiles)
    ([70, 0, 513, 40], 128, 4096),             # the same at 16 column tiles (XCD-pair slots), K of 2 stages
    ([6, 11], 80, 48),                         # K % 16 == 0, H = 24 not a multiple of 16 -> generic
    ([4, 4], 40, 64),                          # K % 16 != 0 -> generic
]


def _gmsq_inputs(counts, K, N, seed):
    g = cpu_gen(seed)
    E, M = len(counts), sum(counts)
    x = rand_i8((M, K), g)
    w = rand_i8((E, K, N), g)
    ws = (torch.rand(E, N, generator=g) * 0.009 + 0.001).to(DEV)
    xs = (torch.rand(M, generator=g) * 0.015 + 0.005).to(DEV)
    return x, w, ws, xs, np.cumsum(counts).tolist()


@pytest.mark.parametrize("counts,K,N", GMSQ_CASES)
def test_gmsq(cb, orc, counts, K, N):
    x, w, ws, xs, gl = _gmsq_inputs(counts, K, N, K + N)
    y, ys = cb.grouped_matmul_swiglu_quant(x, w, ws, xs, gl)
    torch.cuda.synchronize()
    yr, ysr = orc.gmsq(np_i8(x), np_i8(w), ws.cpu().numpy(), xs.cpu().numpy(), np.array(gl))
    np.testing.assert_allclose(ys.cpu().numpy(), ysr, rtol=1e-5)
    assert_int8_close(np_i8(y), yr, label="gmsq y")


def test_generic_paths_past_their_grid(cb, orc):
    """The generic kernels and the requant kernel cap their grids and loop over the rest: more
    virtual blocks (rows x 256-column tiles) than the 2^20-block grid, and more rows than the
    requant kernel's 65536 blocks (K = 8 is off the vector paths)."""
    g = cpu_gen(2024)
    counts = [(1 << 19) + 700, 0, 77]  # x 2 column tiles: 1050130 virtual blocks
    E, M, K, N = len(counts), sum(counts), 8, 272
    x = rand_i8((M, K), g)
    w = rand_i8((E, K, N), g)
    gl = np.cumsum(counts).tolist()
    c = cb.grouped_matmul_int32(x, w, gl).cpu().numpy()
    xn, wn = np_i8(x).astype(np.int64), np_i8(w).astype(np.int64)
    s0 = 0
    for e, cnt in enumerate(counts):
        if cnt:
            np.testing.assert_array_equal(c[s0:s0 + cnt], xn[s0:s0 + cnt] @ wn[e], err_msg=f"group {e}")
        s0 += cnt
    del c
    x2, w2, ws2, xs2, gl2 = _gmsq_inputs([40000, 30001], 8, 64, 99)
    y, ys = cb.grouped_matmul_swiglu_quant(x2, w2, ws2, xs2, gl2)
    yr, ysr = orc.gmsq(np_i8(x2), np_i8(w2), ws2.cpu().numpy(), xs2.cpu().numpy(), np.array(gl2))
    np.testing.assert_allclose(ys.cpu().numpy(), ysr, rtol=1e-5)
    assert_int8_close(np_i8(y), yr, label="gmsq y")


@pytest.mark.parametrize("seed", [0, 1, 2])
def test_gmsq_fused_random_routing(cb, orc, seed):
    """The persistent fused-requant GEMM with its 256-workgroup slot mapping (N = 4096: 16 column
    tiles): 256 experts with ragged random counts (a third of them empty, some above 256 rows), so
    row-tile counts are not a multiple of 4 and the last round has workgroups past the end.
    Every row is compared with the oracle."""
    rng = np.random.default_rng(100 + seed)
    counts = rng.integers(0, 120, size=256)
    counts[rng.random(256) < 0.33] = 0
    counts[rng.integers(0, 256, size=3)] = rng.integers(257, 700, size=3)
    counts = [int(c) for c in counts]
    x, w, ws, xs, gl = _gmsq_inputs(counts, 256, 4096, 40 + seed)
    y, ys = cb.grouped_matmul_swiglu_quant(x, w, ws, xs, gl)
    torch.cuda.synchronize()
    yr, ysr = orc.gmsq(np_i8(x), np_i8(w), ws.cpu().numpy(), xs.cpu().numpy(), np.array(gl))
    np.testing.assert_allclose(ys.cpu().numpy(), ysr, rtol=1e-5)
    assert_int8_close(np_i8(y), yr, label=f"gmsq random routing seed {seed}")


def test_gmsq_zero_rows(cb):
    x, w, ws, xs, gl = _gmsq_inputs([5, 3], 256, 512, 1)
    x[2:4] = 0
    y, ys = cb.grouped_matmul_swiglu_quant(x, w, ws, xs, gl)
    assert (y[2:4] == 0).all()
    fm = np.float32(1.1754944e-38) * np.float32(1 / 127)
    assert (ys[2:4].cpu().numpy() == fm).all()


def test_gmsq_zero_rows_fused(cb):
    """All-zero rows inside groups large enough for the persistent fused-requant GEMM."""
    x, w, ws, xs, gl = _gmsq_inputs([70, 300], 512, 1024, 3)
    x[10:12] = 0
    x[200] = 0
    y, ys = cb.grouped_matmul_swiglu_quant(x, w, ws, xs, gl)
    fm = np.float32(1.1754944e-38) * np.float32(1 / 127)
    for r in (10, 11, 200):
        assert (y[r] == 0).all()
        assert ys[r].item() == fm


def test_gmsq_repeatable_and_stream_ordered(cb):
    """Two back-to-back calls on a side stream give identical results (the workspace's row-max
    buffer is re-cleared on every call)."""
    x, w, ws, xs, gl = _gmsq_inputs([20, 7, 33], 512, 512, 5)
    s = torch.cuda.Stream()
    with torch.cuda.stream(s):
        y1, ys1 = cb.grouped_matmul_swiglu_quant(x, w, ws, xs, gl)
        y2, ys2 = cb.grouped_matmul_swiglu_quant(x, w, ws, xs, gl)
    s.synchronize()
    assert torch.equal(y1, y2) and torch.equal(ys1, ys2)


# ---------------------------------------------------------------------------------------------
# QuantMatmul
# ---------------------------------------------------------------------------------------------
QMM_SHAPES = [(256, 1024, 512), (8, 7168, 256), (3, 64, 48), (130, 200, 40)]


@pytest.mark.parametrize("M,K,N", QMM_SHAPES)
def test_quant_matmul_scale_pertoken(cb, orc, M, K, N):
    g = cpu_gen(M + K + N)
    x1 = rand_i8((M, K), g)
    x2 = rand_i8((K, N), g)
    sc = (torch.rand(N, generator=g) * 0.009 + 0.001).to(DEV)
    pt = (torch.rand(M, generator=g) * 0.015 + 0.005).to(DEV)
    out = cb.quant_matmul(x1, x2, sc, pertoken_scale=pt, output_dtype="bfloat16")
    assert out.dtype == torch.bfloat16
    ref = orc.quant_matmul(np_i8(x1), np_i8(x2), sc.cpu().numpy(), pertoken=pt.cpu().numpy(), out_dtype="bf16")
    np.testing.assert_array_equal(bits16(out), ref)


@pytest.mark.parametrize("variant", ["offset_bias_f32", "bias_i32_scalar_scale", "bf16_scale_f16_out",
                                     "batched_bias", "bias_bf16", "default_fp16"])
def test_quant_matmul_flags(cb, orc, variant):
    g = cpu_gen(77)
    B = 3 if variant == "batched_bias" else 1
    M, K, N = 40, 256, 96
    x1 = rand_i8((B, M, K), g)
    x2 = rand_i8((B, K, N), g)
    scale = (torch.rand(N, generator=g) * 0.009 + 0.001)
    pt = (torch.rand(M, generator=g) * 0.015 + 0.005)
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
    elif variant == "batched_bias":
        bias = torch.rand(B, 1, N, generator=g) * 4 - 2
        kw.update(bias=bias.to(DEV))
        okw.update(bias=bias.numpy(), bias_dtype="f32", bias_batched=True)
    elif variant == "bias_bf16":
        bias = (torch.rand(N, generator=g) * 4 - 2).to(torch.bfloat16)
        kw.update(bias=bias.to(DEV))
        okw.update(bias=bits16(bias), bias_dtype="bf16")
    else:  # output_dtype None -> fp16, no pertoken
        kw = {}
        okw = {"out_dtype": "f16"}
    out = cb.quant_matmul(x1.squeeze(0) if B == 1 else x1, x2.squeeze(0) if B == 1 else x2, scale.to(DEV), **kw)
    sc_np = bits16(scale) if scale.dtype == torch.bfloat16 else scale.numpy()
    ref = orc.quant_matmul(np_i8(x1), np_i8(x2), sc_np, **okw)
    np.testing.assert_array_equal(bits16(out).reshape(ref.shape), ref)


def test_weight_block_past_32bit_offsets(cb):
    """A 4 GiB weight block (K * N = 2^32) is past the 32-bit buffer offsets of the vector paths and
    must take the 64-bit generic kernel: sampled columns bit-exact against an int64 product."""
    M, K, N = 2, 65536, 65536
    g = torch.Generator(device=DEV)
    g.manual_seed(7)
    x1 = torch.randint(-127, 128, (M, K), dtype=torch.int8, device=DEV, generator=g)
    x2 = torch.randint(-127, 128, (K, N), dtype=torch.int8, device=DEV, generator=g)
    sc = torch.rand(N, device=DEV, generator=g) * 0.009 + 0.001
    pt = torch.rand(M, device=DEV, generator=g) * 0.015 + 0.005
    out = cb.quant_matmul(x1, x2, sc, pertoken_scale=pt, output_dtype="bfloat16")
    cols = torch.tensor([0, 1, 255, 4096, 30000, 32767, 32768, 50001, N - 17, N - 2, N - 1], device=DEV)
    c = (x1.long()[:, :, None] * x2[:, cols].long()[None]).sum(1)  # exact int64 [M, len(cols)]
    ref = ((c.float() * sc[cols]) * pt[:, None]).to(torch.bfloat16)
    del x2
    assert torch.equal(out[:, cols].view(torch.int16), ref.view(torch.int16))


# ---------------------------------------------------------------------------------------------
# int8 grouped down-projection
# ---------------------------------------------------------------------------------------------
@pytest.mark.parametrize("counts,K,N", [([3, 0, 5, 1, 16, 0, 2, 8], 2048, 7168), ([300, 0, 45], 512, 768),
                                        ([270, 40], 400, 784),
                                        ([5, 6], 40, 64)])
def test_grouped_matmul_quant(cb, orc, counts, K, N):
    g = cpu_gen(K + N)
    E, M = len(counts), sum(counts)
    x = rand_i8((M, K), g)
    w = rand_i8((E, K, N), g)
    ws = (torch.rand(E, N, generator=g) * 0.009 + 0.001).to(DEV)
    xs = (torch.rand(M, generator=g) * 0.015 + 0.005).to(DEV)
    gl = np.cumsum(counts).tolist()
    out = cb.grouped_matmul_quant(x, w, ws, xs, gl)
    ref = orc.grouped_matmul_quant(np_i8(x), np_i8(w), ws.cpu().numpy(), xs.cpu().numpy(), np.array(gl))
    np.testing.assert_array_equal(bits16(out), ref)


# ---------------------------------------------------------------------------------------------
# committed golden fixtures
# ---------------------------------------------------------------------------------------------
def _golden(name):
    import os
    return np.load(os.path.join(os.path.dirname(__file__), "golden", name + ".npz"), allow_pickle=False)


def test_golden_fixtures(cb):
    g = _golden("gmsq")
    y, ys = cb.grouped_matmul_swiglu_quant(torch.from_numpy(g["x"]).to(DEV), torch.from_numpy(g["w"]).to(DEV),
                                           torch.from_numpy(g["ws"]).to(DEV), torch.from_numpy(g["xs"]).to(DEV),
                                           g["group_list"].tolist())
    assert_int8_close(np_i8(y), g["y"], max_frac=0.02)
    np.testing.assert_allclose(ys.cpu().numpy(), g["y_scale"], rtol=1e-5)
    g = _golden("ardq")
    x1 = torch.from_numpy(g["x1"].view(np.int16)).view(torch.bfloat16).to(DEV)
    x2 = torch.from_numpy(g["x2"].view(np.int16)).view(torch.bfloat16).to(DEV)
    gm = torch.from_numpy(g["gamma"].view(np.int16)).view(torch.bfloat16).to(DEV)
    y, xo, s = cb.add_rms_norm_dynamic_quant(x1, x2, gm, float(g["eps"]))
    assert_int8_close(np_i8(y), g["y"])
    np.testing.assert_array_equal(bits16(xo), g["x_out"])
    g = _golden("quant_matmul")
    out = cb.quant_matmul(torch.from_numpy(g["x1"]).to(DEV), torch.from_numpy(g["x2"]).to(DEV),
                          torch.from_numpy(g["scale"]).to(DEV), pertoken_scale=torch.from_numpy(g["pertoken"]).to(DEV),
                          output_dtype="bfloat16")
    np.testing.assert_array_equal(bits16(out), g["out"])
    g = _golden("grouped_matmul_quant")
    out = cb.grouped_matmul_quant(torch.from_numpy(g["x"]).to(DEV), torch.from_numpy(g["w"]).to(DEV),
                                  torch.from_numpy(g["ws"]).to(DEV), torch.from_numpy(g["xs"]).to(DEV),
                                  g["group_list"].tolist())
    np.testing.assert_array_equal(bits16(out), g["out"])
    g = _golden("dynamic_quant")
    y, s = cb.dynamic_quant(torch.from_numpy(g["x"].view(np.int16)).view(torch.float16).to(DEV))
    assert_int8_close(np_i8(y), g["y"])
    np.testing.assert_allclose(s.cpu().numpy(), g["scale"], rtol=1e-6)


def test_torch_ops_registration(cb):
    cb.register_torch_ops()
    x, w, ws, xs, gl = _gmsq_inputs([4, 12], 256, 512, 9)
    y1, ys1 = torch.ops.cann_bench.grouped_matmul_swiglu_quant(x, w, ws, xs, gl)
    y2, ys2 = cb.grouped_matmul_swiglu_quant(x, w, ws, xs, gl)
    assert torch.equal(y1, y2) and torch.equal(ys1, ys2)


def test_mfma_probe_runs_and_is_deterministic(cb):
    """The measurement kernel: status ok, the operation count it reports, identical checksums on
    two runs, and the sink-length check."""
    import ctypes
    import importlib
    L = importlib.import_module("cannbench-operator-solutions_amd._lib")
    lib = L.load()
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    sink = torch.zeros(8 * cus, dtype=torch.int32, device=DEV)
    ops = ctypes.c_int64(0)
    st = torch.cuda.current_stream().cuda_stream
    assert lib.cb_probe_mfma_i8(10, sink.data_ptr(), sink.numel(), ctypes.byref(ops), st) == L.CB_OK
    torch.cuda.synchronize()
    assert ops.value == 2 * cus * 4 * 10 * 8 * 2 * 32 * 32 * 32
    first = sink.clone()
    assert lib.cb_probe_mfma_i8(10, sink.data_ptr(), sink.numel(), ctypes.byref(ops), st) == L.CB_OK
    torch.cuda.synchronize()
    assert torch.equal(first, sink)
    assert lib.cb_probe_mfma_i8(10, sink.data_ptr(), 8, ctypes.byref(ops), st) == L.CB_ERR_SHAPE
    assert lib.cb_probe_mfma_i8(0, sink.data_ptr(), sink.numel(), ctypes.byref(ops), st) == L.CB_ERR_SHAPE


# ---------------------------------------------------------------------------------------------
# GroupedMatmulSwigluQuant with gathered activation rows
# ---------------------------------------------------------------------------------------------
def _random_256_counts(seed):
    rng = np.random.default_rng(200 + seed)
    counts = rng.integers(0, 120, size=256)
    counts[rng.random(256) < 0.33] = 0
    counts[rng.integers(0, 256, size=3)] = rng.integers(257, 700, size=3)
    return [int(c) for c in counts]


GATHER_CASES = [
    # (counts, K, N, source rows T)  -- path exercised
    ([3, 0, 5, 1, 16, 0, 2, 8], 7168, 4096, 20),   # skinny (decode-shaped), XCD-split order
    ([200, 0, 37, 129, 1], 1024, 512, 150),       # persistent fused kernel
    ([100, 300, 37], 400, 896, 90),               # persistent fused kernel, K tail, half column tile
    (_random_256_counts(0), 256, 4096, 3000),     # persistent fused kernel, 256-workgroup slot mapping
    ([6, 11], 80, 48, 9),                          # generic kernels
]


@pytest.mark.parametrize("counts,K,N,T", GATHER_CASES)
def test_gmsq_gather_equals_explicit_gather(cb, counts, K, N, T):
    """The gathered operator equals GroupedMatmulSwigluQuant on x[row_index], x_scale[row_index]:
    the same kernels see the same values, so the results are identical."""
    g = cpu_gen(T + K + N)
    E, M = len(counts), sum(counts)
    x = rand_i8((T, K), g)
    w = rand_i8((E, K, N), g)
    ws = (torch.rand(E, N, generator=g) * 0.009 + 0.001).to(DEV)
    xs = (torch.rand(T, generator=g) * 0.015 + 0.005).to(DEV)
    idx = torch.randint(0, T, (M,), generator=g, dtype=torch.int32).to(DEV)
    gl = np.cumsum(counts).tolist()
    y1, ys1 = cb.grouped_matmul_swiglu_quant_gather(x, idx, w, ws, xs, gl)
    y2, ys2 = cb.grouped_matmul_swiglu_quant(x[idx.long()], w, ws, xs[idx.long()], gl)
    torch.cuda.synchronize()
    assert torch.equal(y1, y2), "gathered int8 output differs from the explicit gather"
    assert torch.equal(ys1, ys2), "gathered scales differ from the explicit gather"


@pytest.mark.parametrize("counts,K,N", [([3, 5, 16], 512, 4096), ([100, 300], 256, 1024)])
def test_gmsq_gather_out_of_range_rows(cb, counts, K, N):
    """Indices outside [0, T) read a zero row with scale 0 (y = 0, y_scale = FLT_MIN / 127), the
    same as the explicit operator on such a row; the other rows are unaffected."""
    T = 40
    g = cpu_gen(7 + K)
    E, M = len(counts), sum(counts)
    x = rand_i8((T, K), g)
    w = rand_i8((E, K, N), g)
    ws = (torch.rand(E, N, generator=g) * 0.009 + 0.001).to(DEV)
    xs = (torch.rand(T, generator=g) * 0.015 + 0.005).to(DEV)
    idx = torch.randint(0, T, (M,), generator=g, dtype=torch.int32)
    idx[1] = -1
    idx[M // 2] = T
    idx[M - 1] = 1 << 30
    gl = np.cumsum(counts).tolist()
    y1, ys1 = cb.grouped_matmul_swiglu_quant_gather(x, idx.to(DEV), w, ws, xs, gl)
    xe = torch.cat([x, torch.zeros(1, K, dtype=torch.int8, device=DEV)])
    xse = torch.cat([xs, torch.zeros(1, device=DEV)])
    ie = torch.where((idx >= 0) & (idx < T), idx, torch.full_like(idx, T)).long().to(DEV)
    y2, ys2 = cb.grouped_matmul_swiglu_quant(xe[ie], w, ws, xse[ie], gl)
    torch.cuda.synchronize()
    assert torch.equal(y1, y2) and torch.equal(ys1, ys2)
    fm = np.float32(1.1754944e-38) * np.float32(1 / 127)
    for r in (1, M // 2, M - 1):
        assert (y1[r] == 0).all() and ys1[r].item() == fm
