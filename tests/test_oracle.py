"""Pins the CPU oracle (oracle/cb_oracle.c) before it is trusted as the GPU checker.

The reference ships no tests, goldens or fixtures (NOTICE:6-7), so every oracle function is pinned
here by something independent of its own code:
  * numpy / torch library routines (IEEE fp16 and bf16 rounding, int64 matmul),
  * float64 restatements of the documented math (a dropped term, swapped SwiGLU halves or a
    transposed operand moves results by far more than the 1-LSB tolerance),
  * invariants (|y| <= 127, the row max maps to +-127, all-zero rows, y * scale ~ x),
  * reductions (E = 1 GroupedMatmulSwigluQuant == QuantMatmul + SwiGLU + requant; the grouped
    down-projection == per-group QuantMatmul; routing of rows to experts),
  * the committed golden fixtures (tests/golden/*.npz), which freeze the oracle's outputs.
"""
import os

import numpy as np
import pytest
import torch

GOLDEN = os.path.join(os.path.dirname(__file__), "golden")
FLT_MIN = np.float32(1.1754944e-38)


# ---------------------------------------------------------------------------------------------
# rounding primitives
# ---------------------------------------------------------------------------------------------
def _probe_floats(rng, n=20000):
    mags = 2.0 ** rng.uniform(-30, 17, n)
    v = (mags * rng.choice([-1, 1], n)).astype(np.float32)
    ties = (np.arange(-300, 300) + 0.5).astype(np.float32)              # integer ties
    fp16_ties = np.float32(1.0) + np.float32(2.0 ** -11) * np.arange(0, 64, dtype=np.float32)
    edge = np.array([0.0, -0.0, 65504.0, 65519.0, 65520.0, 1e30, -1e30, 6.1e-5, 6.0e-8, 2.9e-8,
                     np.inf, -np.inf], np.float32)
    return np.concatenate([v, ties, fp16_ties, -fp16_ties, edge])


def test_f32_to_f16_matches_numpy(orc):
    v = _probe_floats(np.random.default_rng(1))
    np.testing.assert_array_equal(orc.f32_to_f16_bits(v), v.astype(np.float16).view(np.uint16))


def test_f32_to_bf16_matches_torch(orc):
    v = _probe_floats(np.random.default_rng(2))
    ref = torch.from_numpy(v).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    np.testing.assert_array_equal(orc.f32_to_bf16_bits(v), ref)


def test_rint16_double_rounding(orc):
    v = _probe_floats(np.random.default_rng(3))
    h = v.astype(np.float16).astype(np.float32)
    ref = np.clip(np.rint(h), -128, 127)
    np.testing.assert_array_equal(orc.rint16(v), ref.astype(np.int8))
    # the reference's fp32 -> fp16 -> int8 narrowing differs from direct RNE on purpose:
    # 1.4999 rounds to fp16 1.5, then to even 2 (direct rint gives 1)
    assert orc.rint16(np.float32([1.4999, 2.5, -0.5, 126.97]))[0] == 2
    assert list(orc.rint16(np.float32([2.5, -0.5, 127.6, -300.0, np.nan]))) == [2, 0, 127, -128, 0]


# ---------------------------------------------------------------------------------------------
# exact int32 GEMM
# ---------------------------------------------------------------------------------------------
@pytest.mark.parametrize("m,k,n", [(1, 1, 1), (5, 7, 3), (17, 130, 515), (64, 1024, 96)])
def test_i8_gemm_exact(orc, m, k, n):
    rng = np.random.default_rng(m * 1000 + k)
    a = rng.integers(-128, 128, (m, k), dtype=np.int8)
    b = rng.integers(-128, 128, (k, n), dtype=np.int8)
    np.testing.assert_array_equal(orc.i8_gemm(a, b), a.astype(np.int64) @ b.astype(np.int64))


def test_i8_gemm_extremes(orc):
    a = np.full((3, 7168), -128, np.int8)
    b = np.full((7168, 5), -128, np.int8)
    c = orc.i8_gemm(a, b)
    assert (c == 128 * 128 * 7168).all()  # 117440512 < 2^31: exact int32


# ---------------------------------------------------------------------------------------------
# DynamicQuant
# ---------------------------------------------------------------------------------------------
def _f16_bits(x):
    return x.astype(np.float16).view(np.uint16)


def _bf16_bits(x):
    return torch.from_numpy(np.ascontiguousarray(x, np.float32)).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)


@pytest.mark.parametrize("dtype", ["f16", "bf16"])
def test_dynamic_quant_properties(orc, dtype):
    rng = np.random.default_rng(4)
    x = rng.standard_normal((64, 1000)).astype(np.float32)
    x[3] = 0.0
    x[5, 17] = 60.0
    bits = _f16_bits(x) if dtype == "f16" else _bf16_bits(x)
    xv = orc.f16_bits_to_f32(bits) if dtype == "f16" else orc.bf16_bits_to_f32(bits)
    y, s = orc.dynamic_quant(bits, dtype)
    amax = np.abs(xv).max(axis=1)
    np.testing.assert_array_equal(s[3], np.float32(1e-12) * np.float32(1.0 / 127.0))
    assert (y[3] == 0).all()
    nz = amax > 0
    np.testing.assert_allclose(s[nz], amax[nz] / 127.0, rtol=1e-6)
    assert np.abs(y.astype(np.int32)).max() <= 127
    # the max-abs element of every non-zero row lands on +-127
    am = np.abs(xv).argmax(axis=1)
    assert (np.abs(y[nz, am[nz]]) == 127).all()
    # within one LSB of the float64 quantisation, almost always equal
    ref = np.rint(xv.astype(np.float64) / (amax[:, None].astype(np.float64) / 127.0 + 1e-300))
    d = np.abs(y.astype(np.int32) - ref)
    assert d.max() <= 1 and (d > 0).mean() < 0.01


# ---------------------------------------------------------------------------------------------
# AddRmsNormDynamicQuant
# ---------------------------------------------------------------------------------------------
@pytest.mark.parametrize("dtype,n", [("bf16", 7168), ("f16", 512), ("bf16", 33)])
def test_ardq_against_float64(orc, dtype, n):
    rng = np.random.default_rng(5)
    rows = 24
    x1 = rng.standard_normal((rows, n)).astype(np.float32)
    x2 = rng.standard_normal((rows, n)).astype(np.float32)
    g = rng.uniform(0.5, 1.5, n).astype(np.float32)
    x1[2] = 0.0
    x2[2] = 0.0
    conv = _f16_bits if dtype == "f16" else _bf16_bits
    back = orc.f16_bits_to_f32 if dtype == "f16" else orc.bf16_bits_to_f32
    b1, b2, bg = conv(x1), conv(x2), conv(g)
    eps = 1e-6
    y, xo, s = orc.ardq(b1, b2, bg, dtype, eps)
    xf = back(b1).astype(np.float64) + back(b2).astype(np.float64)
    # xOut: the fp32 sum rounded to the input dtype (a library conversion)
    xsum32 = (back(b1) + back(b2)).astype(np.float32)
    np.testing.assert_array_equal(xo, conv(xsum32))
    rstd = 1.0 / np.sqrt((xf ** 2).mean(axis=1) + eps)
    yn = xf * rstd[:, None] * back(bg).astype(np.float64)[None, :]
    am = np.abs(yn).max(axis=1)
    sref = np.maximum(am, 1e-12) / 127.0
    np.testing.assert_allclose(s, sref, rtol=2e-6)
    ref = np.rint(yn / sref[:, None])
    d = np.abs(y.astype(np.int32) - ref)
    assert d.max() <= 1 and (d > 0).mean() < 0.01
    assert (y[2] == 0).all() and s[2] == np.float32(1e-12) * np.float32(1 / 127)
    nz = am > 0
    assert (np.abs(y[nz]).max(axis=1) == 127).all()


# ---------------------------------------------------------------------------------------------
# GroupedMatmulSwigluQuant
# ---------------------------------------------------------------------------------------------
def _gmsq_case(rng, counts, K, N):
    E, M = len(counts), int(sum(counts))
    x = rng.integers(-127, 128, (M, K), dtype=np.int8)
    w = rng.integers(-127, 128, (E, K, N), dtype=np.int8)
    ws = rng.uniform(0.001, 0.01, (E, N)).astype(np.float32)
    xs = rng.uniform(0.005, 0.02, M).astype(np.float32)
    gl = np.cumsum(counts).astype(np.int64)
    return x, w, ws, xs, gl


def _gmsq_f64(x, w, ws, xs, gl):
    M = x.shape[0]
    H = w.shape[2] // 2
    y = np.zeros((M, H), np.float64)
    ys = np.zeros(M, np.float64)
    starts = np.concatenate([[0], gl[:-1]])
    for g, (s0, s1) in enumerate(zip(starts, gl)):
        if s1 <= s0:
            continue
        c = x[s0:s1].astype(np.int64) @ w[g].astype(np.int64)
        d = c.astype(np.float64) * xs[s0:s1, None] * ws[g][None, :]
        L, R = d[:, :H], d[:, H:]
        act = L / (1.0 + np.exp(-L)) * R
        am = np.maximum(np.abs(act).max(axis=1), float(FLT_MIN))
        ys[s0:s1] = am / 127.0
        y[s0:s1] = np.clip(np.rint(act * (127.0 / am)[:, None]), -128, 127)
    return y, ys


@pytest.mark.parametrize("counts,K,N", [([3, 0, 5, 1], 64, 32), ([17, 0, 0, 40, 2], 160, 96), ([7], 48, 256)])
def test_gmsq_against_float64(orc, counts, K, N):
    rng = np.random.default_rng(sum(counts) + K)
    x, w, ws, xs, gl = _gmsq_case(rng, counts, K, N)
    y, ys = orc.gmsq(x, w, ws, xs, gl)
    yr, ysr = _gmsq_f64(x, w, ws, xs, gl)
    np.testing.assert_allclose(ys, ysr, rtol=1e-5)
    d = np.abs(y.astype(np.int32) - yr)
    assert d.max() <= 1 and (d > 0).mean() < 0.02
    assert (np.abs(y).max(axis=1) >= 126).all()


def test_gmsq_swapped_halves_detected(orc):
    """Gate is the LEFT half: feeding the halves swapped must change the result."""
    rng = np.random.default_rng(9)
    x, w, ws, xs, gl = _gmsq_case(rng, [6], 64, 64)
    y, _ = orc.gmsq(x, w, ws, xs, gl)
    w2 = np.concatenate([w[:, :, 32:], w[:, :, :32]], axis=2)
    ws2 = np.concatenate([ws[:, 32:], ws[:, :32]], axis=1)
    y2, _ = orc.gmsq(x, w2, ws2, xs, gl)
    assert (y != y2).mean() > 0.3


def test_gmsq_routing_and_row_ranges(orc):
    """Each row uses its own expert's weights: the grouped result equals E independent single-group
    calls on the row slices; partial row ranges reproduce the full op."""
    rng = np.random.default_rng(10)
    counts = [4, 0, 9, 1, 6]
    x, w, ws, xs, gl = _gmsq_case(rng, counts, 96, 64)
    y, ys = orc.gmsq(x, w, ws, xs, gl)
    s = 0
    for g, cnt in enumerate(counts):
        if cnt:
            yg, ysg = orc.gmsq(x[s:s + cnt], w[g:g + 1], ws[g:g + 1], xs[s:s + cnt], np.array([cnt]))
            np.testing.assert_array_equal(y[s:s + cnt], yg)
            np.testing.assert_array_equal(ys[s:s + cnt], ysg)
        s += cnt
    yp, ysp = orc.gmsq(x, w, ws, xs, gl, row_begin=3, row_end=15)
    np.testing.assert_array_equal(yp[3:15], y[3:15])
    np.testing.assert_array_equal(ysp[3:15], ys[3:15])
    assert (yp[:3] == 0).all() and (yp[15:] == 0).all()


def test_gmsq_e1_reduces_to_qmm_swiglu_quant(orc):
    """E = 1: GMSQ == QuantMatmul(int32 -> fp32 dequant) + SwiGLU + per-token requant."""
    rng = np.random.default_rng(11)
    x, w, ws, xs, gl = _gmsq_case(rng, [12], 128, 64)
    y, ys = orc.gmsq(x, w, ws, xs, gl)
    c = orc.i8_gemm(x, w[0]).astype(np.float32)
    d = (c * xs[:, None]).astype(np.float32) * ws[0][None, :]
    L, R = d[:, :32], d[:, 32:]
    act = (L / (np.float32(1) + np.exp(-L, dtype=np.float32))) * R
    am = np.abs(act).max(axis=1)
    np.testing.assert_allclose(ys, am * np.float32(1 / 127), rtol=1e-6)
    yq = np.clip(np.rint(act * (np.float32(127) / am)[:, None]), -128, 127)
    assert np.abs(y.astype(np.int32) - yq).max() <= 1


def test_gmsq_zero_rows(orc):
    x, w, ws, xs, gl = _gmsq_case(np.random.default_rng(12), [5], 32, 32)
    x[:] = 0
    y, ys = orc.gmsq(x, w, ws, xs, gl)
    assert (y == 0).all()
    np.testing.assert_array_equal(ys, np.full(5, FLT_MIN * np.float32(1 / 127), np.float32))


# ---------------------------------------------------------------------------------------------
# QuantMatmul and the grouped down-projection
# ---------------------------------------------------------------------------------------------
def _bf16_to_f64(bits):
    return (np.asarray(bits, np.uint16).astype(np.uint32) << 16).view(np.float32).astype(np.float64)


@pytest.mark.parametrize("variant", ["scale_pt", "offset_bias_f32", "bias_i32_scalar_scale", "bf16_scale_f16_out",
                                     "batched_bias"])
def test_quant_matmul_against_float64(orc, variant):
    rng = np.random.default_rng(13)
    B = 3 if variant == "batched_bias" else 1
    M, K, N = 9, 80, 40
    x1 = rng.integers(-127, 128, (B, M, K), dtype=np.int8)
    x2 = rng.integers(-127, 128, (B, K, N), dtype=np.int8)
    scale = rng.uniform(0.001, 0.01, N).astype(np.float32)
    pt = rng.uniform(0.005, 0.02, M).astype(np.float32)
    kw = dict(pertoken=pt, out_dtype="bf16")
    c = np.einsum("bmk,bkn->bmn", x1.astype(np.int64), x2.astype(np.int64)).astype(np.float64)
    if variant == "scale_pt":
        ref = c * scale * pt[None, :, None]
    elif variant == "offset_bias_f32":
        off = rng.uniform(-1, 1, N).astype(np.float32)
        bias = rng.uniform(-2, 2, N).astype(np.float32)
        kw.update(offset=off, bias=bias, bias_dtype="f32")
        ref = (c * scale + off) * pt[None, :, None] + bias
    elif variant == "bias_i32_scalar_scale":
        scale = scale[:1]
        bias = rng.integers(-1000, 1000, N).astype(np.int32)
        kw.update(bias=bias, bias_dtype="i32")
        ref = (c + bias) * scale[0] * pt[None, :, None]
    elif variant == "bf16_scale_f16_out":
        sb = _bf16_bits(scale)
        kw.update(scale_dtype="bf16", out_dtype="f16")
        ref = c * _bf16_to_f64(sb) * pt[None, :, None]
        scale = sb
    else:
        bias = rng.uniform(-2, 2, (B, 1, N)).astype(np.float32)
        kw.update(bias=bias, bias_dtype="f32", bias_batched=True)
        ref = c * scale * pt[None, :, None] + bias
    out = orc.quant_matmul(x1, x2, scale, **kw)
    got = orc.f16_bits_to_f32(out) if kw["out_dtype"] == "f16" else orc.bf16_bits_to_f32(out)
    ulp = 2.0 ** -10 if kw["out_dtype"] == "f16" else 2.0 ** -7
    np.testing.assert_allclose(got, ref, rtol=ulp, atol=1e-6)


def test_grouped_matmul_quant_equals_per_group_qmm(orc):
    rng = np.random.default_rng(14)
    counts = [5, 0, 11, 3]
    E, M, K, N = 4, 19, 64, 48
    x = rng.integers(-127, 128, (M, K), dtype=np.int8)
    w = rng.integers(-127, 128, (E, K, N), dtype=np.int8)
    ws = rng.uniform(0.001, 0.01, (E, N)).astype(np.float32)
    xs = rng.uniform(0.005, 0.02, M).astype(np.float32)
    gl = np.cumsum(counts)
    out = orc.grouped_matmul_quant(x, w, ws, xs, gl)
    s = 0
    for g, cnt in enumerate(counts):
        if cnt:
            ref = orc.quant_matmul(x[s:s + cnt], w[g], ws[g], pertoken=xs[s:s + cnt], out_dtype="bf16")
            np.testing.assert_array_equal(out[s:s + cnt], ref)
        s += cnt


# ---------------------------------------------------------------------------------------------
# golden fixtures (frozen oracle outputs, regenerated only by tests/golden/make_golden.py)
# ---------------------------------------------------------------------------------------------
def _golden(name):
    p = os.path.join(GOLDEN, name + ".npz")
    if not os.path.exists(p):
        pytest.skip(f"missing fixture {p}")
    return np.load(p, allow_pickle=False)


def test_golden_dynamic_quant(orc):
    g = _golden("dynamic_quant")
    y, s = orc.dynamic_quant(g["x"], "f16")
    np.testing.assert_array_equal(y, g["y"])
    np.testing.assert_array_equal(s, g["scale"])


def test_golden_ardq(orc):
    g = _golden("ardq")
    y, xo, s = orc.ardq(g["x1"], g["x2"], g["gamma"], "bf16", float(g["eps"]))
    np.testing.assert_array_equal(y, g["y"])
    np.testing.assert_array_equal(xo, g["x_out"])
    np.testing.assert_array_equal(s, g["scale"])


def test_golden_gmsq(orc):
    g = _golden("gmsq")
    y, ys = orc.gmsq(g["x"], g["w"], g["ws"], g["xs"], g["group_list"])
    np.testing.assert_array_equal(y, g["y"])
    np.testing.assert_array_equal(ys, g["y_scale"])


def test_golden_quant_matmul(orc):
    g = _golden("quant_matmul")
    out = orc.quant_matmul(g["x1"], g["x2"], g["scale"], pertoken=g["pertoken"], out_dtype="bf16")
    np.testing.assert_array_equal(out, g["out"])


def test_golden_grouped_matmul(orc):
    g = _golden("grouped_matmul")
    y = orc.grouped_matmul(g["x"], g["w"], g["group_list"], g["bias"], dtype="bf16", bias_dtype="bf16")
    np.testing.assert_array_equal(y, g["y"])


def test_golden_grouped_matmul_quant(orc):
    g = _golden("grouped_matmul_quant")
    out = orc.grouped_matmul_quant(g["x"], g["w"], g["ws"], g["xs"], g["group_list"])
    np.testing.assert_array_equal(out, g["out"])


# ---------------------------------------------------------------------------------------------
# GroupedMatmul (float)
# ---------------------------------------------------------------------------------------------
def _gmm_np(x, w, ends, bias, trans):
    """float64 numpy product per expert (a library matmul, not the oracle's loop)."""
    y = np.zeros((x.shape[0], w.shape[1] if trans else w.shape[2]))
    s = 0
    for g, e in enumerate(ends):
        wg = w[g].T if trans else w[g]
        y[s:e] = x[s:e] @ wg + (0.0 if bias is None else bias[g])
        s = e
    return y


@pytest.mark.parametrize("trans", [False, True])
def test_grouped_matmul_f32_against_numpy(orc, trans):
    rng = np.random.default_rng(3)
    counts = [7, 0, 30, 1]
    M, K, N, E = sum(counts), 40, 24, len(counts)
    ends = np.cumsum(counts)
    x = rng.standard_normal((M, K)).astype(np.float32)
    w = rng.standard_normal((E, N, K) if trans else (E, K, N)).astype(np.float32)
    b = rng.standard_normal((E, N)).astype(np.float32)
    y = orc.grouped_matmul(x, w, ends, b, dtype="f32", trans=trans)
    ref = _gmm_np(x.astype(np.float64), w.astype(np.float64), ends, b.astype(np.float64), trans)
    np.testing.assert_allclose(y, ref, rtol=1e-6, atol=1e-5)
    # the transposed layout of the same weights gives the same result
    wt = np.ascontiguousarray(np.swapaxes(w, 1, 2))
    np.testing.assert_array_equal(orc.grouped_matmul(x, wt, ends, b, dtype="f32", trans=not trans), y)


@pytest.mark.parametrize("dtype", ["bf16", "f16"])
@pytest.mark.parametrize("bias_dtype", [None, "f32", "bf16"])
def test_grouped_matmul_16bit_rounding(orc, dtype, bias_dtype):
    """16-bit inputs: the output is the float64 product narrowed to fp32 then to the dtype (torch's
    RNE), and a swapped expert or a dropped bias is detected."""
    rng = np.random.default_rng(4)
    counts = [12, 3, 0, 17]
    M, K, N, E = sum(counts), 64, 40, len(counts)
    ends = np.cumsum(counts)
    tdt = torch.bfloat16 if dtype == "bf16" else torch.float16
    xt = torch.from_numpy(rng.standard_normal((M, K)).astype(np.float32)).to(tdt)
    wt = torch.from_numpy(rng.standard_normal((E, K, N)).astype(np.float32)).to(tdt)
    bits = lambda t: t.contiguous().view(torch.int16).numpy().view(np.uint16)
    bt, bb = None, None
    if bias_dtype == "f32":
        bt = torch.from_numpy(rng.standard_normal((E, N)).astype(np.float32))
        bb = bt.numpy()
    elif bias_dtype == "bf16":
        bt = torch.from_numpy(rng.standard_normal((E, N)).astype(np.float32)).to(torch.bfloat16)
        bb = bits(bt)
    y = orc.grouped_matmul(bits(xt), bits(wt), ends, bb, dtype=dtype, bias_dtype=bias_dtype)
    ref = _gmm_np(xt.double().numpy(), wt.double().numpy(), ends, None if bt is None else bt.double().numpy(), False)
    ref_bits = bits(torch.from_numpy(ref.astype(np.float32)).to(tdt))
    d = np.abs(y.astype(np.int32) - ref_bits.astype(np.int32))
    assert d.max() <= 1 and (d > 0).mean() < 0.01
    # an expert swap moves the rows of the swapped groups by far more than one ulp
    ends_sw = ends.copy()
    y_sw = orc.grouped_matmul(bits(xt), bits(wt[[1, 0, 2, 3]]), ends_sw, bb, dtype=dtype, bias_dtype=bias_dtype)
    assert (np.abs(y_sw[:15].astype(np.int32) - y[:15].astype(np.int32)) > 1).mean() > 0.5


def test_grouped_matmul_k0_gives_bias(orc):
    b = np.arange(6, dtype=np.float32).reshape(2, 3)
    y = orc.grouped_matmul(np.zeros((3, 0), np.float32), np.zeros((2, 0, 3), np.float32), [1, 3], b, dtype="f32")
    np.testing.assert_array_equal(y, np.stack([b[0], b[1], b[1]]))
