"""Pins the oracle's routing operators (CPU only).

Each check is independent of the oracle's own formulation:
  * MoeReRouting: the expert-major order is a stable sort of the source rows by expert id (the
    source is rank-major and expert-ordered inside each rank), so permute_idx must equal numpy's
    stable argsort; the column sums are numpy sums.
  * MoeFinalizeRouting: a vectorised numpy float32 evaluation in the same operation order (IEEE
    float32 add/mul, so bit-equal), drop-mode layout equivalence (mode 0 with esdr laid out [K, R]
    == mode 2 with the transposed [R, K] layout), and the K=1 / no-extras reduction to a pure gather.
  * DequantSwigluQuant: float64 SwiGLU (y within 1 LSB), the left/right swap identity, and the
    int32 path with unit scales equal to the 16-bit path on the same integer values.
  * MoeGatingTopKSoftmax: torch.softmax + torch.topk on tie-free rows, a known answer for an
    all-equal row (columns 0..k-1, value 1/E), finished rows, and the row_idx closed form.
"""
import numpy as np
import pytest
import torch

from oracle import oracle as orc


def _bf16_bits(a):
    return torch.from_numpy(np.asarray(a, np.float32)).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)


def _f16_bits(a):
    return np.asarray(a, np.float32).astype(np.float16).view(np.uint16)


# ---------------------------------------------------------------------------------------------
# MoeReRouting
# ---------------------------------------------------------------------------------------------
@pytest.mark.parametrize("n,e,cnt_max", [(1, 1, 5), (4, 8, 7), (16, 32, 3), (3, 5, 0)])
def test_re_routing_is_stable_sort_by_expert(n, e, cnt_max):
    rng = np.random.default_rng(n * 100 + e)
    cnt = rng.integers(0, cnt_max + 1, size=(n, e))
    total = int(cnt.sum())
    A = total + 3
    H = 24
    tokens = rng.integers(-128, 128, size=(A, H), dtype=np.int8)
    scales = rng.random(A).astype(np.float32)
    out, osc, oidx, etn, routed = orc.moe_re_routing(tokens, cnt, scales)
    assert routed == total
    np.testing.assert_array_equal(etn, cnt.sum(axis=0))
    # expert id of every routed source row: rank-major, expert-ordered within each rank
    src_expert = np.concatenate([np.repeat(np.arange(e), cnt[i]) for i in range(n)]) if total else np.zeros(0, int)
    want = np.argsort(src_expert, kind="stable")
    np.testing.assert_array_equal(oidx[:total], want)
    np.testing.assert_array_equal(out[:total], tokens[want])
    np.testing.assert_array_equal(osc[:total], scales[want])


def test_re_routing_without_scales_writes_zero_scales():
    cnt = np.array([[2, 1], [0, 3]])
    tokens = np.arange(6 * 4, dtype=np.uint16).reshape(6, 4)
    out, osc, oidx, etn, _ = orc.moe_re_routing(tokens, cnt, None)
    # rank0: e0 rows 0,1; e1 row 2.  rank1: e1 rows 3,4,5.  expert-major: 0,1 | 2,3,4,5
    np.testing.assert_array_equal(oidx, [0, 1, 2, 3, 4, 5])
    np.testing.assert_array_equal(osc, 0)
    np.testing.assert_array_equal(etn, [2, 4])
    cnt = np.array([[1, 2], [2, 1]])
    out, osc, oidx, etn, _ = orc.moe_re_routing(tokens, cnt, None)
    # rank0: e0 row 0; e1 rows 1,2.  rank1: e0 rows 3,4; e1 row 5 -> 0,3,4 | 1,2,5
    np.testing.assert_array_equal(oidx, [0, 3, 4, 1, 2, 5])
    np.testing.assert_array_equal(out, tokens[[0, 3, 4, 1, 2, 5]])


# ---------------------------------------------------------------------------------------------
# MoeFinalizeRouting
# ---------------------------------------------------------------------------------------------
def _mfr_numpy_f32(epr, esdr_rk, skip1, skip2, bias, scales, expert):
    """Vectorised float32 restatement: esdr_rk [R, K] row-arranged destination rows."""
    R, K = esdr_rk.shape
    H = epr.shape[1]
    acc = np.zeros((R, H), np.float32)
    if skip1 is not None:
        acc = skip1.astype(np.float32).copy()
    if skip2 is not None:
        acc = (acc + skip2.astype(np.float32)).astype(np.float32)
    for k in range(K):
        p = esdr_rk[:, k]
        valid = (p >= 0) & (p < epr.shape[0])
        term = epr[np.where(valid, p, 0)].astype(np.float32)
        if bias is not None:
            eid = expert[:, k]
            bv = (eid >= 0) & (eid < bias.shape[0])
            term = np.where(bv[:, None], term + bias[np.where(bv, eid, 0)], term).astype(np.float32)
        if scales is not None:
            term = (term * scales[:, k:k + 1]).astype(np.float32)
        acc = np.where(valid[:, None], acc + term, acc).astype(np.float32)
    return acc


@pytest.mark.parametrize("with_extras", [False, True])
def test_finalize_matches_vectorised_float32(with_extras):
    rng = np.random.default_rng(7)
    R, K, H, E = 33, 4, 40, 6
    num_dst = R * K
    epr = rng.standard_normal((num_dst, H)).astype(np.float32)
    esdr_rk = rng.permutation(num_dst).reshape(R, K).astype(np.int32)
    esdr_rk[3, 1] = -1
    esdr_rk[5, 2] = num_dst + 4
    skip1 = rng.standard_normal((R, H)).astype(np.float32) if with_extras else None
    skip2 = rng.standard_normal((R, H)).astype(np.float32) if with_extras else None
    bias = rng.standard_normal((E, H)).astype(np.float32) if with_extras else None
    expert = rng.integers(-1, E + 1, size=(R, K)).astype(np.int32)
    scales = rng.random((R, K)).astype(np.float32)
    want = _mfr_numpy_f32(epr, esdr_rk, skip1, skip2, bias, scales, expert if with_extras else None)
    got2 = orc.moe_finalize_routing(epr, "f32", esdr_rk.ravel(), K, skip1, skip2, bias, scales, "f32",
                                    expert if with_extras else None, drop_pad_mode=2)
    got0 = orc.moe_finalize_routing(epr, "f32", esdr_rk.T.ravel(), K, skip1, skip2, bias, scales, "f32",
                                    expert if with_extras else None, drop_pad_mode=0)
    np.testing.assert_array_equal(got2, want)
    np.testing.assert_array_equal(got0, want)
    # modes outside [0, 3] clamp
    np.testing.assert_array_equal(
        orc.moe_finalize_routing(epr, "f32", esdr_rk.ravel(), K, skip1, skip2, bias, scales, "f32",
                                 expert if with_extras else None, drop_pad_mode=9), want)


def test_finalize_k1_is_gather_and_bias_needs_expert():
    rng = np.random.default_rng(3)
    epr = _bf16_bits(rng.standard_normal((10, 16)))
    esdr = np.array([9, 0, 4, 4, 2], np.int32)
    got = orc.moe_finalize_routing(epr, "bf16", esdr, 1)
    np.testing.assert_array_equal(got, epr[esdr])
    bias = _bf16_bits(rng.standard_normal((3, 16)))
    # bias without expert_for_source_row is ignored
    np.testing.assert_array_equal(orc.moe_finalize_routing(epr, "bf16", esdr, 1, bias=bias), epr[esdr])


def test_finalize_bf16_rounds_half_even():
    # acc = 1 + 2^-8 lies half way between bf16 neighbours 1 and 1 + 2^-7: RNE -> 1.0
    epr = np.array([[1.0], [2.0 ** -8]], np.float32)
    esdr = np.array([0, 1], np.int32)  # R=1, K=2, mode 2
    scales = np.ones((1, 2), np.float32)
    got = orc.moe_finalize_routing(_bf16_bits(epr), "bf16", esdr, 2, scales=scales, scales_dtype="f32",
                                   drop_pad_mode=2)
    assert orc.bf16_bits_to_f32(got)[0, 0] == 1.0
    # an fp32 row keeps the exact fp32 sum
    epr2 = np.array([[1.0], [3 * 2.0 ** -8]], np.float32)
    got2 = orc.moe_finalize_routing(epr2.astype(np.float32), "f32", esdr, 2, scales=scales, drop_pad_mode=2)
    assert got2[0, 0] == np.float32(1 + 3 * 2.0 ** -8)


# ---------------------------------------------------------------------------------------------
# DequantSwigluQuant
# ---------------------------------------------------------------------------------------------
def _dqsq_f64(A, B, act_left):
    G = A if act_left else B
    return A * B / (1.0 + np.exp(-G))


@pytest.mark.parametrize("act_left", [False, True])
def test_dqsq_f16_against_float64(act_left):
    rng = np.random.default_rng(11)
    M, H = 17, 96
    x = (rng.standard_normal((M, 2 * H)) * 3).astype(np.float16)
    y, s = orc.dequant_swiglu_quant(x.view(np.uint16), "f16", activate_left=act_left)
    xf = x.astype(np.float64)
    out = _dqsq_f64(xf[:, :H], xf[:, H:], act_left)
    s64 = np.maximum(np.abs(out).max(axis=1) / 127.0, 1e-12)
    np.testing.assert_allclose(s, s64, rtol=1e-5)
    q = np.clip(np.rint(out / s64[:, None]), -128, 127)
    assert np.abs(y.astype(np.int32) - q).max() <= 1
    assert np.abs(y).max() <= 127 and (np.abs(y).max(axis=1) == 127).all()


def test_dqsq_left_right_swap_identity_and_int32_unit_scales():
    rng = np.random.default_rng(5)
    M, H = 9, 64
    v = rng.integers(-300, 300, size=(M, 2 * H)).astype(np.int32)
    qs = (rng.random(H) + 0.5).astype(np.float32)
    y0, s0 = orc.dequant_swiglu_quant(v, "i32", np.ones(2 * H, np.float32), np.ones(M, np.float32), qs, False)
    swapped = np.concatenate([v[:, H:], v[:, :H]], axis=1)
    y1, s1 = orc.dequant_swiglu_quant(swapped, "i32", np.ones(2 * H, np.float32), np.ones(M, np.float32), qs, True)
    np.testing.assert_array_equal(y0, y1)
    np.testing.assert_array_equal(s0, s1)
    # integers up to 300 are exact in fp16: the 16-bit path gives the same bits
    y2, s2 = orc.dequant_swiglu_quant(v.astype(np.float16).view(np.uint16), "f16", quant_scale=qs)
    np.testing.assert_array_equal(y0, y2)
    np.testing.assert_array_equal(s0, s2)


def test_dqsq_scales_order_weight_then_quant_then_activation():
    # int32 x with weight_scale w, quant_scale q, activation_scale a: the linear half is
    # ((x * w) * q) * a and the gate half (x * w) * a  -> compare with float64 on exact inputs
    M, H = 2, 8
    x = np.arange(1, M * 2 * H + 1, dtype=np.int32).reshape(M, 2 * H) - 10
    w = np.linspace(0.01, 0.05, 2 * H).astype(np.float32)
    a = np.array([0.5, 2.0], np.float32)
    q = np.linspace(0.5, 1.5, H).astype(np.float32)
    y, s = orc.dequant_swiglu_quant(x, "i32", w, a, q, False)
    A = x[:, :H] * w[:H].astype(np.float64) * q * a[:, None]
    B = x[:, H:] * w[H:].astype(np.float64) * a[:, None]
    out = _dqsq_f64(A, B, False)
    s64 = np.abs(out).max(axis=1) / 127.0
    np.testing.assert_allclose(s, s64, rtol=1e-5)
    assert np.abs(y - np.rint(out / s64[:, None])).max() <= 1


def test_dqsq_zero_row_scale_floor():
    y, s = orc.dequant_swiglu_quant(np.zeros((2, 8), np.uint16), "bf16")
    np.testing.assert_array_equal(s, np.float32(1e-12))
    np.testing.assert_array_equal(y, 0)


# ---------------------------------------------------------------------------------------------
# MoeGatingTopKSoftmax
# ---------------------------------------------------------------------------------------------
@pytest.mark.parametrize("dtype", ["f32", "bf16", "f16"])
@pytest.mark.parametrize("E,k", [(8, 2), (64, 6), (256, 8), (129, 1)])
def test_gating_against_torch_on_tie_free_rows(dtype, E, k):
    rows = 37
    g = torch.Generator().manual_seed(E * 10 + k)
    # a permutation per row keeps every value distinct in every dtype
    base = torch.stack([torch.randperm(E, generator=g) for _ in range(rows)]).float() * (4.0 / E) - 2.0
    tdt = {"f32": torch.float32, "bf16": torch.bfloat16, "f16": torch.float16}[dtype]
    xt = base.to(tdt)
    assert all(len(set(r.tolist())) == E for r in xt.float())
    xnp = xt.float().numpy() if dtype == "f32" else xt.view(torch.int16).numpy().view(np.uint16)
    y, ei, ri = orc.moe_gating_top_k_softmax(xnp, dtype, k)
    p = torch.softmax(xt.float(), dim=-1)
    tv, ti = torch.topk(p, k, dim=-1)
    np.testing.assert_array_equal(ei, ti.numpy())
    yf = y if dtype == "f32" else (orc.bf16_bits_to_f32(y) if dtype == "bf16" else orc.f16_bits_to_f32(y))
    tol = 1e-6 if dtype == "f32" else 1e-2
    np.testing.assert_allclose(yf, tv.to(tdt).float().numpy(), rtol=tol, atol=1e-7)
    np.testing.assert_array_equal(ri, np.arange(k)[None, :] * rows + np.arange(rows)[:, None])


def test_gating_ties_and_finished():
    E, k, rows = 16, 4, 3
    x = np.zeros((rows, E), np.float32)
    x[1, [3, 9, 12]] = 1.0  # three equal maxima, then the zeros in column order
    fin = np.array([0, 0, 1], np.uint8)
    y, ei, ri = orc.moe_gating_top_k_softmax(x, "f32", k, fin)
    np.testing.assert_array_equal(ei[0], [0, 1, 2, 3])
    np.testing.assert_allclose(y[0], 1.0 / E, rtol=1e-6)
    np.testing.assert_array_equal(ei[1], [3, 9, 12, 0])
    np.testing.assert_array_equal(ei[2], [E] * k)  # finished row
    np.testing.assert_allclose(y[2], y[0])  # values unchanged by finished


# ---------------------------------------------------------------------------------------------
# golden fixtures of the routing operators (frozen oracle outputs, regenerated only by
# tests/golden/make_golden.py); each also checked against a property the fixture must hold
# ---------------------------------------------------------------------------------------------
def _golden(name):
    import os
    p = os.path.join(os.path.dirname(__file__), "golden", name + ".npz")
    if not os.path.exists(p):
        pytest.skip(f"missing fixture {p}")
    return np.load(p, allow_pickle=False)


def test_golden_moe_gating():
    g = _golden("moe_gating")
    k = int(g["k"])
    y, ei, ri = orc.moe_gating_top_k_softmax(g["x"], "f32", k, g["finished"])
    np.testing.assert_array_equal(y, g["y"])
    np.testing.assert_array_equal(ei, g["expert_idx"])
    np.testing.assert_array_equal(ri, g["row_idx"])
    # finished rows name expert E; the all-tied row picks columns 0..k-1
    E = g["x"].shape[1]
    assert (g["expert_idx"][g["finished"] == 1] == E).all()
    if not g["finished"][3]:
        np.testing.assert_array_equal(g["expert_idx"][3], np.arange(k))


def test_golden_moe_re_routing():
    g = _golden("moe_re_routing")
    pt, ps, pi, etn, total = orc.moe_re_routing(g["tokens"], g["counts"], g["scales"])
    assert total == int(g["total"])
    for name, got in (("permute_tokens", pt), ("permute_scales", ps), ("permute_idx", pi),
                      ("expert_token_num", etn)):
        np.testing.assert_array_equal(got, g[name], err_msg=name)
    # rows move unchanged: permute_tokens[i] = tokens[permute_idx[i]]
    np.testing.assert_array_equal(g["permute_tokens"][:total], g["tokens"][g["permute_idx"][:total]])
    np.testing.assert_array_equal(g["expert_token_num"], g["counts"].sum(0))


def test_golden_moe_finalize_routing():
    g = _golden("moe_finalize_routing")
    out = orc.moe_finalize_routing(g["epr"], "bf16", g["esdr"], int(g["k"]), g["skip1"], g["skip2"], g["bias"],
                                   g["scales"], "f32", g["expert"], 0)
    np.testing.assert_array_equal(out, g["out"])


def test_golden_dequant_swiglu_quant():
    g = _golden("dequant_swiglu_quant")
    y, s = orc.dequant_swiglu_quant(g["x"], "i32", g["weight_scale"], g["activation_scale"], g["quant_scale"], False)
    np.testing.assert_array_equal(y, g["y"])
    np.testing.assert_array_equal(s, g["scale"])
    assert (np.abs(g["y"].astype(np.int32)).max(axis=1) == 127).all()  # each row reaches full scale
