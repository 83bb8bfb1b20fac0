"""GPU parity of the routing operators (MoeReRouting, MoeFinalizeRouting, DequantSwigluQuant,
MoeGatingTopKSoftmax) against the CPU oracle on identical seeded inputs.

Bars: permutations, indices, counts and the expert choice bit-exact; MoeFinalizeRouting bit-exact
(same fp32 operation order, no FMA contraction, round-half-even store); DequantSwigluQuant int8 within
+-1 LSB on at most 1% of elements and scales within 1e-5 relative (exp ulps differ between the CPU
and GPU math libraries); MoeGatingTopKSoftmax values within 1e-5 relative for fp32 rows (the row sum
is reduced in a different order) and within one 16-bit ulp for bf16 / fp16 rows.
"""
import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu

DEV = "cuda"


def gen(seed):
    g = torch.Generator()
    g.manual_seed(seed)
    return g


def bits16(t):
    return t.contiguous().cpu().view(torch.int16).numpy().view(np.uint16)


def host(t, dt):
    """numpy view of a tensor in the oracle's encoding (uint16 bits for 16-bit floats)."""
    return t.cpu().numpy() if dt in ("f32", "i32", "i8") else bits16(t)


TD = {"bf16": torch.bfloat16, "f16": torch.float16, "f32": torch.float32, "i8": torch.int8, "i32": torch.int32}


# ---------------------------------------------------------------------------------------------
# MoeReRouting
# ---------------------------------------------------------------------------------------------
@pytest.mark.parametrize("tok_dt", ["bf16", "f16", "i8"])
@pytest.mark.parametrize("cnt_dt", [torch.int32, torch.int64])
@pytest.mark.parametrize("n,e,H,cmax,scales", [
    (4, 8, 128, 6, True),       # 16-byte rows
    (16, 16, 7168, 40, True),   # EP-16 shape, wide rows
    (3, 5, 33, 4, False),       # ragged rows (not a multiple of 16 bytes), no scales
    (1, 1, 16, 9, True),        # one rank, one expert
    (8, 32, 64, 2, False),      # many empty cells
])
def test_moe_re_routing(cb, orc, tok_dt, cnt_dt, n, e, H, cmax, scales):
    g = gen(n * 1000 + e * 10 + H)
    cnt = torch.randint(0, cmax + 1, (n, e), generator=g)
    cnt[0, 0] = 0
    total = int(cnt.sum())
    A = total + 5  # rows past the routed total stay unwritten
    if tok_dt == "i8":
        tokens = torch.randint(-128, 128, (A, H), dtype=torch.int8, generator=g)
    else:
        tokens = torch.randn(A, H, generator=g).to(TD[tok_dt])
    sc = torch.rand(A, generator=g) if scales else None
    pt, ps, pi, etn = cb.moe_re_routing(tokens.to(DEV), cnt.to(cnt_dt).to(DEV), None if sc is None else sc.to(DEV))
    torch.cuda.synchronize()
    assert pt.dtype == tokens.dtype and ps.dtype == torch.float32 and pi.dtype == torch.int32
    assert etn.dtype == cnt_dt and etn.shape == (e,)
    r_out, r_sc, r_idx, r_etn, r_total = orc.moe_re_routing(host(tokens, tok_dt), cnt.numpy(),
                                                            None if sc is None else sc.numpy())
    assert r_total == total
    np.testing.assert_array_equal(etn.cpu().numpy(), r_etn)
    np.testing.assert_array_equal(pi.cpu().numpy()[:total], r_idx[:total])
    np.testing.assert_array_equal(host(pt, tok_dt)[:total], r_out[:total])
    np.testing.assert_array_equal(ps.cpu().numpy()[:total], r_sc[:total])


def test_moe_re_routing_empty_and_checks(cb):
    tok = torch.zeros(0, 8, dtype=torch.bfloat16, device=DEV)
    outs = cb.moe_re_routing(tok, torch.zeros(2, 3, dtype=torch.int32, device=DEV))
    assert outs[0].shape == (0, 8) and outs[3].shape == (3,)
    with pytest.raises(RuntimeError, match="idx_type == 0"):
        cb.moe_re_routing(tok, torch.zeros(2, 3, dtype=torch.int32, device=DEV), idx_type=1)
    with pytest.raises(RuntimeError, match="unsupported tokens dtype"):
        cb.moe_re_routing(torch.zeros(4, 8, dtype=torch.float32, device=DEV),
                          torch.ones(2, 2, dtype=torch.int32, device=DEV))


# ---------------------------------------------------------------------------------------------
# MoeFinalizeRouting
# ---------------------------------------------------------------------------------------------
@pytest.mark.parametrize("dt", ["bf16", "f16", "f32"])
@pytest.mark.parametrize("sdt", ["f32", "same"])
@pytest.mark.parametrize("mode", [0, 2])
@pytest.mark.parametrize("R,K,H,extras", [
    (64, 8, 7168, True),    # DeepSeek-style: top-8, hidden 7168, skips + bias
    (37, 4, 40, True),      # small ragged H
    (5, 1, 16, False),      # K = 1, gather only (scales still given)
])
def test_moe_finalize_routing(cb, orc, dt, sdt, mode, R, K, H, extras):
    sdt = dt if sdt == "same" else sdt
    g = gen(R * 31 + K * 7 + H + mode)
    num_dst = R * K
    tdt = TD[dt]
    epr = torch.randn(num_dst, H, generator=g).to(tdt)
    perm = torch.randperm(num_dst, generator=g).to(torch.int32).reshape(R, K)
    if R > 5:
        perm[3, 0] = -1           # dropped (padded) slot
        perm[4, K - 1] = num_dst  # out of range: dropped too
    esdr = perm.t().contiguous().reshape(-1) if mode <= 1 else perm.reshape(-1)
    scales = torch.rand(R, K, generator=g).to(TD[sdt])
    E = 6
    skip1 = torch.randn(R, H, generator=g).to(tdt) if extras else None
    skip2 = torch.randn(R, H, generator=g).to(tdt) if extras else None
    bias = torch.randn(E, H, generator=g).to(tdt) if extras else None
    expert = torch.randint(-1, E + 1, (R, K), generator=g).to(torch.int32) if extras else None
    d = (lambda t: None if t is None else t.to(DEV))
    out = cb.moe_finalize_routing(d(epr), d(esdr), d(skip1), d(skip2), d(bias), d(scales), d(expert), mode)
    torch.cuda.synchronize()
    assert out.shape == (R, H) and out.dtype == tdt
    h = (lambda t, x=dt: None if t is None else host(t, x))
    want = orc.moe_finalize_routing(h(epr), dt, esdr.numpy(), K, h(skip1), h(skip2), h(bias), h(scales, sdt), sdt,
                                    None if expert is None else expert.numpy(), mode)
    np.testing.assert_array_equal(host(out, dt), want)


def test_moe_finalize_routing_no_scales(cb, orc):
    g = gen(5)
    epr = torch.randn(12, 256, generator=g).to(torch.bfloat16)
    esdr = torch.tensor([11, 0, 3, 3, 7], dtype=torch.int32)
    skip = torch.randn(5, 256, generator=g).to(torch.bfloat16)
    out = cb.moe_finalize_routing(epr.to(DEV), esdr.to(DEV), skip.to(DEV))
    want = orc.moe_finalize_routing(bits16(epr), "bf16", esdr.numpy(), 1, bits16(skip))
    np.testing.assert_array_equal(bits16(out), want)


# ---------------------------------------------------------------------------------------------
# DequantSwigluQuant
# ---------------------------------------------------------------------------------------------
def _assert_i8(got, ref, label):
    d = np.abs(got.astype(np.int32) - ref.astype(np.int32))
    assert d.max() <= 1, f"{label}: int8 diff {d.max()}"
    assert (d > 0).mean() <= 0.01, f"{label}: {(d > 0).mean():.4%} differ by 1 LSB"


@pytest.mark.parametrize("xdt", ["i32", "bf16", "f16"])
@pytest.mark.parametrize("qs", [False, True])
@pytest.mark.parametrize("left", [False, True])
@pytest.mark.parametrize("M,H", [(256, 2048), (7, 4096), (3, 12000), (1, 1), (33, 100)])
def test_dequant_swiglu_quant(cb, orc, xdt, qs, left, M, H):
    g = gen(M * 13 + H + int(qs) * 3 + int(left))
    if xdt == "i32":
        x = torch.randint(-40000, 40000, (M, 2 * H), dtype=torch.int32, generator=g)
        ws = (torch.rand(2 * H, generator=g) * 1e-4 + 1e-5)
        asc = torch.rand(M, generator=g) * 0.05 + 0.01
    else:
        x = (torch.randn(M, 2 * H, generator=g) * 2).to(TD[xdt])
        ws = asc = None
    q = (torch.rand(H, generator=g) + 0.5) if qs else None
    d = (lambda t: None if t is None else t.to(DEV))
    y, s = cb.dequant_swiglu_quant(d(x), d(ws), d(asc), d(q), left)
    torch.cuda.synchronize()
    ry, rs = orc.dequant_swiglu_quant(host(x, xdt), xdt, None if ws is None else ws.numpy(),
                                      None if asc is None else asc.numpy(), None if q is None else q.numpy(), left)
    np.testing.assert_allclose(s.cpu().numpy(), rs, rtol=1e-5)
    _assert_i8(y.cpu().numpy(), ry, f"dqsq {xdt} M={M} H={H}")


def test_dequant_swiglu_quant_zero_rows_and_checks(cb):
    x = torch.zeros(3, 64, dtype=torch.bfloat16, device=DEV)
    y, s = cb.dequant_swiglu_quant(x)
    torch.cuda.synchronize()
    assert (y == 0).all() and (s.cpu() == torch.tensor(1e-12, dtype=torch.float32)).all()
    with pytest.raises(RuntimeError, match="weight_scale is required"):
        cb.dequant_swiglu_quant(torch.zeros(2, 8, dtype=torch.int32, device=DEV))
    with pytest.raises(RuntimeError, match="even last dimension"):
        cb.dequant_swiglu_quant(torch.zeros(2, 7, dtype=torch.bfloat16, device=DEV))


# ---------------------------------------------------------------------------------------------
# MoeGatingTopKSoftmax
# ---------------------------------------------------------------------------------------------
@pytest.mark.parametrize("dt", ["f32", "bf16", "f16"])
@pytest.mark.parametrize("rows,E,k", [(4096, 256, 8), (2000, 256, 1), (1000, 64, 6), (77, 8, 2), (500, 256, 2), (33, 2048, 16),
                                      (9, 130, 130), (20, 300, 100), (5, 1, 1), (16, 16, 16)])
@pytest.mark.parametrize("fin", [False, True])
def test_moe_gating_top_k_softmax(cb, orc, dt, rows, E, k, fin):
    g = gen(rows + E * 3 + k)
    x = torch.randn(rows, E, generator=g).to(TD[dt])
    if rows > 3:
        x[2] = 0.5  # an all-tied row
    finished = (torch.rand(rows, generator=g) < 0.3) if fin else None
    y, ei, ri = cb.moe_gating_top_k_softmax(x.to(DEV), None if finished is None else finished.to(DEV), k)
    torch.cuda.synchronize()
    ry, rei, rri = orc.moe_gating_top_k_softmax(host(x, dt), dt, k,
                                                None if finished is None else finished.numpy().astype(np.uint8))
    np.testing.assert_array_equal(ei.cpu().numpy(), rei)
    np.testing.assert_array_equal(ri.cpu().numpy(), rri)
    if dt == "f32":
        np.testing.assert_allclose(y.cpu().numpy(), ry, rtol=1e-5, atol=1e-9)
    else:
        got = y.cpu().float().numpy()
        ref = torch.from_numpy(ry.view(np.int16)).view(TD[dt]).float().numpy()
        np.testing.assert_allclose(got, ref, rtol=1e-2, atol=1e-6)


@pytest.mark.parametrize("dt", ["f32", "bf16"])
@pytest.mark.parametrize("E,k,span", [(256, 8, 16), (256, 12, 16), (256, 16, 32), (2048, 24, 32), (130, 40, 9)])
def test_moe_gating_one_lane_holds_the_top(cb, orc, dt, E, k, span):
    """The k largest values of a row lie in `span` consecutive columns, i.e. one or two lanes'
    slots, so those lanes win many rounds in a row and refill their candidate lists from the
    columns after the last one they emitted; bf16 rounding adds ties among them."""
    g = gen(E + k + span)
    rows = 300
    x = torch.randn(rows, E, generator=g)
    start = torch.randint(0, E - span + 1, (rows,), generator=g)
    for r in range(rows):
        x[r, start[r]:start[r] + span] += 6.0
    x = x.to(TD[dt])
    y, ei, ri = cb.moe_gating_top_k_softmax(x.to(DEV), None, k)
    torch.cuda.synchronize()
    ry, rei, rri = orc.moe_gating_top_k_softmax(host(x, dt), dt, k, None)
    np.testing.assert_array_equal(ei.cpu().numpy(), rei)
    np.testing.assert_array_equal(ri.cpu().numpy(), rri)
    if dt == "f32":
        np.testing.assert_allclose(y.cpu().numpy(), ry, rtol=1e-5, atol=1e-9)
    else:
        ref = torch.from_numpy(ry.view(np.int16)).view(TD[dt]).float().numpy()
        np.testing.assert_allclose(y.cpu().float().numpy(), ref, rtol=1e-2, atol=1e-6)


def test_moe_gating_batched_shape(cb):
    x = torch.randn(2, 3, 16, device=DEV)
    y, ei, ri = cb.moe_gating_top_k_softmax(x, None, 4)
    assert y.shape == (2, 3, 4) and ei.shape == (2, 3, 4) and ri.shape == (2, 3, 4)
    ref = torch.topk(torch.softmax(x.float(), -1), 4, -1)
    torch.testing.assert_close(y, ref.values, rtol=1e-5, atol=1e-7)


def test_routing_torch_ops(cb):
    cb.register_torch_ops()
    x = torch.randn(8, 32, device=DEV)
    y, ei, ri = torch.ops.cann_bench.moe_gating_top_k_softmax(x, None, 2)
    assert ei.dtype == torch.int32
    h = torch.randn(4, 64, device=DEV).to(torch.bfloat16)
    yq, s = torch.ops.cann_bench.dequant_swiglu_quant(h)
    assert yq.shape == (4, 32) and s.shape == (4,)
    tok = torch.randn(6, 16, device=DEV).to(torch.bfloat16)
    outs = torch.ops.cann_bench.moe_re_routing(tok, torch.tensor([[1, 2], [2, 1]], dtype=torch.int32, device=DEV))
    assert outs[2].cpu().tolist() == [0, 3, 4, 1, 2, 5]
    out = torch.ops.cann_bench.moe_finalize_routing(tok, torch.arange(6, dtype=torch.int32, device=DEV))
    torch.testing.assert_close(out, tok, rtol=0, atol=0)


@pytest.mark.parametrize("case", ["odd_h", "big_k", "misaligned"])
def test_moe_finalize_routing_scalar_paths(cb, orc, case):
    """Shapes off the 16-byte vector path: odd H, K above the LDS slot table, and rows that are
    not 16-byte aligned (a view one element into a larger buffer)."""
    g = gen({"odd_h": 1, "big_k": 2, "misaligned": 3}[case])
    R, K, H = (9, 3, 37) if case == "odd_h" else ((6, 80, 64) if case == "big_k" else (7, 4, 64))
    num_dst = R * K
    base = torch.randn(num_dst * H + 1, generator=g).to(torch.bfloat16)
    epr = base[1:].reshape(num_dst, H) if case == "misaligned" else base[:num_dst * H].reshape(num_dst, H)
    esdr = torch.randperm(num_dst, generator=g).to(torch.int32)
    esdr[0] = -1
    scales = torch.rand(R, K, generator=g)
    skip = torch.randn(R, H, generator=g).to(torch.bfloat16)
    bias = torch.randn(5, H, generator=g).to(torch.bfloat16)
    expert = torch.randint(0, 5, (R, K), generator=g).to(torch.int32)
    dev_base = base.to(DEV)
    depr = dev_base[1:].reshape(num_dst, H) if case == "misaligned" else dev_base[:num_dst * H].reshape(num_dst, H)
    out = cb.moe_finalize_routing(depr, esdr.to(DEV), skip.to(DEV), None, bias.to(DEV), scales.to(DEV),
                                  expert.to(DEV), 2)
    torch.cuda.synchronize()
    want = orc.moe_finalize_routing(bits16(epr), "bf16", esdr.numpy(), K, bits16(skip), None, bits16(bias),
                                    scales.numpy(), "f32", expert.numpy(), 2)
    np.testing.assert_array_equal(bits16(out), want)


def test_moe_re_routing_large_cell_table(cb, orc):
    """More than 8192 (rank, expert) cells: the serial prefix kernel."""
    g = gen(11)
    n, e, H = 40, 256, 32
    cnt = torch.randint(0, 2, (n, e), generator=g)
    total = int(cnt.sum())
    tokens = torch.randn(total, H, generator=g).to(torch.bfloat16)
    pt, ps, pi, etn = cb.moe_re_routing(tokens.to(DEV), cnt.to(torch.int64).to(DEV))
    torch.cuda.synchronize()
    r_out, _, r_idx, r_etn, _ = orc.moe_re_routing(bits16(tokens), cnt.numpy())
    np.testing.assert_array_equal(etn.cpu().numpy(), r_etn)
    np.testing.assert_array_equal(pi.cpu().numpy(), r_idx)
    np.testing.assert_array_equal(bits16(pt), r_out)


# ---------------------------------------------------------------------------------------------
# committed golden fixtures of the routing operators
# ---------------------------------------------------------------------------------------------
def _golden(name):
    import os
    return np.load(os.path.join(os.path.dirname(__file__), "golden", name + ".npz"), allow_pickle=False)


def _bf16_dev(bits):
    return torch.from_numpy(bits.view(np.int16)).view(torch.bfloat16).to(DEV)


def test_golden_routing_fixtures(cb):
    g = _golden("moe_gating")
    y, ei, ri = cb.moe_gating_top_k_softmax(torch.from_numpy(g["x"]).to(DEV),
                                            torch.from_numpy(g["finished"].astype(bool)).to(DEV), int(g["k"]))
    np.testing.assert_array_equal(ei.cpu().numpy(), g["expert_idx"])
    np.testing.assert_array_equal(ri.cpu().numpy(), g["row_idx"])
    np.testing.assert_allclose(y.cpu().numpy(), g["y"], rtol=1e-5, atol=1e-9)

    g = _golden("moe_re_routing")
    total = int(g["total"])
    pt, ps, pi, etn = cb.moe_re_routing(_bf16_dev(g["tokens"]), torch.from_numpy(g["counts"]).to(DEV),
                                        torch.from_numpy(g["scales"]).to(DEV))
    np.testing.assert_array_equal(bits16(pt)[:total], g["permute_tokens"][:total])
    np.testing.assert_array_equal(ps.cpu().numpy()[:total], g["permute_scales"][:total])
    np.testing.assert_array_equal(pi.cpu().numpy()[:total], g["permute_idx"][:total])
    np.testing.assert_array_equal(etn.cpu().numpy(), g["expert_token_num"])

    g = _golden("moe_finalize_routing")
    out = cb.moe_finalize_routing(_bf16_dev(g["epr"]), torch.from_numpy(g["esdr"]).to(DEV), _bf16_dev(g["skip1"]),
                                  _bf16_dev(g["skip2"]), _bf16_dev(g["bias"]), torch.from_numpy(g["scales"]).to(DEV),
                                  torch.from_numpy(g["expert"]).to(DEV), 0)
    np.testing.assert_array_equal(bits16(out), g["out"])

    g = _golden("dequant_swiglu_quant")
    y, s = cb.dequant_swiglu_quant(torch.from_numpy(g["x"]).to(DEV), torch.from_numpy(g["weight_scale"]).to(DEV),
                                   torch.from_numpy(g["activation_scale"]).to(DEV),
                                   torch.from_numpy(g["quant_scale"]).to(DEV), False)
    _assert_i8(y.cpu().numpy(), g["y"], "dequant_swiglu_quant fixture")
    np.testing.assert_allclose(s.cpu().numpy(), g["scale"], rtol=1e-5)
