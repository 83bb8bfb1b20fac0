"""Writes the golden fixtures under tests/golden/ from the CPU oracle on small seeded inputs.

The reference ships no golden vectors (NOTICE:6-7), so these fixtures freeze the oracle's outputs
(pinned independently by tests/test_oracle.py) and give the GPU tests a fixed, committed target.
Run: python tests/golden/make_golden.py
"""
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))
from oracle import oracle as orc  # noqa: E402


def bf16_bits(x):
    u = np.ascontiguousarray(x, np.float32).view(np.uint32).astype(np.uint64)
    return ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)


def main():
    rng = np.random.default_rng(2024)
    # DynamicQuant: fp16 [16, 256], 0.1% outliers x50
    x = rng.standard_normal((16, 256)).astype(np.float32)
    x.reshape(-1)[rng.choice(x.size, 4, replace=False)] *= 50
    xb = x.astype(np.float16).view(np.uint16)
    y, s = orc.dynamic_quant(xb, "f16")
    np.savez_compressed(os.path.join(HERE, "dynamic_quant.npz"), x=xb, y=y, scale=s)

    # ARDQ: bf16 [8, 1024]
    x1 = bf16_bits(rng.standard_normal((8, 1024)))
    x2 = bf16_bits(rng.standard_normal((8, 1024)))
    g = bf16_bits(rng.uniform(0.5, 1.5, 1024))
    y, xo, s = orc.ardq(x1, x2, g, "bf16", 1e-6)
    np.savez_compressed(os.path.join(HERE, "ardq.npz"), x1=x1, x2=x2, gamma=g, eps=np.float32(1e-6),
                        y=y, x_out=xo, scale=s)

    # GMSQ: E=4 (one empty group), M=23, K=128, N=64
    counts = np.array([7, 0, 12, 4])
    M, K, N = int(counts.sum()), 128, 64
    xg = rng.integers(-127, 128, (M, K), dtype=np.int8)
    w = rng.integers(-127, 128, (4, K, N), dtype=np.int8)
    ws = rng.uniform(0.001, 0.01, (4, N)).astype(np.float32)
    xs = rng.uniform(0.005, 0.02, M).astype(np.float32)
    gl = np.cumsum(counts).astype(np.int64)
    y, ys = orc.gmsq(xg, w, ws, xs, gl)
    np.savez_compressed(os.path.join(HERE, "gmsq.npz"), x=xg, w=w, ws=ws, xs=xs, group_list=gl, y=y, y_scale=ys)

    # QuantMatmul: [24, 160] x [160, 48], per-channel scale + per-token scale, bf16 out
    x1 = rng.integers(-127, 128, (24, 160), dtype=np.int8)
    x2 = rng.integers(-127, 128, (160, 48), dtype=np.int8)
    sc = rng.uniform(0.001, 0.01, 48).astype(np.float32)
    pt = rng.uniform(0.005, 0.02, 24).astype(np.float32)
    out = orc.quant_matmul(x1, x2, sc, pertoken=pt, out_dtype="bf16")
    np.savez_compressed(os.path.join(HERE, "quant_matmul.npz"), x1=x1, x2=x2, scale=sc, pertoken=pt, out=out)

    # int8 grouped down-projection: E=3, M=20, K=96, N=80
    counts = np.array([9, 0, 11])
    xd = rng.integers(-127, 128, (20, 96), dtype=np.int8)
    wd = rng.integers(-127, 128, (3, 96, 80), dtype=np.int8)
    wsd = rng.uniform(0.001, 0.01, (3, 80)).astype(np.float32)
    xsd = rng.uniform(0.005, 0.02, 20).astype(np.float32)
    gld = np.cumsum(counts).astype(np.int64)
    out = orc.grouped_matmul_quant(xd, wd, wsd, xsd, gld)
    np.savez_compressed(os.path.join(HERE, "grouped_matmul_quant.npz"), x=xd, w=wd, ws=wsd, xs=xsd,
                        group_list=gld, out=out)

    # GroupedMatmul (float): bf16 x [28, 64], w [4, 64, 48], bf16 bias, an empty group
    rg = np.random.default_rng(2025)
    counts = np.array([5, 0, 20, 3])
    gl = np.cumsum(counts).astype(np.int64)
    xg = bf16_bits(rg.standard_normal((int(gl[-1]), 64)).astype(np.float32))
    wg = bf16_bits(rg.standard_normal((4, 64, 48)).astype(np.float32))
    bg = bf16_bits(rg.standard_normal((4, 48)).astype(np.float32))
    yg = orc.grouped_matmul(xg, wg, gl, bg, dtype="bf16", bias_dtype="bf16")
    np.savez_compressed(os.path.join(HERE, "grouped_matmul.npz"), x=xg, w=wg, bias=bg, group_list=gl, y=yg)
    routing_fixtures()
    print("wrote fixtures to", HERE)


def routing_fixtures():
    """The routing operators around the experts, each on a small case with its edge conditions."""
    rr = np.random.default_rng(2026)
    # MoeGatingTopKSoftmax: fp32 [12, 64], top 4, an all-tied row and finished rows
    x = rr.standard_normal((12, 64)).astype(np.float32)
    x[3] = 0.25
    fin = (rr.random(12) < 0.25).astype(np.uint8)
    y, ei, ri = orc.moe_gating_top_k_softmax(x, "f32", 4, fin)
    np.savez_compressed(os.path.join(HERE, "moe_gating.npz"), x=x, finished=fin, k=np.int64(4), y=y,
                        expert_idx=ei, row_idx=ri)
    # MoeReRouting: bf16 tokens [A = 24, H = 40] over 3 ranks x 4 experts (empty cells), scales
    cnt = rr.integers(0, 4, (3, 4)).astype(np.int32)
    cnt[1, 2] = 0
    A = int(cnt.sum()) + 3
    tok = bf16_bits(rr.standard_normal((A, 40)).astype(np.float32))
    sc = rr.uniform(0.5, 1.5, A).astype(np.float32)
    pt, ps, pi, etn, total = orc.moe_re_routing(tok, cnt, sc)
    np.savez_compressed(os.path.join(HERE, "moe_re_routing.npz"), tokens=tok, counts=cnt, scales=sc,
                        total=np.int64(total), permute_tokens=pt, permute_scales=ps, permute_idx=pi,
                        expert_token_num=etn)
    # MoeFinalizeRouting: bf16, 6 rows x top 2, H 24, both skips, bias over 3 experts, fp32 scales,
    # a dropped slot (-1); drop_pad_mode 0 (column-major expanded_src_to_dst_row)
    R, K, H, E = 6, 2, 24, 3
    epr = bf16_bits(rr.standard_normal((R * K, H)).astype(np.float32))
    perm = rr.permutation(R * K).astype(np.int32).reshape(R, K)
    perm[2, 1] = -1
    esdr = np.ascontiguousarray(perm.T).reshape(-1)
    s1 = bf16_bits(rr.standard_normal((R, H)).astype(np.float32))
    s2 = bf16_bits(rr.standard_normal((R, H)).astype(np.float32))
    bias = bf16_bits(rr.standard_normal((E, H)).astype(np.float32))
    scl = rr.random((R, K)).astype(np.float32)
    ex = rr.integers(0, E, (R, K)).astype(np.int32)
    out = orc.moe_finalize_routing(epr, "bf16", esdr, K, s1, s2, bias, scl, "f32", ex, 0)
    np.savez_compressed(os.path.join(HERE, "moe_finalize_routing.npz"), epr=epr, esdr=esdr, skip1=s1, skip2=s2,
                        bias=bias, scales=scl, expert=ex, k=np.int64(K), out=out)
    # DequantSwigluQuant: int32 x [5, 2 x 48] with weight, activation and quant scales
    xq = rr.integers(-40000, 40000, (5, 96)).astype(np.int32)
    wsq = rr.uniform(1e-5, 1e-4, 96).astype(np.float32)
    asq = rr.uniform(0.01, 0.06, 5).astype(np.float32)
    qsq = rr.uniform(0.5, 1.5, 48).astype(np.float32)
    yq, sq = orc.dequant_swiglu_quant(xq, "i32", wsq, asq, qsq, False)
    np.savez_compressed(os.path.join(HERE, "dequant_swiglu_quant.npz"), x=xq, weight_scale=wsq,
                        activation_scale=asq, quant_scale=qsq, y=yq, scale=sq)


if __name__ == "__main__":
    main()
