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
    print("wrote fixtures to", HERE)


if __name__ == "__main__":
    main()
