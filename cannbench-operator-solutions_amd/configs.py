"""Seeded synthetic inputs for the five benchmark configurations of the W8A8 MoE-FFN path.

    dq          DynamicQuant: fp16 x [1024, 4096] ~ N(0,1), 0.1% of entries x50 (outliers)
    ardq        AddRmsNormDynamicQuant: bf16 x1, x2 [8192, 7168] ~ N(0,1), gamma ~ U(0.5, 1.5), eps 1e-6
    qmm         QuantMatmul: int8 x1 [4096, 7168], x2 [7168, 4096] ~ U{-127..127},
                scale ~ U(0.001, 0.01) [4096], pertoken ~ U(0.005, 0.02) [4096], bf16 out
    gmsq_prefill  GroupedMatmulSwigluQuant: 131072 rows, K 7168, N 4096, E 256, group counts from a
                multinomial over p_e ~ (e+1)^-1.1 (numpy default_rng(0)); x_scale ~ U(0.005, 0.02),
                weight_scale ~ U(0.001, 0.01)
    gmsq_decode GroupedMatmulSwigluQuant: 256 tokens x top-8 distinct experts chosen uniformly
                (numpy default_rng(0), one draw per token) = 2048 rows; same shapes and scales,
                followed by the int8 down-projection [2048, 2048] x [256, 2048, 7168] -> bf16.

Routing operators around the experts (a 16384-token prefill batch, top-8 of 256 experts, hidden 7168):
    gating      MoeGatingTopKSoftmax: fp32 logits [16384, 256] ~ N(0,1), k = 8
    rerouting   MoeReRouting: int8 tokens [131072, 7168] from 16 ranks x 16 local experts, counts from
                a multinomial over U(0.5, 1.5) weights (numpy default_rng(0)), fp32 per-token scales
    finalize    MoeFinalizeRouting: bf16 expert outputs [131072, 7168], a random permutation as
                expanded_src_to_dst_row (drop_pad_mode 0), fp32 scales [16384, 8], bf16 skip1 [16384, 7168]
    dqsq        DequantSwigluQuant: int32 x [131072, 4096] ~ U{-2^15..2^15}, weight_scale [4096],
                activation_scale [131072]

Every tensor is drawn on the host with numpy: one numpy.random.default_rng stream per tensor,
spawned from SeedSequence(seed) in the listed order (so the data does not depend on the torch or
ROCm version), generated in chunks of at most 256 MiB and copied to the device chunk by chunk.
Group counts come from numpy.random.default_rng(seed) directly.  `scale` < 1 shrinks the
row/column counts for quick runs while keeping the group structure.
"""
import numpy as np
import torch

E_DEFAULT = 256


def zipf_group_counts(rows, experts, a=1.1, seed=0):
    p = (np.arange(experts) + 1.0) ** (-a)
    p /= p.sum()
    return np.random.default_rng(seed).multinomial(rows, p).astype(np.int64)


def topk_group_counts(tokens, experts, k=8, seed=0):
    rng = np.random.default_rng(seed)
    ids = np.stack([rng.choice(experts, k, replace=False) for _ in range(tokens)])
    return np.bincount(ids.ravel(), minlength=experts).astype(np.int64)


def cumsum_list(counts):
    return [int(v) for v in np.cumsum(counts)]


_CHUNK = 1 << 28  # host bytes generated per step


def streams(seed, n):
    """n independent numpy generators, one per tensor, in the listed order."""
    return [np.random.default_rng(s) for s in np.random.SeedSequence(seed).spawn(n)]


def _fill(shape, device, dtype, draw):
    """A device tensor filled chunk by chunk (along the flattened order) by draw(count) -> ndarray."""
    out = torch.empty(shape, dtype=dtype, device=device)
    flat = out.view(-1)
    per = max(1, _CHUNK // out.element_size())
    for i in range(0, flat.numel(), per):
        n = min(per, flat.numel() - i)
        flat[i:i + n].copy_(torch.from_numpy(np.ascontiguousarray(draw(n))))
    return out


def rand_i8(shape, device, rng):
    """int8 uniform over -127..127."""
    return _fill(shape, device, torch.int8, lambda n: rng.integers(-127, 128, size=n, dtype=np.int8))


def rand_uniform(shape, lo, hi, device, rng, dtype=torch.float32):
    t = _fill(shape, device, torch.float32, lambda n: rng.uniform(lo, hi, size=n).astype(np.float32))
    return t.to(dtype)


def rand_normal(shape, device, rng, dtype=torch.float32):
    t = _fill(shape, device, torch.float32, lambda n: rng.standard_normal(size=n, dtype=np.float32))
    return t.to(dtype)


def make_dq(device="cuda", rows=1024, cols=4096, seed=0):
    rng = np.random.default_rng(seed)
    x = rng.standard_normal((rows, cols)).astype(np.float32)
    n_out = max(1, int(round(0.001 * x.size)))
    idx = rng.choice(x.size, n_out, replace=False)
    x.reshape(-1)[idx] *= 50.0
    return {"x": torch.from_numpy(x.astype(np.float16)).to(device)}


def make_ardq(device="cuda", rows=8192, cols=7168, seed=0, dtype=torch.bfloat16):
    r = streams(seed, 3)
    return {
        "x1": rand_normal((rows, cols), device, r[0], dtype),
        "x2": rand_normal((rows, cols), device, r[1], dtype),
        "gamma": rand_uniform((cols,), 0.5, 1.5, device, r[2], dtype),
        "epsilon": 1e-6,
    }


def make_qmm(device="cuda", M=4096, K=7168, N=4096, seed=0):
    r = streams(seed, 4)
    return {
        "x1": rand_i8((M, K), device, r[0]),
        "x2": rand_i8((K, N), device, r[1]),
        "scale": rand_uniform((N,), 0.001, 0.01, device, r[2]),
        "pertoken_scale": rand_uniform((M,), 0.005, 0.02, device, r[3]),
        "output_dtype": "bfloat16",
    }


def make_gmsq(device="cuda", counts=None, K=7168, N=4096, seed=0, extra=0):
    """GMSQ inputs; `extra` more generator streams are returned under "rngs" (the decode
    config's down-projection tensors, drawn after these)."""
    E = len(counts)
    M = int(np.sum(counts))
    r = streams(seed, 4 + extra)
    return {
        "x": rand_i8((M, K), device, r[0]),
        "weight": rand_i8((E, K, N), device, r[1]),
        "weight_scale": rand_uniform((E, N), 0.001, 0.01, device, r[2]),
        "x_scale": rand_uniform((M,), 0.005, 0.02, device, r[3]),
        "group_list": cumsum_list(counts),
        "rngs": r[4:],
    }


def make_gmsq_prefill(device="cuda", scale=1.0, seed=0):
    rows = int(131072 * scale)
    return make_gmsq(device, zipf_group_counts(rows, E_DEFAULT), seed=seed)


def make_gmsq_decode(device="cuda", seed=0, with_down=True):
    counts = topk_group_counts(256, E_DEFAULT)
    d = make_gmsq(device, counts, seed=seed, extra=2)
    if with_down:
        r = d["rngs"]
        d["down_weight"] = rand_i8((E_DEFAULT, 2048, 7168), device, r[0])
        d["down_weight_scale"] = rand_uniform((E_DEFAULT, 7168), 0.001, 0.01, device, r[1])
    return d


def make_gating(device="cuda", tokens=16384, experts=256, k=8, seed=0):
    return {"x": rand_normal((tokens, experts), device, streams(seed, 1)[0]), "k": k}


def make_rerouting(device="cuda", rows=131072, hidden=7168, ranks=16, experts=16, seed=0):
    rng = np.random.default_rng(seed)
    w = rng.uniform(0.5, 1.5, ranks * experts)
    counts = rng.multinomial(rows, w / w.sum()).reshape(ranks, experts).astype(np.int64)
    r = streams(seed, 2)
    return {"tokens": rand_i8((rows, hidden), device, r[0]),
            "counts": torch.from_numpy(counts).to(device=device, dtype=torch.int32),
            "scales": rand_uniform((rows,), 0.005, 0.02, device, r[1])}


def make_finalize(device="cuda", tokens=16384, k=8, hidden=7168, seed=0):
    r = streams(seed, 4)
    return {"epr": rand_normal((tokens * k, hidden), device, r[0], torch.bfloat16),
            "esdr": torch.from_numpy(r[1].permutation(tokens * k).astype(np.int32)).to(device),
            "scales": rand_uniform((tokens, k), 0.0, 0.25, device, r[2]),
            "skip1": rand_normal((tokens, hidden), device, r[3], torch.bfloat16)}


def make_dqsq(device="cuda", rows=131072, n2=4096, seed=0):
    r = streams(seed, 3)
    return {"x": _fill((rows, n2), device, torch.int32,
                       lambda n: r[0].integers(-(1 << 15), 1 << 15, size=n, dtype=np.int32)),
            "weight_scale": rand_uniform((n2,), 1e-4, 1e-3, device, r[1]),
            "activation_scale": rand_uniform((rows,), 0.005, 0.02, device, r[2])}
