"""HIP graph capture of the operator chain (AddRmsNormDynamicQuant -> GroupedMatmulSwigluQuant ->
int8 down-projection, and QuantMatmul).

The library launches only kernels on the caller's stream, and clears the GroupedMatmulSwigluQuant
exchange state with a fill kernel rather than a memset, so a captured call sequence can be replayed.
Each replay here follows eager work on new inputs written in place into the captured buffers, and
must equal the eager call on the same inputs bit for bit (the fused kernels' exchange state is
cleared by every replay, not only by the capture).
"""
import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu

DEV = "cuda"


def cpu_gen(seed):
    g = torch.Generator()
    g.manual_seed(seed)
    return g


def rand_i8(shape, g):
    return torch.randint(-127, 128, shape, dtype=torch.int8, generator=g)


@pytest.mark.parametrize("counts,K,N", [
    ([300, 0, 700, 45, 1000], 512, 4096),   # fused prefill kernel + fix-up
    ([5, 0, 17, 32, 1, 9] * 8, 448, 4096),  # fused decode kernel + fix-up
])
def test_gmsq_graph_replays_match_eager(cb, counts, K, N):
    g = cpu_gen(sum(counts) + K)
    E, M = len(counts), sum(counts)
    x = rand_i8((M, K), g).to(DEV)
    w = rand_i8((E, K, N), g).to(DEV)
    ws = (torch.rand(E, N, generator=g) * 0.009 + 0.001).to(DEV)
    xs = (torch.rand(M, generator=g) * 0.015 + 0.005).to(DEV)
    gl = np.cumsum(counts).tolist()
    cb.grouped_matmul_swiglu_quant(x, w, ws, xs, gl)  # warm-up outside the capture
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        y_g, ys_g = cb.grouped_matmul_swiglu_quant(x, w, ws, xs, gl)
    torch.cuda.synchronize()
    for i in range(4):
        x.copy_(rand_i8((M, K), g).to(DEV))
        xs.copy_((torch.rand(M, generator=g) * 0.015 + 0.005).to(DEV))
        y_e, ys_e = cb.grouped_matmul_swiglu_quant(x, w, ws, xs, gl)
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(y_g, y_e), f"replay {i}: y"
        assert torch.equal(ys_g, ys_e), f"replay {i}: y_scale"


def test_ffn_chain_graph_replays_match_eager(cb):
    """The MoE-FFN step of one layer, captured whole: norm + quant, gate/up with SwiGLU and requant,
    down-projection; replayed on new hidden states."""
    g = cpu_gen(7)
    counts = [40, 0, 300, 7, 129]
    E, M, H, F = len(counts), sum(counts), 1024, 2048  # hidden, gate + up width
    gl = np.cumsum(counts).tolist()
    bf = lambda t: t.to(torch.bfloat16).to(DEV)
    x1, x2 = bf(torch.randn(M, H, generator=g)), bf(torch.randn(M, H, generator=g))
    gamma = bf(torch.rand(H, generator=g) + 0.5)
    w1 = rand_i8((E, H, F), g).to(DEV)
    ws1 = (torch.rand(E, F, generator=g) * 0.009 + 0.001).to(DEV)
    w2 = rand_i8((E, F // 2, H), g).to(DEV)
    ws2 = (torch.rand(E, H, generator=g) * 0.009 + 0.001).to(DEV)

    def step():
        y, _, s = cb.add_rms_norm_dynamic_quant(x1, x2, gamma, 1e-6)
        h, hs = cb.grouped_matmul_swiglu_quant(y, w1, ws1, s, gl)
        return cb.grouped_matmul_quant(h, w2, ws2, hs, gl)

    step()
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        out_g = step()
    torch.cuda.synchronize()
    for i in range(3):
        x1.copy_(bf(torch.randn(M, H, generator=g)))
        out_e = step()
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out_g, out_e), f"replay {i}"


def test_quant_matmul_graph_replays_match_eager(cb):
    g = cpu_gen(11)
    M, K, N = 1024, 2048, 2048
    x1 = rand_i8((M, K), g).to(DEV)
    x2 = rand_i8((K, N), g).to(DEV)
    sc = (torch.rand(N, generator=g) * 0.009 + 0.001).to(DEV)
    pt = (torch.rand(M, generator=g) * 0.015 + 0.005).to(DEV)
    f = lambda: cb.quant_matmul(x1, x2, sc, pertoken_scale=pt, output_dtype="bfloat16")
    f()
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        out_g = f()
    torch.cuda.synchronize()
    for i in range(3):
        x1.copy_(rand_i8((M, K), g).to(DEV))
        out_e = f()
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out_g, out_e), f"replay {i}"
