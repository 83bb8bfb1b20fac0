"""cb_grouped_matmul_swiglu_quant_noalloc (no workspace argument, no allocation: the library's fixed
per-GPU scratch array) against cb_grouped_matmul_swiglu_quant with a caller workspace, bit for
bit, on consecutive calls that reuse the scratch (the second one smaller), for prefill-shaped and
decode-shaped groups; the fix-up path through the scratch; and the size limit's status."""
import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu

DEV = "cuda"


def _inputs(counts, K, N, seed):
    g = torch.Generator()
    g.manual_seed(seed)
    E, M = len(counts), sum(counts)
    x = torch.randint(-127, 128, (M, K), dtype=torch.int8, generator=g).to(DEV)
    w = torch.randint(-127, 128, (E, K, N), dtype=torch.int8, generator=g).to(DEV)
    ws = (torch.rand(E, N, generator=g) * 0.009 + 0.001).to(DEV)
    xs = (torch.rand(M, generator=g) * 0.015 + 0.005).to(DEV)
    return x, w, ws, xs, np.cumsum(counts).tolist()


def _noalloc(cb, x, w, ws, xs, gl):
    lib = cb._lib.load()
    M, K = x.shape
    E, _, N = w.shape
    y = torch.full((M, N // 2), 99, dtype=torch.int8, device=DEV)
    ys = torch.full((M,), -1.0, dtype=torch.float32, device=DEV)
    gla = cb._lib.int64_array(gl)
    rc = lib.cb_grouped_matmul_swiglu_quant_noalloc(x.data_ptr(), w.data_ptr(), ws.data_ptr(), xs.data_ptr(), gla,
                                                    len(gl), M, K, N, E, y.data_ptr(), ys.data_ptr(),
                                                    torch.cuda.current_stream().cuda_stream)
    assert rc == 0, cb._lib.status_string(rc)
    return y, ys


@pytest.mark.parametrize("first,second", [
    # prefill-shaped then a smaller prefill-shaped call
    (([700, 0, 1300, 90, 2000, 300], 512, 4096), ([260, 0, 300], 512, 4096)),
    # decode-shaped (at most 32 rows per expert) then a smaller one
    (([5, 0, 17, 32, 1, 9] * 8, 448, 4096), ([3, 31, 0, 12], 448, 4096)),
])
def test_noalloc_matches_workspace_entry(cb, first, second):
    for counts, K, N in (first, second):
        x, w, ws, xs, gl = _inputs(counts, K, N, sum(counts) + K)
        y0, ys0 = cb.grouped_matmul_swiglu_quant(x, w, ws, xs, gl)
        y1, ys1 = _noalloc(cb, x, w, ws, xs, gl)
        torch.cuda.synchronize()
        assert torch.equal(y0, y1), counts
        assert torch.equal(ys0, ys1), counts


def test_noalloc_fixup_path(cb, overrides):
    """Every exchange wait gives up at once (test hook), so the fix-up launches recompute every tile
    from the marks and row maxima held in the scratch array: the outputs still equal the workspace
    entry point's normal run, for prefill- and decode-shaped groups."""
    for counts, K, N in (([700, 0, 1300, 90], 512, 4096), ([5, 0, 17, 32, 1, 9] * 8, 448, 4096)):
        x, w, ws, xs, gl = _inputs(counts, K, N, 7 * sum(counts) + K)
        y0, ys0 = cb.grouped_matmul_swiglu_quant(x, w, ws, xs, gl)
        torch.cuda.synchronize()
        overrides(exchange_spin_limit=-1)
        y1, ys1 = _noalloc(cb, x, w, ws, xs, gl)
        torch.cuda.synchronize()
        overrides()
        assert torch.equal(y0, y1), counts
        assert torch.equal(ys0, ys1), counts


def test_noalloc_size_limit(cb):
    lib = cb._lib.load()
    M, K, N, E = 1 << 20, 512, 4096, 1
    gla = cb._lib.int64_array([M])
    # rejected before any pointer is touched or any launch is made
    rc = lib.cb_grouped_matmul_swiglu_quant_noalloc(1, 1, 1, 1, gla, 1, M, K, N, E, 1, 1, None)
    assert rc == cb._lib.CB_ERR_SCRATCH_LIMIT
    assert "scratch" in cb._lib.status_string(rc)
