"""Benchmark of the W8A8 MoE-FFN hot path on one MI355X.

Headline (`value`): GroupedMatmulSwigluQuant on the prefill configuration (131072 int8 rows,
256 experts, K 7168, N 4096, Zipf(1.1) routing), in TOPS = 2*M*K*N / device time of the whole op
(all of its kernels), inputs resident in HBM.  The same JSON line also carries the decode
configuration (GB/s of algorithmic bytes), its down-projection, AddRmsNormDynamicQuant, the
dense QuantMatmul and the routing operators (gating, re-routing, finalize, DequantSwigluQuant),
each with its own roofline figure, plus CPU baselines (the C oracle on bounded samples of the
prefill and decode experts, on the host cores).  Every time is the median over the timed calls of
HIP events around each call; configs 2 and 3 (whose inputs would fit the 256 MB MALL) are preceded
by a 512 MB flush (a write, then a read) outside the events.

A step is one operator call over one batch of synthetic input.  Usage:
    python bench.py [--gpus 1] [--steps K] [--warmup W] [--only prefill,decode,...] [--no-cpu]
    python bench.py --power prefill,decode,... [--seconds S] [--lib variant.so]   (power / clock samples)
"""
import argparse
import importlib
import json
import os
import sys
import time

import numpy as np
import torch

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)
cb = importlib.import_module("cannbench-operator-solutions_amd")
cfgs = importlib.import_module("cannbench-operator-solutions_amd.configs")
L = importlib.import_module("cannbench-operator-solutions_amd._lib")

METRIC = "GroupedMatmulSwigluQuant int8 TOPS (%MFMA peak) + decode HBM GB/s (%peak), 1 GPU"
PEAK_INT8_TOPS = 5000.0      # MI355X dense int8 MFMA, published
PEAK_HBM_GBS = 8000.0        # MI355X HBM3E, published
PEAK_BF16_TFLOPS = 2500.0    # MI355X dense bf16 / fp16 MFMA, published


class KernelTimer:
    """HIP events around the main GEMM kernel of the next call (cb_set_kernel_timing), recorded on
    the stream the kernel is launched on."""

    def __init__(self, n):
        self.pairs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(n)]
        for a, b in self.pairs:  # materialise the underlying hipEvent_t handles
            a.record()
            b.record()
        torch.cuda.synchronize()
        self.i = 0

    def arm(self):
        a, b = self.pairs[self.i]
        self.i += 1
        L.load().cb_set_kernel_timing(a.cuda_event, b.cuda_event)

    def median_ms(self):
        ts = [a.elapsed_time(b) for a, b in self.pairs[: self.i]]
        return float(np.median(ts)) if ts else None


FLUSH_BYTES = 512 << 20  # twice the 256 MB MALL: a write of it evicts every cache level


class Flush:
    """A 512 MB device write, then a read of the same buffer, issued before a timed call and outside
    its events, so that the call's inputs come from HBM rather than the 256 MB MALL or the L2s
    (the inputs of configs 2 and 3 would fit the MALL).  The read leaves the caches holding clean lines, so the timed
    call does not also pay for writing back the flush's dirty ones."""

    def __init__(self, dev):
        self.buf = torch.empty(FLUSH_BYTES // 4, dtype=torch.int32, device=dev)
        self.sink = torch.empty((), dtype=torch.int64, device=dev)
        self.k = 0

    def __call__(self):
        self.k += 1
        self.buf.fill_(self.k)
        torch.sum(self.buf, dim=0, dtype=torch.int64, out=self.sink)


def time_op(fn, steps, warmup, timer=None, flush=None):
    """Per-call device time of `fn` (HIP events on the current stream, which the operators enqueue
    on), median over `steps` calls after `warmup` untimed ones.  `flush`, when given, runs before
    every call, outside the events.  Returns (median ms, mean wall ms per call of the timed loop)."""
    for _ in range(warmup):
        if flush is not None:
            flush()
        fn()
    ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(steps)]
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for a, b in ev:
        if flush is not None:
            flush()
        if timer is not None:
            timer.arm()
        a.record()
        fn()
        b.record()
    torch.cuda.synchronize()
    wall = (time.perf_counter() - t0) * 1e3 / steps
    return float(np.median([a.elapsed_time(b) for a, b in ev])), wall


def roofline(bound, achieved, unit, traffic=None, peak=None):
    if peak is None:
        peak = PEAK_INT8_TOPS if bound == "mfma" else PEAK_HBM_GBS
    return {"bound": bound, "achieved": round(achieved, 2), "peak": peak, "unit": unit,
            "frac": round(achieved / peak, 4), "traffic": traffic}


# ------------------------------------------------------------------------------------------------
def bench_prefill(steps, warmup, dev, keep):
    d = cfgs.make_gmsq_prefill(dev)
    M, K = d["x"].shape
    N = d["weight"].shape[2]
    ops = 2.0 * M * K * N
    fn = lambda: cb.grouped_matmul_swiglu_quant(d["x"], d["weight"], d["weight_scale"], d["x_scale"], d["group_list"])
    timer = KernelTimer(steps)
    ms, wall = time_op(fn, steps, warmup, timer)
    kms = timer.median_ms()
    counts = np.diff([0] + d["group_list"])
    res = {"ms": ms, "wall_ms": wall, "tops": ops / (ms * 1e-3) / 1e12, "gemm_kernel_ms": kms,
           "roofline": roofline("mfma", ops / (kms * 1e-3) / 1e12, "TFLOP/s"),
           "config": {"workload": "gmsq_prefill", "rows": M, "experts": len(counts), "K": K, "N": N,
                      "routing": "zipf(1.1) multinomial, numpy seed 0",
                      "rows_per_expert_max": int(counts.max()), "rows_per_expert_min": int(counts.min())}}
    keep["prefill"] = d
    return res


def bench_prefill_gather(steps, warmup, dev, keep):
    """GroupedMatmulSwigluQuant with gathered rows on the MoE prefill flow: 16384 tokens x 7168 (the
    first rows of the prefill activations), 131072 routed rows over the prefill config's Zipf expert
    counts, each routed row naming a seeded-random source token (about 8 routed rows per token).
    Against the unfused sequence: an explicit gather (torch index_select) of the 131072 rows and their
    scales, then the plain operator."""
    d = keep["prefill"]
    T = 16384
    x_tok, xs_tok = d["x"][:T], d["x_scale"][:T]
    M, K = d["x"].shape
    N = d["weight"].shape[2]
    idx = torch.from_numpy(np.random.default_rng(21).integers(0, T, M, dtype=np.int32)).to(dev)
    # a stable sort of the (token, slot) pairs by expert leaves each expert's token ids ascending
    bounds = [0] + list(d["group_list"])
    idx = torch.cat([idx[s:e].sort().values for s, e in zip(bounds[:-1], bounds[1:])])
    ops = 2.0 * M * K * N
    fused = lambda: cb.grouped_matmul_swiglu_quant_gather(x_tok, idx, d["weight"], d["weight_scale"], xs_tok,
                                                          d["group_list"])
    timer = KernelTimer(steps)
    ms, _ = time_op(fused, steps, warmup, timer)
    kms = timer.median_ms()
    il = idx.long()
    unfused = lambda: cb.grouped_matmul_swiglu_quant(x_tok.index_select(0, il), d["weight"], d["weight_scale"],
                                                     xs_tok.index_select(0, il), d["group_list"])
    ms_u, _ = time_op(unfused, steps, warmup)
    return {"value": round(ops / (ms * 1e-3) / 1e12, 2), "unit": "TOPS", "ms_per_step": round(ms, 4),
            "gemm_kernel_ms": round(kms, 4), "roofline": roofline("mfma", ops / (kms * 1e-3) / 1e12, "TFLOP/s"),
            "unfused_ms_per_step": round(ms_u, 4), "saving_ms": round(ms_u - ms, 4),
            "config": {"workload": "gmsq_prefill_gather", "tokens": T, "rows": M, "experts": len(d["group_list"]),
                       "K": K, "N": N, "row_index": "uniform random source token per routed row (numpy seed 21), ascending within each expert"}}


def bench_down_prefill(steps, warmup, dev, keep):
    """The int8 grouped down-projection at the prefill size (context, not a BASELINE config): the GMSQ
    prefill output shape x int8 [131072, 2048] (seeded random) over the prefill Zipf routing, weights
    int8 [256, 2048, 7168], bf16 out [131072, 7168]."""
    d = keep["prefill"]
    M = d["x"].shape[0]
    r = cfgs.streams(41, 4)
    x = cfgs.rand_i8((M, 2048), dev, r[0])
    xs = cfgs.rand_uniform((M,), 0.005, 0.02, dev, r[1])
    w = cfgs.rand_i8((256, 2048, 7168), dev, r[2])
    ws = cfgs.rand_uniform((256, 7168), 0.001, 0.01, dev, r[3])
    ops = 2.0 * M * 2048 * 7168
    fn = lambda: cb.grouped_matmul_quant(x, w, ws, xs, d["group_list"])
    timer = KernelTimer(steps)
    ms, _ = time_op(fn, steps, warmup, timer)
    kms = timer.median_ms()
    del x, w
    return {"value": round(ops / (ms * 1e-3) / 1e12, 2), "unit": "TOPS", "ms_per_step": round(ms, 4),
            "gemm_kernel_ms": round(kms, 4), "roofline": roofline("mfma", ops / (kms * 1e-3) / 1e12, "TFLOP/s"),
            "config": {"workload": "down_proj_prefill", "rows": M, "K": 2048, "N": 7168, "experts": 256,
                       "routing": "prefill zipf(1.1)"}}


def decode_bytes(counts, K, N):
    M = int(np.sum(counts))
    act = int(np.sum(np.asarray(counts) > 0))
    return act * K * N + M * K + M * (N // 2) + 8 * M + 4 * N * act


def bench_decode(steps, warmup, dev, keep):
    d = cfgs.make_gmsq_decode(dev)
    keep["decode"] = d
    M, K = d["x"].shape
    E, _, N = d["weight"].shape
    counts = np.diff([0] + d["group_list"])
    nbytes = decode_bytes(counts, K, N)
    fn = lambda: cb.grouped_matmul_swiglu_quant(d["x"], d["weight"], d["weight_scale"], d["x_scale"], d["group_list"])
    timer = KernelTimer(steps)
    ms, _ = time_op(fn, steps, warmup, timer)
    kms = timer.median_ms()
    res = {"ms": ms, "gbs": nbytes / (ms * 1e-3) / 1e9, "bytes": nbytes, "gemm_kernel_ms": kms,
           "roofline": roofline("hbm", nbytes / (kms * 1e-3) / 1e9, "GB/s"),
           "config": {"workload": "gmsq_decode", "rows": M, "experts": E, "K": K, "N": N,
                      "routing": "256 tokens x top-8 uniform, numpy seed 0",
                      "rows_per_expert_max": int(counts.max()), "rows_per_expert_min": int(counts.min())}}
    # down-projection on the decode output
    y, ys = fn()
    w2, ws2 = d["down_weight"], d["down_weight_scale"]
    K2, N2 = w2.shape[1], w2.shape[2]
    act_e = int(np.sum(counts > 0))
    b2 = act_e * K2 * N2 + M * K2 + 2 * M * N2 + 4 * M + 4 * N2 * act_e
    fn2 = lambda: cb.grouped_matmul_quant(y, w2, ws2, ys, d["group_list"])
    timer2 = KernelTimer(steps)
    ms2, _ = time_op(fn2, steps, warmup, timer2)
    k2 = timer2.median_ms()
    down = {"ms": ms2, "gbs": b2 / (ms2 * 1e-3) / 1e9, "bytes": b2, "gemm_kernel_ms": k2,
            "roofline": roofline("hbm", b2 / (k2 * 1e-3) / 1e9, "GB/s"),
            "config": {"workload": "down_proj", "rows": M, "K": K2, "N": N2, "experts": E}}
    return res, down


def bench_ardq(steps, warmup, dev):
    d = cfgs.make_ardq(dev)
    R, H = d["x1"].shape
    nbytes = 2 * (2 * R * H) + 2 * H + 2 * R * H + R * H + 4 * R
    fn = lambda: cb.add_rms_norm_dynamic_quant(d["x1"], d["x2"], d["gamma"], d["epsilon"])
    timer = KernelTimer(steps)
    ms, _ = time_op(fn, steps, warmup, timer, flush=Flush(dev))
    kms = timer.median_ms()
    return {"ms": ms, "gbs": nbytes / (ms * 1e-3) / 1e9, "bytes": nbytes, "kernel_ms": kms,
            "roofline": roofline("hbm", nbytes / (kms * 1e-3) / 1e9, "GB/s"),
            "config": {"workload": "ardq", "rows": R, "cols": H, "dtype": "bf16"}}


def bench_qmm(steps, warmup, dev):
    d = cfgs.make_qmm(dev)
    M, K = d["x1"].shape
    N = d["x2"].shape[1]
    ops = 2.0 * M * K * N
    fn = lambda: cb.quant_matmul(d["x1"], d["x2"], d["scale"], pertoken_scale=d["pertoken_scale"],
                                 output_dtype="bfloat16")
    timer = KernelTimer(steps)
    ms, _ = time_op(fn, steps, warmup, timer, flush=Flush(dev))
    kms = timer.median_ms()
    return {"ms": ms, "tops": ops / (ms * 1e-3) / 1e12, "gemm_kernel_ms": kms,
            "roofline": roofline("mfma", ops / (kms * 1e-3) / 1e12, "TFLOP/s"),
            "config": {"workload": "qmm", "M": M, "K": K, "N": N}}


def bench_gmm(steps, warmup, dev):
    """Context: GroupedMatmul, the reference's float grouped GEMM, in bf16 on 64 experts (its expert
    limit) x 256 rows, K = N = 4096, with a bf16 bias; against the 2.5 PFLOP/s dense bf16 peak."""
    E, rows, K, N = 64, 256, 4096, 4096
    g = torch.Generator(device=dev)
    g.manual_seed(31)
    x = torch.randn(E * rows, K, device=dev, generator=g).to(torch.bfloat16)
    w = torch.randn(E, K, N, device=dev, generator=g).to(torch.bfloat16)
    b = torch.randn(E, N, device=dev, generator=g).to(torch.bfloat16)
    gl = [rows * (i + 1) for i in range(E)]
    flops = 2.0 * E * rows * K * N
    fn = lambda: cb.grouped_matmul(x, w, gl, bias=b, split_item=2)
    timer = KernelTimer(steps)
    ms, _ = time_op(fn, steps, warmup, timer)
    kms = timer.median_ms()
    # the same problem with the weight stored [E, N, K] (transpose_weight), and the vendor batched
    # bf16 GEMM (torch.bmm -> hipBLASLt, no bias) on the equal-sized groups, wall-clock timed
    wt = w.transpose(1, 2).contiguous()
    ms_t, _ = time_op(lambda: cb.grouped_matmul(x, wt, gl, bias=b, split_item=2, transpose_weight=True), steps, warmup)
    del wt
    xb = x.view(E, rows, K)
    ms_v, _ = time_op(lambda: torch.bmm(xb, w), steps, warmup)
    return {"value": round(flops / (ms * 1e-3) / 1e12, 1), "unit": "TFLOP/s", "ms_per_step": round(ms, 4),
            "kernel_ms": round(kms, 4),
            "transpose_weight_tflops": round(flops / (ms_t * 1e-3) / 1e12, 1),
            "vendor_bmm_tflops": round(flops / (ms_v * 1e-3) / 1e12, 1),
            "roofline": roofline("mfma", flops / (kms * 1e-3) / 1e12, "TFLOP/s", peak=PEAK_BF16_TFLOPS),
            "config": {"workload": "grouped_matmul", "dtype": "bf16", "experts": E, "rows_per_expert": rows,
                       "K": K, "N": N, "bias": "bf16", "transpose_weight": False}}


def bench_vendor(steps, warmup, dev):
    """Context for the GEMM figures: the vendor int8 GEMM (torch._int_mm -> hipBLASLt, int32 out, no
    epilogue) on the QuantMatmul shape, with the weight as the operator receives it (N contiguous)
    and pre-transposed (K contiguous, a layout the drop-in boundary does not hand over)."""
    d = cfgs.make_qmm(dev)
    x1, x2 = d["x1"], d["x2"]
    M, K = x1.shape
    N = x2.shape[1]
    ops = 2.0 * M * K * N
    res = {"op": "torch._int_mm (hipBLASLt)", "M": M, "K": K, "N": N}
    for name, w in (("n_contiguous", x2), ("k_contiguous", x2.t().contiguous().t())):
        try:
            ms, _ = time_op(lambda: torch._int_mm(x1, w), steps, warmup)
            res[name] = {"tops": round(ops / (ms * 1e-3) / 1e12, 1), "ms": round(ms, 4)}
        except Exception as exc:  # reported, not fatal: the vendor path is context only
            res[name] = {"error": str(exc).splitlines()[0][:200]}
    return res


def bench_mfma_probe(dev, iters=20000):
    """Context for the int8 roofline: the matrix-core rate this device sustains with no memory
    traffic (cb_probe_mfma_i8: independent 32x32x32 int8 MFMA chains on every CU), timed with HIP
    events around the kernel.  The published 5.0 POPS assumes the peak clock; this is what the part
    delivers at the clock it holds under MFMA load."""
    import ctypes
    lib = L.load()
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    sink = torch.zeros(8 * cus, dtype=torch.int32, device=dev)
    ops = ctypes.c_int64(0)
    st = torch.cuda.current_stream().cuda_stream
    best = None
    for _ in range(4):
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record(); b.record()
        torch.cuda.synchronize()
        lib.cb_set_kernel_timing(a.cuda_event, b.cuda_event)
        rc = lib.cb_probe_mfma_i8(iters, sink.data_ptr(), sink.numel(), ctypes.byref(ops), st)
        if rc != 0:
            return {"error": L.status_string(rc)}
        torch.cuda.synchronize()
        ms = a.elapsed_time(b)
        best = ms if best is None else min(best, ms)
    tops = ops.value / (best * 1e-3) / 1e12
    return {"tops": round(tops, 1), "frac_of_published_peak": round(tops / PEAK_INT8_TOPS, 4), "ms": round(best, 4),
            "kernel": "cb_probe_mfma_i8", "iters": iters}


def _hbm_entry(fn, nbytes, steps, warmup, config):
    """value: algorithmic bytes / wall time of the whole op call (host wrapper included);
    roofline: the same bytes / device time of the op's kernels (HIP events on its stream)."""
    timer = KernelTimer(steps)
    ms, _ = time_op(fn, steps, warmup, timer)
    kms = timer.median_ms()
    gbs = nbytes / (ms * 1e-3) / 1e9
    return {"value": round(gbs, 1), "unit": "GB/s", "ms_per_step": round(ms, 4), "kernel_ms": round(kms, 4),
            "bytes": int(nbytes), "roofline": roofline("hbm", nbytes / (kms * 1e-3) / 1e9, "GB/s"), "config": config}


def bench_routing(steps, warmup, dev):
    """The routing operators on either side of the experts; algorithmic bytes = every input byte read
    once plus every output byte written once."""
    res = {}
    d = cfgs.make_gating(dev)
    T, E = d["x"].shape
    k = d["k"]
    res["gating"] = _hbm_entry(lambda: cb.moe_gating_top_k_softmax(d["x"], None, k), T * E * 4 + T * k * 12,
                               steps, warmup, {"workload": "moe_gating_top_k_softmax", "tokens": T, "experts": E,
                                               "k": k, "dtype": "fp32"})
    del d
    d = cfgs.make_rerouting(dev)
    A, H = d["tokens"].shape
    n, e = d["counts"].shape
    res["rerouting"] = _hbm_entry(lambda: cb.moe_re_routing(d["tokens"], d["counts"], d["scales"]),
                                  2 * A * H + A * (4 + 4 + 4) + n * e * 4 + e * 4, steps, warmup,
                                  {"workload": "moe_re_routing", "rows": A, "hidden": H, "ranks": n,
                                   "local_experts": e, "dtype": "int8"})
    del d
    d = cfgs.make_finalize(dev)
    RK, H = d["epr"].shape
    R, K = d["scales"].shape
    res["finalize"] = _hbm_entry(
        lambda: cb.moe_finalize_routing(d["epr"], d["esdr"], d["skip1"], None, None, d["scales"], None, 0),
        RK * H * 2 + R * H * 2 * 2 + RK * 4 + R * K * 4, steps, warmup,
        {"workload": "moe_finalize_routing", "tokens": R, "k": K, "hidden": H, "dtype": "bf16"})
    del d
    d = cfgs.make_dqsq(dev)
    M, N2 = d["x"].shape
    res["dqsq"] = _hbm_entry(lambda: cb.dequant_swiglu_quant(d["x"], d["weight_scale"], d["activation_scale"]),
                             M * N2 * 4 + N2 * 4 + M * 4 + M * (N2 // 2) + M * 4, steps, warmup,
                             {"workload": "dequant_swiglu_quant", "rows": M, "cols": N2, "dtype": "int32"})
    return res


def bench_copy(steps, warmup, dev):
    """Plain device copy of 2 GiB: the calibration kernel for the FETCH_SIZE / WRITE_SIZE counters."""
    n = 2 << 30
    a = torch.empty(n, dtype=torch.uint8, device=dev).fill_(1)
    b = torch.empty_like(a)
    ms, _ = time_op(lambda: b.copy_(a), steps, warmup)
    return {"ms": ms, "gbs": 2 * n / (ms * 1e-3) / 1e9, "bytes_read": n, "bytes_written": n}


def traffic_from_profiles(kernel_tag, kernel):
    """HBM bytes per launch of a kernel as recorded in profiles/<kernel_tag>_traffic.md (a line
    'traffic_bytes_per_launch: N', derived from FETCH_SIZE + WRITE_SIZE scaled by the copy-kernel
    calibration), or None when no such summary is committed or when the summary's 'kernel_name:'
    line does not name `kernel` (the kernel this library launches today), so that a figure measured
    on an earlier kernel is never reported."""
    path = os.path.join(ROOT, "profiles", f"{kernel_tag}_traffic.md")
    if not os.path.exists(path):
        return None
    name, value = None, None
    for line in open(path):
        line = line.strip()
        if line.startswith("kernel_name:"):
            name = line.split(":", 1)[1].strip()
        elif line.startswith("traffic_bytes_per_launch:"):
            value = int(float(line.split(":", 1)[1].strip()))
    return value if name is not None and kernel in name else None


ROUTING_KERNELS = {"finalize": "cb::mfr_vec_kernel", "rerouting": "cb::mrr_copy_kernel", "dqsq": "cb::dqsq_vec_kernel"}


def cpu_baseline(d, budget_s=12.0):
    """The C oracle on the host cores over whole experts of the prefill config, until ~budget_s."""
    from oracle import oracle as orc
    gl = d["group_list"]
    starts = [0] + gl[:-1]
    K = d["x"].shape[1]
    N = d["weight"].shape[2]
    ws = d["weight_scale"].cpu().numpy()
    xs = d["x_scale"].cpu().numpy()
    order = np.argsort([e - s for s, e in zip(starts, gl)])  # lightest experts first, then heavier
    done_rows, t_total, experts = 0, 0.0, []
    for g in order[len(order) // 2:]:
        s, e = starts[g], gl[g]
        if e == s:
            continue
        x = d["x"][s:e].cpu().numpy()
        w = d["weight"][g:g + 1].cpu().numpy()
        t0 = time.perf_counter()
        orc.gmsq(x, w, ws[g:g + 1], xs[s:e], np.array([e - s]))
        t_total += time.perf_counter() - t0
        done_rows += e - s
        experts.append(int(g))
        if t_total >= budget_s:
            break
    ops = 2.0 * done_rows * K * N
    # OpenMP runs one thread per core of this process's CPU set unless OMP_NUM_THREADS says fewer
    cores = len(os.sched_getaffinity(0))
    if os.environ.get("OMP_NUM_THREADS", "").isdigit():
        cores = min(cores, int(os.environ["OMP_NUM_THREADS"]))
    return {"value": round(ops / t_total / 1e12, 4), "unit": "TOPS", "cores": cores, "kind": "port",
            "sample": f"oracle/cb_oracle.c or_gmsq (OpenMP) on {done_rows} rows = {len(experts)} whole experts "
                      f"of the prefill config, {t_total:.1f} s"}


def cpu_baseline_decode(d, budget_s=8.0):
    """The C oracle on the host cores over the whole decode config (config 5), in passes over every
    active expert until ~budget_s, in GB/s of the same algorithmic bytes as the GPU figure: each
    active expert's weights once, its rows of x, y and the scales.  Every pass streams all experts'
    weights (7.5 GB), so no pass finds them in a CPU cache."""
    from oracle import oracle as orc
    gl = d["group_list"]
    starts = [0] + gl[:-1]
    K = d["x"].shape[1]
    N = d["weight"].shape[2]
    ws = d["weight_scale"].cpu().numpy()
    xs = d["x_scale"].cpu().numpy()
    xh = d["x"].cpu().numpy()
    wh = d["weight"].cpu().numpy()
    groups = [(g, starts[g], gl[g]) for g in range(len(gl)) if gl[g] > starts[g]]
    pass_bytes = sum(decode_bytes([e - s], K, N) for _, s, e in groups)
    nbytes, t_total, passes = 0, 0.0, 0
    while t_total < budget_s:
        for g, s, e in groups:
            t0 = time.perf_counter()
            orc.gmsq(xh[s:e], wh[g:g + 1], ws[g:g + 1], xs[s:e], np.array([e - s]))
            t_total += time.perf_counter() - t0
        nbytes += pass_bytes
        passes += 1
    del wh
    cores = len(os.sched_getaffinity(0))
    if os.environ.get("OMP_NUM_THREADS", "").isdigit():
        cores = min(cores, int(os.environ["OMP_NUM_THREADS"]))
    rows = sum(e - s for _, s, e in groups)
    return {"value": round(nbytes / t_total / 1e9, 3), "unit": "GB/s", "cores": cores, "kind": "port",
            "sample": f"oracle/cb_oracle.c or_gmsq (OpenMP), {passes} passes over the decode config's "
                      f"{len(groups)} active experts ({rows} rows), {t_total:.1f} s"}


def power_workload(name, dev):
    """(label, fn) of one operator call for the --power mode: the bench's own inputs of each workload,
    and the light / heavy expert subsets of the prefill routing (experts with at most / more than 256
    rows, their rows gathered into a contiguous problem)."""
    if name in ("prefill", "heavy", "light"):
        d = cfgs.make_gmsq_prefill(dev)
        if name != "prefill":
            cnt = np.diff([0] + d["group_list"])
            sel = np.nonzero(cnt > 256 if name == "heavy" else cnt <= 256)[0]
            starts = np.concatenate([[0], np.cumsum(cnt)[:-1]])
            rows = torch.from_numpy(np.concatenate([np.arange(starts[e], starts[e] + cnt[e]) for e in sel])).to(dev)
            es = torch.from_numpy(sel).to(dev)
            d = {"x": d["x"].index_select(0, rows), "weight": d["weight"].index_select(0, es),
                 "weight_scale": d["weight_scale"].index_select(0, es), "x_scale": d["x_scale"].index_select(0, rows),
                 "group_list": [int(v) for v in np.cumsum(cnt[sel])]}
            torch.cuda.empty_cache()
        return (f"gmsq_{name}", lambda: cb.grouped_matmul_swiglu_quant(d["x"], d["weight"], d["weight_scale"],
                                                                        d["x_scale"], d["group_list"]))
    if name == "decode":
        d = cfgs.make_gmsq_decode(dev, with_down=False)
        return "gmsq_decode", lambda: cb.grouped_matmul_swiglu_quant(d["x"], d["weight"], d["weight_scale"],
                                                                      d["x_scale"], d["group_list"])
    if name == "qmm":
        d = cfgs.make_qmm(dev)
        return "qmm", lambda: cb.quant_matmul(d["x1"], d["x2"], d["scale"], pertoken_scale=d["pertoken_scale"],
                                              output_dtype="bfloat16")
    if name == "down_prefill":
        gl = cfgs.cumsum_list(cfgs.zipf_group_counts(131072, 256))
        r = cfgs.streams(41, 4)
        x = cfgs.rand_i8((131072, 2048), dev, r[0])
        xs = cfgs.rand_uniform((131072,), 0.005, 0.02, dev, r[1])
        w = cfgs.rand_i8((256, 2048, 7168), dev, r[2])
        ws = cfgs.rand_uniform((256, 7168), 0.001, 0.01, dev, r[3])
        return "down_proj_prefill", lambda: cb.grouped_matmul_quant(x, w, ws, xs, gl)
    if name == "ardq":
        d = cfgs.make_ardq(dev)
        return "ardq", lambda: cb.add_rms_norm_dynamic_quant(d["x1"], d["x2"], d["gamma"], d["epsilon"])
    if name == "dqsq":
        d = cfgs.make_dqsq(dev)
        return "dqsq", lambda: cb.dequant_swiglu_quant(d["x"], d["weight_scale"], d["activation_scale"])
    if name == "mfma_probe":
        import ctypes
        lib = L.load()
        sink = torch.zeros(8 * 256, dtype=torch.int32, device=dev)
        ops = ctypes.c_int64(0)
        return "mfma_probe", lambda: lib.cb_probe_mfma_i8(2000, sink.data_ptr(), sink.numel(), ctypes.byref(ops),
                                                          torch.cuda.current_stream().cuda_stream)
    raise SystemExit(f"bench.py --power: unknown workload {name}")


def power_mode(names, seconds, dev):
    """Loops each workload for `seconds` while `amd-smi metric --power --clock` is sampled about once
    a second (after a 2 s settling time), and prints one JSON line per workload: the median socket
    power and GFX clock over the samples and the mean time per call."""
    import re
    import subprocess
    import threading
    for name in names:
        label, fn = power_workload(name, dev)
        fn()
        torch.cuda.synchronize()
        samples, stop = [], threading.Event()

        def sample():
            time.sleep(2.0)
            while not stop.is_set():
                r = subprocess.run(["amd-smi", "metric", "--power", "--clock"], capture_output=True, text=True)
                pw = re.search(r"SOCKET_POWER:\s*([0-9.]+)", r.stdout)
                k = r.stdout.find("GFX")  # the first CLK line after it is the GFX clock
                gfx = re.search(r"\bCLK:\s*([0-9.]+)", r.stdout[k if k >= 0 else 0:])
                if pw and gfx:
                    samples.append((float(pw.group(1)), float(gfx.group(1))))
                time.sleep(1.0)

        th = threading.Thread(target=sample, daemon=True)
        th.start()
        t0, n = time.perf_counter(), 0
        while time.perf_counter() - t0 < seconds:
            for _ in range(10):
                fn()
            torch.cuda.synchronize()
            n += 10
        ms = (time.perf_counter() - t0) * 1e3 / n
        stop.set()
        th.join()
        pw = [p for p, _ in samples]
        ck = [c for _, c in samples]
        print(json.dumps({"power_mode": label, "library": L.LIB_PATH, "ms_per_call": round(ms, 4), "calls": n,
                          "samples": len(samples),
                          "socket_power_w_median": float(np.median(pw)) if pw else None,
                          "gfx_clock_mhz_median": float(np.median(ck)) if ck else None,
                          "gfx_clock_mhz_range": [min(ck), max(ck)] if ck else None}), flush=True)


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=10,
                    help="untimed calls per workload first: the clock settles at the board power limit over "
                         "the first 5-6 prefill calls (4.7-5.0 ms, then 4.1-4.2 ms)")
    ap.add_argument("--only", default="prefill,gather,down_prefill,decode,ardq,qmm,routing,gmm,vendor",
                    help="comma list of prefill, gather and down_prefill (need prefill), decode, ardq, qmm, "
                         "routing, gmm, vendor, copy")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--power", default=None,
                    help="comma list of workloads (prefill, heavy, light, decode, qmm, down_prefill, ardq, dqsq, "
                         "mfma_probe): loop each for --seconds while sampling socket power and GFX clock with "
                         "amd-smi, print one JSON line each, and exit (no bench line)")
    ap.add_argument("--seconds", type=float, default=8.0)
    ap.add_argument("--lib", default=None, help="operator library to load instead of the in-tree build "
                                                "(a variant built from a patched source tree, for --power)")
    args = ap.parse_args()
    if args.lib:
        L.LIB_PATH = os.path.abspath(args.lib)
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py: this build measures one GPU only (the operators are single-device; expert "
              "parallelism across GPUs is a design note, not a measured path). Use --gpus 1.", file=sys.stderr)
        sys.exit(2)
    if not torch.cuda.is_available():
        print("bench.py: no ROCm device visible", file=sys.stderr)
        sys.exit(2)
    dev = "cuda:0"
    torch.cuda.set_device(0)
    if args.power:
        power_mode(args.power.split(","), args.seconds, dev)
        return
    only = set(args.only.split(","))
    keep = {}
    out = {"metric": METRIC, "value": None, "unit": "TOPS", "n_gpus": 1, "steps": args.steps,
           "warmup": args.warmup, "ms_per_step": None, "higher_is_better": True, "scaling": "weak",
           "vs_baseline": None, "dtype": "int8",
           "data": "synthetic: int8 / fp32 tensors and routing drawn with seeded numpy generators on the host, then copied to HBM before timing"}
    if "prefill" in only:
        p = bench_prefill(args.steps, args.warmup, dev, keep)
        out.update(value=round(p["tops"], 2), ms_per_step=round(p["ms"], 4), config=p["config"],
                   roofline=p["roofline"])
        out["timing"] = ("ms_per_step: median over the timed calls of HIP events around each whole "
                         "operator call (every kernel it launches); wall_ms_per_step: host clock over "
                         "the timed loop / steps")
        out["wall_ms_per_step"] = round(p["wall_ms"], 4)
        out["prefill_gemm_kernel_ms"] = round(p["gemm_kernel_ms"], 4)
        out["frac_of_int8_peak"] = round(p["tops"] / PEAK_INT8_TOPS, 4)
        if "gather" in only:
            out["prefill_gather"] = bench_prefill_gather(args.steps, args.warmup, dev, keep)
        if "down_prefill" in only:
            out["down_proj_prefill"] = bench_down_prefill(args.steps, args.warmup, dev, keep)
    if "decode" in only:
        keep.pop("prefill_tensors", None)
        dres, down = bench_decode(args.steps, args.warmup, dev, keep)
        out["decode"] = {"value": round(dres["gbs"], 1), "unit": "GB/s", "ms_per_step": round(dres["ms"], 4),
                         "frac_of_hbm_peak": round(dres["gbs"] / PEAK_HBM_GBS, 4), "bytes": dres["bytes"],
                         "roofline": dres["roofline"], "config": dres["config"]}
        out["down_proj"] = {"value": round(down["gbs"], 1), "unit": "GB/s", "ms_per_step": round(down["ms"], 4),
                            "bytes": down["bytes"], "roofline": down["roofline"], "config": down["config"]}
    if "ardq" in only:
        a = bench_ardq(args.steps, args.warmup, dev)
        out["ardq"] = {"value": round(a["gbs"], 1), "unit": "GB/s", "ms_per_step": round(a["ms"], 4),
                       "kernel_ms": round(a["kernel_ms"], 4),
                       "roofline": a["roofline"], "config": a["config"]}
    if "qmm" in only:
        q = bench_qmm(args.steps, args.warmup, dev)
        out["qmm"] = {"value": round(q["tops"], 2), "unit": "TOPS", "ms_per_step": round(q["ms"], 4),
                      "roofline": q["roofline"], "config": q["config"]}
    if "routing" in only:
        out["routing"] = bench_routing(args.steps, args.warmup, dev)
    if "gmm" in only:
        out["grouped_matmul"] = bench_gmm(args.steps, args.warmup, dev)
    if "vendor" in only:
        out["vendor_int8_gemm"] = bench_vendor(args.steps, args.warmup, dev)
        out["mfma_probe"] = bench_mfma_probe(dev)
    if "copy" in only:
        c = bench_copy(args.steps, args.warmup, dev)
        out["copy"] = {"value": round(c["gbs"], 1), "unit": "GB/s", "ms_per_step": round(c["ms"], 4),
                       "bytes_read": c["bytes_read"], "bytes_written": c["bytes_written"]}
    if out.get("roofline") is not None:
        out["roofline"]["traffic"] = traffic_from_profiles("prefill_gemm", "cb::gmsq_prefill_kernel<false, true>(")
    if "decode" in out:
        out["decode"]["roofline"]["traffic"] = traffic_from_profiles("decode_gemm", "cb::gmsq_decode_kernel(")
        out["down_proj"]["roofline"]["traffic"] = traffic_from_profiles("down_proj_gemm", "cb::skinny_kernel<1")
    for name in ("finalize", "rerouting", "dqsq"):
        if name in out.get("routing", {}):
            out["routing"][name]["roofline"]["traffic"] = traffic_from_profiles("routing_" + name, ROUTING_KERNELS[name])
    if not args.no_cpu and "prefill" in keep:
        out["cpu_baseline"] = cpu_baseline(keep["prefill"])
    if not args.no_cpu and "decode" in keep:
        out["decode"]["cpu_baseline"] = cpu_baseline_decode(keep["decode"])
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
