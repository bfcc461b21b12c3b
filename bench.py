#!/usr/bin/env python
"""Benchmark of the hip provider on one MI355X.

Headline (the JSON line's `value`): BASELINE config 2, fused row softmax forward +
backward in f16 storage with f32 math, 16384 x 4096 — one step = stable_softmax_f16
then softmax_backward_f16 through prepared intent.jit calls; throughput = algorithmic
bytes (fwd 4*M*N + bwd 6*M*N = 671,088,640 B) / measured step time (K eager steps between HIP
events; the same step as hipGraph replays is reported beside it), inputs resident in HBM. `roofline` is the dominant kernel (the backward), timed with HIP events on the launch
stream between the launches of the real fwd/bwd sequence, with the same kernel timed cold (after a MALL flush)
beside it as `cold_backward`. `operators` carries every other configuration: the median
of 33 cold calls (first dropped, 512 MiB write-then-read flush of the 256 MB MALL before each), events around the
launches queued behind the flush so that they bracket the kernels as the reference's in-graph events do
(operator_ms); the median of graph replays timed around graph.replay() is kept beside it as graph_ms. `cpu_baseline`
is the oracle on a bounded sample on this host.

Usage: python bench.py [--gpus 1] [--steps 20] [--warmup 5] [--no-operators] [--no-cpu-baseline]
"""
from __future__ import annotations

import argparse
import json
import os
import statistics
import sys
import time
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

METRIC = "HBM GB/s (softmax, SpMV) and TFLOP/s (GEMM, attention) vs 1-GPU roofline"
HBM_PEAK_GBS = 8000.0
MFMA_PEAK_TFLOPS = 2500.0          # dense bf16 / fp16
INT8_PEAK_TOPS = 5000.0            # dense int8
MFMA_F32_PEAK_TFLOPS = 157.3       # dense fp32 MFMA
FWD_BYTES_PER_ELEMENT, BWD_BYTES_PER_ELEMENT = 4, 6
ATTENTION_FLOP = 4 * 4 * 32 * 4096 * 4096 * 128 // 2   # config 4, causal half of 4*B*H*S^2*D


def log(*parts):
    print("[bench]", *parts, file=sys.stderr, flush=True)


def parse():
    parser = argparse.ArgumentParser()
    parser.add_argument("--gpus", type=int, default=1)
    parser.add_argument("--steps", type=int, default=20)
    parser.add_argument("--warmup", type=int, default=5)
    parser.add_argument("--no-operators", action="store_true")
    parser.add_argument("--no-cpu-baseline", action="store_true")
    parser.add_argument("--operators",
                        default="softmax_f32,gemm,attention,spmv,gemm_f16_relu,gemm_f32,linear_f32,gqa,attention_bf16,"
                                "attention_bwd,attention_bwd_large,paged_decode,spmm,varlen_prefill,gemm_i8,quantized_gemm,"
                                "attention_bias,continuous_decode,grouped_decode,varlen_decode,mla_prefill,mla_prefill_large")
    parser.add_argument("--copy-calibration", action="store_true",
                        help="only run 20 device copies of 512 MiB (a known-traffic kernel for counter scaling)")
    parser.add_argument("--only", default=None,
                        help="run only this operator's timing (softmax_fwd, softmax_bwd or a name in --operators), "
                             "for per-kernel profiling")
    return parser.parse_args()


# ------------------------------------------------------------------------------ GPU timing
class Flush:
    """Writes zeros over 512 MiB (twice the 256 MB MALL), then reads it back, outside each timed
    interval. The zero fill alone evicts the inputs but leaves the caches full of dirty lines
    whose write-back the next (timed) kernel would pay for (measured: +28 us on the paged-decode
    partials); the read-back leaves clean, unrelated lines, so the timed kernel starts cold and
    pays only for its own traffic."""

    def __init__(self, device):
        import torch

        self.buffer = torch.empty(512 << 20, dtype=torch.uint8, device=device)
        self.floats = self.buffer.view(torch.float32)       # zeros; summed in place, no cast copy

    def __call__(self):
        import torch

        self.buffer.zero_()
        torch.sum(self.floats)


def graph_median_ms(launch, flush, replays=33):
    """Graph replays with a flush before each, HIP events recorded around graph.replay(); drops
    the first sample and reports the median. The interval includes the replay's own launch path
    (about 7 us more than operator_ms on a 6 us kernel)."""
    import torch

    launch()
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(stream):
        with torch.cuda.graph(graph, stream=stream):
            launch()
    torch.cuda.current_stream().wait_stream(stream)
    torch.cuda.synchronize()
    samples = []
    for _ in range(replays):
        flush()
        start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        start.record()
        graph.replay()
        end.record()
        end.synchronize()
        samples.append(start.elapsed_time(end))
    return statistics.median(samples[1:])


# graph-replay time of the last operator_ms call, attached to its operator's record
_LAST_GRAPH_MS = {}


def operator_ms(launch, flush, replays=33):
    """Median duration of one call's kernels, cold, as the reference measures it.

    The reference (runtime/triton/cuda.py:18-44 with the hooks of runtime/triton/program.py:47-63)
    captures zero-fill, start.record(), the launch and end.record() in one graph, so its events
    bracket the kernels and not the graph launch. ROCm's torch refuses event records inside a
    capture ("External events are disallowed in rocm"). Here the 512 MiB flush (about 200 us of
    GPU work) is enqueued first, then start, the eager launch and end: the launches reach the
    queue while the flush still runs, so the events again bracket only the kernels. The graph
    replay time (events around graph.replay()) is sampled in the same loop, alternating with the
    eager samples so both see the same clocks, and kept beside it."""
    import torch

    launch()
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(stream):
        with torch.cuda.graph(graph, stream=stream):
            launch()
    torch.cuda.current_stream().wait_stream(stream)
    torch.cuda.synchronize()
    eager, replayed = [], []
    for _ in range(replays):
        for samples, body in ((eager, launch), (replayed, graph.replay)):
            flush()
            start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            start.record()
            body()
            end.record()
            end.synchronize()
            samples.append(start.elapsed_time(end))
    _LAST_GRAPH_MS["graph_ms"] = statistics.median(replayed[1:])
    return statistics.median(eager[1:])


def events_ms(launch, count):
    """Average duration of `count` back-to-back launches, HIP events on the launch stream."""
    import torch

    torch.cuda.synchronize()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    for _ in range(count):
        launch()
    end.record()
    end.synchronize()
    return start.elapsed_time(end) / count


def sequence_kernel_ms(first, second, steps):
    """Median duration of each of two launches inside the real step sequence (first, second,
    first, ...), HIP events recorded on the launch stream between them. Timing a kernel alone in
    a loop would re-read inputs the 256 MB MALL still holds; inside the sequence they are cold."""
    import torch

    events = [torch.cuda.Event(enable_timing=True) for _ in range(2 * steps + 1)]
    torch.cuda.synchronize()
    events[0].record()
    for i in range(steps):
        first()
        events[2 * i + 1].record()
        second()
        events[2 * i + 2].record()
    events[-1].synchronize()
    a = sorted(events[2 * i].elapsed_time(events[2 * i + 1]) for i in range(steps))
    b = sorted(events[2 * i + 1].elapsed_time(events[2 * i + 2]) for i in range(steps))
    return statistics.median(a), statistics.median(b)


# ------------------------------------------------------------------------------ CPU baseline
# seconds of the last cpu_median_seconds call with every allowed CPU as the oracle's worker count
_LAST_CPU_ALL = {}


def cpu_model() -> str:
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def cpu_median_seconds(run):
    """Reference CPU protocol (runtime/mojo/compilation.py:34,56-91; mojo/program.py:28-34):
    64 MiB eviction write outside the interval, repetitions = clamp(10 ms / first, 1, 50),
    median of 7 samples. Timed with the oracle's default worker count (the reference's
    min(8, allowed CPUs), targets/execution.py:20-26), the figure returned, and again with every
    allowed CPU, kept in _LAST_CPU_ALL for the operator's record."""
    import oracle

    seconds = _cpu_median_seconds(run)
    allowed = len(os.sched_getaffinity(0))
    default = oracle.default_workers
    oracle.default_workers = lambda: allowed
    try:
        _LAST_CPU_ALL.update(seconds=_cpu_median_seconds(run), cores=allowed, default_seconds=seconds)
    finally:
        oracle.default_workers = default
    return seconds


def _cpu_median_seconds(run):
    import numpy as np

    evict = np.empty(64 << 20, np.uint8)
    begin = time.perf_counter()
    run()
    first = time.perf_counter() - begin
    reps = int(min(50, max(1, 0.010 / max(first, 1e-9))))
    samples = []
    for _ in range(7):
        evict.fill(1)
        begin = time.perf_counter()
        for _ in range(reps):
            run()
        samples.append((time.perf_counter() - begin) / reps)
    return statistics.median(samples)


def attach_all_cores(op):
    """The operator's CPU record gains the host CPU model and its rate with every allowed CPU
    (the rate fields scaled by the default-workers time over the all-CPU time of the same sample)."""
    record = op.get("cpu")
    if not isinstance(record, dict) or "seconds" not in _LAST_CPU_ALL:
        return
    ratio = _LAST_CPU_ALL["default_seconds"] / _LAST_CPU_ALL["seconds"]
    rates = {key: round(value * ratio, 6) for key, value in record.items()
             if key in ("gbs", "tflops", "tops") and isinstance(value, (int, float))}
    if isinstance(record.get("ms"), (int, float)):
        rates["ms"] = round(record["ms"] / ratio, 3)
    record["cpu_model"] = cpu_model()
    record["all_cores"] = {"cores": _LAST_CPU_ALL["cores"], **rates}


def headline_cpu_baseline(x, dy):
    """The oracle on a bounded sample, with the reference's default worker count (min(8, allowed
    CPUs), targets/execution.py:20-26) and again with every allowed CPU."""
    import oracle

    rows = 2048
    xs, gs = x[:rows], dy[:rows]
    nbytes = (FWD_BYTES_PER_ELEMENT + BWD_BYTES_PER_ELEMENT) * rows * x.shape[1]

    def rate(workers):
        def run():
            y = oracle.softmax_fwd(xs, workers=workers)
            oracle.softmax_bwd(y, gs, workers=workers)

        return round(nbytes / _cpu_median_seconds(run) / 1e9, 3)

    workers = oracle.default_workers()
    allowed = len(os.sched_getaffinity(0))
    return {"value": rate(workers), "unit": "GB/s", "cores": workers, "kind": "port", "cpu_model": cpu_model(),
            "sample": f"oracle softmax fwd+bwd f16 on rows 0..{rows - 1} of the 16384x4096 input "
                      f"(1/{x.shape[0] // rows} of the workload), median of 7 samples, "
                      f"{workers} OpenMP workers (min(8, allowed CPUs)); host has {os.cpu_count()} CPUs",
            "all_cores": {"value": rate(allowed), "cores": allowed}}


def box_reference(device, flush):
    """Figures of the box itself, beside the kernels' rooflines: a torch device copy of 512 MiB
    (read + write GB/s) and torch.matmul bf16 8192^3 (hipBLASLt), both timed like the operators
    (operator_ms)."""
    import torch

    src = torch.ones(512 << 20, dtype=torch.uint8, device=device)
    dst = torch.empty_like(src)
    copy_ms = operator_ms(lambda: dst.copy_(src), flush)
    del src, dst
    g = torch.Generator(device="cpu").manual_seed(0)
    a = (torch.rand((8192, 8192), generator=g) * 2 - 1).to(torch.bfloat16).to(device)
    b = (torch.rand((8192, 8192), generator=g) * 2 - 1).to(torch.bfloat16).to(device)
    c = torch.empty((8192, 8192), dtype=torch.bfloat16, device=device)
    gemm_ms = operator_ms(lambda: torch.matmul(a, b, out=c), flush)
    del a, b, c
    sdpa = box_sdpa(device, flush)
    probes = box_probes(device, flush)
    return {"torch_copy_gbs": round(2 * (512 << 20) / copy_ms / 1e6, 1),
            "hipblaslt_bf16_gemm_8192_tflops": round(2 * 8192 ** 3 / gemm_ms / 1e9, 1),
            "hipblaslt_bf16_gemm_8192_ms": round(gemm_ms, 4), **sdpa, **probes}


def box_sdpa(device, flush):
    """torch's scaled_dot_product_attention at config 4 (causal f16, B4 H32 S4096 D128), timed like
    the operators: the box's own fused-attention library kernel beside attention_fwd."""
    import torch
    import torch.nn.functional as F

    g = torch.Generator(device="cpu").manual_seed(0)
    q, k, v = (torch.randn((4, 32, 4096, 128), generator=g).to(torch.float16).to(device) for _ in range(3))
    out = {}
    try:
        ms = operator_ms(lambda: F.scaled_dot_product_attention(q, k, v, is_causal=True, scale=128 ** -0.5), flush)
        out = {"torch_sdpa_causal_f16_config4_ms": round(ms, 4),
               "torch_sdpa_causal_f16_config4_tflops": round(ATTENTION_FLOP / ms / 1e9, 1)}
    except RuntimeError as error:                         # a backend that refuses capture is reported, not fatal
        out = {"torch_sdpa_causal_f16_config4_error": str(error)[:200]}
    del q, k, v
    return out


def box_probes(device, flush):
    """The library's MFMA probe, timed like the operators: the sustained rate of
    v_mfma_f32_32x32x16_{bf16,f16} on register operands, two waves per SIMD (TFLOP/s), with varied
    operands (the switching activity of real data; the figure operators are read against) and
    with one fixed operand pair."""
    import torch

    from intent_amd.runtime.hip.library import BF16, F16, library

    lib = library()
    stream = lambda: torch.cuda.current_stream().cuda_stream  # noqa: E731
    blocks = 2 * lib.device_info(torch.device(device).index or 0)["compute_units"]
    iterations = 2048
    out = torch.empty(blocks * 4, dtype=torch.float32, device=device)
    flops = blocks * 4 * iterations * 8 * 2 * 32 * 32 * 16
    rates = {}
    for name, code in (("bf16", BF16), ("f16", F16)):
        for varied, label in ((1, ""), (0, "_fixed_operands")):
            ms = operator_ms(lambda code=code, varied=varied: lib.check(lib.fn["mfma_probe"](
                code, varied, blocks, iterations, out.data_ptr(), stream())), flush)
            rates[f"mfma_{name}_probe_tflops{label}"] = round(flops / ms / 1e9, 1)
    return {**rates,
            "mfma_probe": f"{blocks} workgroups x 4 waves x {iterations} rounds of 8 independent 32x32x16 MFMAs"}


# ------------------------------------------------------------------------------ operators
def op_softmax_f32(device, flush, cpu):
    import torch

    import intent_amd as intent
    from intent_amd.examples import inputs
    from intent_amd.examples.kernels.normalization.softmax import stable_softmax

    x = inputs.softmax_f32()
    call = intent.jit(stable_softmax, backend="hip").prepare(torch.from_numpy(x).to(device))
    ms = operator_ms(call.launch, flush)
    nbytes = 2 * 4 * x.size
    out = {"config": "softmax fwd f32 4096x1024 (config 1)", "median_ms": round(ms, 5),
           "achieved": round(nbytes / ms / 1e6, 1), "unit": "GB/s",
           "roofline_frac": round(nbytes / ms / 1e6 / HBM_PEAK_GBS, 4), "bytes": nbytes,
           "note": "33.5 MB working set; timed after a 512 MiB flush"}
    if cpu:
        import oracle

        seconds = cpu_median_seconds(lambda: oracle.softmax_fwd(x))
        out["cpu"] = {"ms": round(seconds * 1e3, 3), "cores": oracle.default_workers(), "kind": "port"}
    return out


def op_gemm(device, flush, cpu):
    import intent_amd as intent
    from intent_amd.examples import inputs
    from intent_amd.examples.kernels.contraction.gemm import bf16_gemm
    from intent_amd.examples.inputs import bf16_tensor as to_bf16_tensor

    m = n = k = 8192
    a, b = inputs.gemm_bf16()
    call = intent.jit(bf16_gemm, backend="hip").prepare(to_bf16_tensor(a, device), to_bf16_tensor(b, device))
    ms = operator_ms(call.launch, flush)
    flops = 2 * m * n * k
    out = {"config": "GEMM bf16 8192^3, fp32 accumulate (config 3)", "median_ms": round(ms, 4),
           "achieved": round(flops / ms / 1e9, 1), "unit": "TFLOP/s",
           "roofline_frac": round(flops / ms / 1e9 / MFMA_PEAK_TFLOPS, 4), "flops": flops,
           "traffic": read_traffic("gemm_bf16_8192")}
    if cpu:
        import oracle

        rows = 16
        seconds = cpu_median_seconds(lambda: oracle.gemm_bf16(a[:rows], b))
        out["cpu"] = {"tflops": round(2 * rows * n * k / seconds / 1e12, 5), "cores": oracle.default_workers(),
                      "kind": "port", "sample": f"{rows} rows of A"}
    return out


def op_attention(device, flush, cpu):
    import torch

    import intent_amd as intent
    from intent_amd.examples import inputs
    from intent_amd.examples.kernels.streaming.attention import flash_attention_fwd

    q, k, v, scale = inputs.attention_f16()
    t = lambda a: torch.from_numpy(a).to(device)  # noqa: E731
    call = intent.jit(flash_attention_fwd, backend="hip", constexprs={"CAUSAL": True}).prepare(
        t(q), t(k), t(v), scale)
    ms = operator_ms(call.launch, flush)
    b, h, s, d = q.shape
    flops = 4 * b * h * s * s * d // 2
    out = {"config": "causal attention fwd f16 B4 H32 S4096 D128 (config 4)", "median_ms": round(ms, 4),
           "achieved": round(flops / ms / 1e9, 1), "unit": "TFLOP/s",
           "roofline_frac": round(flops / ms / 1e9 / MFMA_PEAK_TFLOPS, 4), "flops": flops,
           "traffic": read_traffic("attention_fwd_config4")}
    if cpu:
        import oracle

        seconds = cpu_median_seconds(lambda: oracle.attention_fwd_f16(q[:1, :1, :1024], k[:1, :1], v[:1, :1],
                                                                      scale, True))
        sample_flops = 4 * 1024 * 1024 * d // 2
        out["cpu"] = {"tflops": round(sample_flops / seconds / 1e12, 5), "cores": oracle.default_workers(),
                      "kind": "port", "sample": "1 (batch, head) pair, first 1024 queries"}
    return out


def op_spmv(device, flush, cpu):
    import torch

    import intent_amd as intent
    from intent_amd.examples import inputs
    from intent_amd.examples.kernels.sparse.csr_spmv import csr_spmv

    offsets, columns, values, x = inputs.spmv_f32()
    t = lambda a: torch.from_numpy(a).to(device)  # noqa: E731
    call = intent.jit(csr_spmv, backend="hip").prepare(t(offsets), t(columns), t(values), t(x))
    ms = operator_ms(call.launch, flush)
    rows, nnz = offsets.shape[0] - 1, int(offsets[-1])
    nbytes = 4 * (rows + 1) + 8 * nnz + 4 * x.shape[0] + 4 * rows
    out = {"config": f"CSR SpMV f32 {rows}^2, {nnz} nnz, rank-law Zipf(1.5) rows (config 5)",
           "median_ms": round(ms, 4), "achieved": round(nbytes / ms / 1e6, 1), "unit": "GB/s",
           "roofline_frac": round(nbytes / ms / 1e6 / HBM_PEAK_GBS, 4), "bytes": nbytes,
           "traffic": read_traffic("spmv_config5")}
    if cpu:
        import oracle

        seconds = cpu_median_seconds(lambda: oracle.csr_spmv(offsets, columns, values, x))
        out["cpu"] = {"gbs": round(nbytes / seconds / 1e9, 3), "cores": oracle.default_workers(), "kind": "port"}
    return out


def op_gemm_f16_relu(device, flush, cpu):
    """`gemm` (contraction/gemm.py:54-73), f16 operands, ACTIVATION = RELU, at the config-3 shape."""
    import torch

    import intent_amd as intent
    from intent_amd.examples import inputs
    from intent_amd.examples.kernels.contraction.gemm import Activation, gemm

    m = n = k = 8192
    rng = np.random.default_rng(0)
    a = inputs.uniform(rng, (m, k), -1.0, 1.0, "f16")
    b = inputs.uniform(rng, (k, n), -1.0, 1.0, "f16")
    call = intent.jit(gemm, backend="hip", constexprs={"ACTIVATION": Activation.RELU}).prepare(
        torch.from_numpy(a).to(device), torch.from_numpy(b).to(device))
    ms = operator_ms(call.launch, flush)
    flops = 2 * m * n * k
    out = {"config": "gemm f16 8192^3, ACTIVATION=RELU, fp32 accumulate", "median_ms": round(ms, 4),
           "achieved": round(flops / ms / 1e9, 1), "unit": "TFLOP/s",
           "roofline_frac": round(flops / ms / 1e9 / MFMA_PEAK_TFLOPS, 4), "flops": flops}
    if cpu:
        import oracle

        rows = 16
        seconds = cpu_median_seconds(lambda: oracle.gemm16(a[:rows], b, relu=True))
        out["cpu"] = {"tflops": round(2 * rows * n * k / seconds / 1e12, 5), "cores": oracle.default_workers(),
                      "kind": "port", "sample": f"{rows} rows of A"}
    return out


def _op_f32(device, flush, cpu, transpose_b):
    """gemm_f32 / linear_f32 (contraction/gemm.py:15-38) at the reference module's shape
    M = K = 4096, N = 14336 (gemm.py:5-7)."""
    import torch

    import intent_amd as intent
    from intent_amd.examples import inputs
    from intent_amd.examples.kernels.contraction.gemm import gemm_f32, linear_f32

    m, k, n = 4096, 4096, 14336
    rng = np.random.default_rng(1)
    a = inputs.uniform(rng, (m, k), -1.0, 1.0)
    b = inputs.uniform(rng, (n, k) if transpose_b else (k, n), -1.0, 1.0)
    defn = linear_f32 if transpose_b else gemm_f32
    call = intent.jit(defn, backend="hip").prepare(torch.from_numpy(a).to(device), torch.from_numpy(b).to(device))
    ms = operator_ms(call.launch, flush)
    flops = 2 * m * n * k
    out = {"config": f"{defn.__name__} M=4096 K=4096 N=14336, f32", "median_ms": round(ms, 4),
           "achieved": round(flops / ms / 1e9, 1), "unit": "TFLOP/s",
           "roofline_frac": round(flops / ms / 1e9 / MFMA_F32_PEAK_TFLOPS, 4), "peak": MFMA_F32_PEAK_TFLOPS,
           "flops": flops}
    if cpu:
        import oracle

        rows = 8
        seconds = cpu_median_seconds(lambda: oracle.gemm_f32(a[:rows], b, transpose_b=transpose_b))
        out["cpu"] = {"tflops": round(2 * rows * n * k / seconds / 1e12, 5), "cores": oracle.default_workers(),
                      "kind": "port", "sample": f"{rows} rows of A"}
    return out


def op_gemm_f32(device, flush, cpu):
    return _op_f32(device, flush, cpu, False)


def op_linear_f32(device, flush, cpu):
    return _op_f32(device, flush, cpu, True)


def _op_attention_grouped(device, flush, cpu, bf16):
    """flash_gqa_attention_fwd (f16, 32 query heads over 8 key/value heads) or
    flash_attention_bf16_fwd (config 4 shapes in bf16), causal, S = 4096, D = 128."""
    import torch

    import intent_amd as intent
    from intent_amd.examples import inputs
    from intent_amd.examples.kernels.streaming.attention import flash_attention_bf16_fwd, flash_gqa_attention_fwd
    from intent_amd.examples.inputs import bf16_tensor as to_bf16_tensor

    b, hq, s, d = 4, 32, 4096, 128
    group = 1 if bf16 else 4
    hk = hq // group
    rng = np.random.default_rng(2)
    dtype = "bf16" if bf16 else "f16"
    q = inputs.normal(rng, (b, hq, s, d), dtype)
    k = inputs.normal(rng, (b, hk, s, d), dtype)
    v = inputs.normal(rng, (b, hk, s, d), dtype)
    scale = float(np.float32(1 / np.sqrt(d)))
    conv = (lambda a: to_bf16_tensor(a, device)) if bf16 else (lambda a: torch.from_numpy(a).to(device))
    defn = flash_attention_bf16_fwd if bf16 else flash_gqa_attention_fwd
    call = intent.jit(defn, backend="hip", constexprs={"HEAD_GROUP": group, "CAUSAL": True}).prepare(
        conv(q), conv(k), conv(v), scale)
    ms = operator_ms(call.launch, flush)
    flops = 4 * b * hq * s * s * d // 2
    name = ("causal attention fwd bf16 B4 H32 S4096 D128 (flash_attention_bf16_fwd)" if bf16 else
            "causal GQA attention fwd f16 B4 HQ32 HK8 S4096 D128 (flash_gqa_attention_fwd)")
    out = {"config": name, "median_ms": round(ms, 4), "achieved": round(flops / ms / 1e9, 1), "unit": "TFLOP/s",
           "roofline_frac": round(flops / ms / 1e9 / MFMA_PEAK_TFLOPS, 4), "flops": flops}
    if cpu:
        import oracle

        seconds = cpu_median_seconds(lambda: oracle.attention_fwd(
            np.ascontiguousarray(q[:1, :group, :1024]), np.ascontiguousarray(k[:1, :1]),
            np.ascontiguousarray(v[:1, :1]), scale, True, head_group=group, storage="bf16" if bf16 else None))
        sample_flops = group * 4 * 1024 * 1024 * d // 2
        out["cpu"] = {"tflops": round(sample_flops / seconds / 1e12, 5), "cores": oracle.default_workers(),
                      "kind": "port", "sample": f"{group} query head(s) of one key head, first 1024 queries"}
    return out


def op_gqa(device, flush, cpu):
    return _op_attention_grouped(device, flush, cpu, False)


def op_attention_bf16(device, flush, cpu):
    return _op_attention_grouped(device, flush, cpu, True)


def op_gemm_i8(device, flush, cpu):
    """gemm_i8 at the reference module's extents (contraction/gemm.py:5-7): int8 operands in the
    full range, int32 bias and output; against the dense int8 MFMA peak."""
    import torch

    import intent_amd as intent
    from intent_amd.examples.kernels.contraction.gemm import gemm_i8

    m, k, n = 4096, 4096, 14336
    rng = np.random.default_rng(7)
    a = rng.integers(-128, 128, (m, k)).astype(np.int8)
    b = rng.integers(-128, 128, (k, n)).astype(np.int8)
    bias = rng.integers(-2**20, 2**20, n).astype(np.int32)
    dev = lambda x: torch.from_numpy(x).to(device)  # noqa: E731
    call = intent.jit(gemm_i8, backend="hip").prepare(dev(a), dev(b), dev(bias))
    ms = operator_ms(call.launch, flush)
    ops = 2 * m * n * k
    out = {"config": f"gemm_i8 M={m} K={k} N={n}, int8 operands, int32 bias and output", "median_ms": round(ms, 4),
           "achieved": round(ops / ms / 1e9, 1), "unit": "TOP/s",
           "roofline_frac": round(ops / ms / 1e9 / INT8_PEAK_TOPS, 4), "ops": ops,
           "bytes": int(m * k + k * n + 4 * n + 4 * m * n)}
    if cpu:
        import oracle

        rows, cols = 16, 1024
        b_part = np.ascontiguousarray(b[:, :cols])
        seconds = cpu_median_seconds(lambda: oracle.gemm_i8(a[:rows], b_part, bias[:cols]))
        out["cpu"] = {"tops": round(2 * rows * cols * k / seconds / 1e12, 5), "cores": 1, "kind": "port",
                      "sample": f"the first {rows} x {cols} block of C (numpy int64 product)"}
    return out


def op_quantized_gemm(device, flush, cpu):
    """quantized_gemm at the reference module's extents: f16 operands N(0,1) and N(0,1)/64, bias
    N(0,1), residual 4 N(0,1), output scales U(0.05, 0.5); int8 output. Against the f16 peak."""
    import torch

    import intent_amd as intent
    from intent_amd.examples.kernels.contraction.gemm import quantized_gemm

    m, k, n = 4096, 4096, 14336
    rng = np.random.default_rng(11)
    a = rng.standard_normal((m, k), np.float32).astype(np.float16)
    b = (rng.standard_normal((k, n), np.float32) / 64).astype(np.float16)
    bias = rng.standard_normal(n, np.float32)
    residual = (4 * rng.standard_normal((m, n), np.float32)).astype(np.float16)
    scale = rng.uniform(0.05, 0.5, n).astype(np.float32)
    dev = lambda x: torch.from_numpy(x).to(device)  # noqa: E731
    call = intent.jit(quantized_gemm, backend="hip").prepare(dev(a), dev(b), dev(bias), dev(residual), dev(scale))
    ms = operator_ms(call.launch, flush)
    flops = 2 * m * n * k
    out = {"config": f"quantized_gemm M={m} K={k} N={n}, f16 operands, int8 output", "median_ms": round(ms, 4),
           "achieved": round(flops / ms / 1e9, 1), "unit": "TFLOP/s",
           "roofline_frac": round(flops / ms / 1e9 / MFMA_PEAK_TFLOPS, 4), "flops": flops}
    if cpu:
        import oracle

        rows, cols = 16, 1024
        b_part, r_part = np.ascontiguousarray(b[:, :cols]), np.ascontiguousarray(residual[:rows, :cols])
        seconds = cpu_median_seconds(lambda: oracle.quantized_gemm(a[:rows], b_part, bias[:cols], r_part,
                                                                   scale[:cols]))
        out["cpu"] = {"tflops": round(2 * rows * cols * k / seconds / 1e12, 5), "cores": 1, "kind": "port",
                      "sample": f"the first {rows} x {cols} block of the output (numpy float64 product)"}
    return out


def op_varlen_prefill(device, flush, cpu):
    """flash_varlen_gqa_prefill: 16 packed sequences of 1..4096 rows (uniform, seed 5), 32 query heads
    over 8 key/value heads, D = 128, causal. FLOPs count each sequence's causal half, as config 4."""
    import torch

    import intent_amd as intent
    from intent_amd.examples import inputs
    from intent_amd.examples.kernels.streaming.attention import flash_varlen_gqa_prefill

    rng = np.random.default_rng(5)
    lengths = rng.integers(1, 4097, 16).astype(np.int32)
    cu = np.concatenate(([0], np.cumsum(lengths))).astype(np.int32)
    total, hq, hk, d = int(cu[-1]), 32, 8, 128
    q = inputs.normal(rng, (total, hq, d), "f16")
    k = inputs.normal(rng, (total, hk, d), "f16")
    v = inputs.normal(rng, (total, hk, d), "f16")
    scale = float(np.float32(1 / np.sqrt(d)))
    dev = lambda a: torch.from_numpy(a).to(device)  # noqa: E731
    call = intent.jit(flash_varlen_gqa_prefill, backend="hip", constexprs={"HEAD_GROUP": hq // hk}).prepare(
        dev(q), dev(k), dev(v), dev(lengths), dev(cu), scale)
    ms = operator_ms(call.launch, flush)
    flops = int(sum(4 * hq * int(n) * int(n) * d // 2 for n in lengths))
    out = {"config": f"causal varlen GQA prefill f16, 16 sequences of 1..4096 rows ({total} in all), HQ{hq} HK{hk} "
                     f"D{d} (flash_varlen_gqa_prefill)", "median_ms": round(ms, 4),
           "achieved": round(flops / ms / 1e9, 1), "unit": "TFLOP/s",
           "roofline_frac": round(flops / ms / 1e9 / MFMA_PEAK_TFLOPS, 4), "flops": flops}
    if cpu:
        import oracle

        first = min(int(lengths[0]), 1024)
        seconds = cpu_median_seconds(lambda: oracle.attention_varlen_fwd(
            np.ascontiguousarray(q[:first, :4]), np.ascontiguousarray(k[:first, :1]),
            np.ascontiguousarray(v[:first, :1]), np.array([0, first], np.int32), scale, True, head_group=4))
        sample_flops = 4 * 4 * first * first * d // 2
        out["cpu"] = {"tflops": round(sample_flops / seconds / 1e12, 5), "cores": oracle.default_workers(),
                      "kind": "port", "sample": f"4 query heads of one key head over the first {first} rows of "
                                                f"the first sequence"}
    return out


def _op_mla_prefill(device, flush, cpu, large):
    """mla_prefill at the reference's extents (streaming/attention.py:35-44): B1, 8 query heads over
    2 key heads, S1024, content D128 and position P64, causal; `large`: config 4's B4 H32 (over 8
    key heads) S4096. FLOPs: the causal half of the score product over D + P and of P @ V over D."""
    import torch

    import intent_amd as intent
    from intent_amd.examples import inputs
    from intent_amd.examples.kernels.streaming.attention import mla_prefill

    rng = np.random.default_rng(15)
    b, h, hk, s, d, p = (4, 32, 8, 4096, 128, 64) if large else (1, 8, 2, 1024, 128, 64)
    arrays = (inputs.normal(rng, (b, h, s, d), "f16"), inputs.normal(rng, (b, h, s, p), "f16"),
              inputs.normal(rng, (b, hk, s, d), "f16"), inputs.normal(rng, (b, 1, s, p), "f16"),
              inputs.normal(rng, (b, hk, s, d), "f16"))
    scale = float(np.float32(1 / np.sqrt(d + p)))
    t = lambda a: torch.from_numpy(a).to(device)  # noqa: E731
    call = intent.jit(mla_prefill, backend="hip", constexprs={"HEAD_GROUP": h // hk}).prepare(
        *(t(a) for a in arrays), scale)
    ms = operator_ms(call.launch, flush)
    flops = b * h * s * s * (2 * (d + p) + 2 * d) // 2
    out = {"config": f"latent attention prefill f16 B{b} H{h} HK{hk} S{s} D{d} P{p}, causal (mla_prefill)",
           "median_ms": round(ms, 4), "achieved": round(flops / ms / 1e9, 1), "unit": "TFLOP/s",
           "roofline_frac": round(flops / ms / 1e9 / MFMA_PEAK_TFLOPS, 4), "flops": flops}
    if large:
        out["traffic"] = read_traffic("mla_prefill_b4_h32_hk8_s4096")
    if cpu:
        import oracle

        if large:
            part = (arrays[0][:1, :4, :1024], arrays[1][:1, :4, :1024], arrays[2][:1, :1, :1024],
                    arrays[3][:1, :, :1024], arrays[4][:1, :1, :1024])
            sample_flops, sample = 4 * 1024 * 1024 * (2 * (d + p) + 2 * d) // 2, "4 query heads of one key head, first 1024 rows"
        else:
            part, sample_flops, sample = arrays, flops, "the whole workload"
        seconds = cpu_median_seconds(lambda: oracle.mla_prefill(*part, scale))
        out["cpu"] = {"tflops": round(sample_flops / seconds / 1e12, 5), "cores": oracle.default_workers(),
                      "kind": "port", "sample": sample}
    return out


def op_mla_prefill(device, flush, cpu):
    return _op_mla_prefill(device, flush, cpu, False)


def op_mla_prefill_large(device, flush, cpu):
    return _op_mla_prefill(device, flush, cpu, True)


def op_attention_bias(device, flush, cpu):
    """flash_attention_bias_fwd at config 4's extents (B4 H32 S4096 D128), every key admitted, with
    a normal(0, 2) f32 bias per (batch, head, key). FLOPs: the two products over all S x S pairs."""
    import torch

    import intent_amd as intent
    from intent_amd.examples import inputs
    from intent_amd.examples.kernels.streaming.attention import flash_attention_bias_fwd

    q, k, v, scale = inputs.attention_f16()
    b, h, s, d = q.shape
    bias = (2.0 * np.random.default_rng(11).standard_normal((b, h, s))).astype(np.float32)
    t = lambda a: torch.from_numpy(a).to(device)  # noqa: E731
    call = intent.jit(flash_attention_bias_fwd, backend="hip").prepare(t(q), t(k), t(v), t(bias), scale)
    ms = operator_ms(call.launch, flush)
    flops = 4 * b * h * s * s * d
    out = {"config": "key-biased attention fwd f16 B4 H32 S4096 D128, no mask (flash_attention_bias_fwd)",
           "median_ms": round(ms, 4), "achieved": round(flops / ms / 1e9, 1), "unit": "TFLOP/s",
           "roofline_frac": round(flops / ms / 1e9 / MFMA_PEAK_TFLOPS, 4), "flops": flops,
           "traffic": read_traffic("attention_bias_config4")}
    if cpu:
        import oracle

        seconds = cpu_median_seconds(lambda: oracle.attention_bias_fwd(
            q[:1, :1, :512], k[:1, :1], v[:1, :1], bias[:1, :1], scale))
        sample_flops = 4 * 512 * s * d
        out["cpu"] = {"tflops": round(sample_flops / seconds / 1e12, 5), "cores": oracle.default_workers(),
                      "kind": "port", "sample": "1 (batch, head) pair, first 512 queries over all 4096 keys"}
    return out


def _op_attention_bwd(device, flush, cpu, large):
    """The three-kernel attention backward (programs/attention_backward.py) as one prepared
    sequence: the reference example's shape (backward/attention.py:7-13: B2, HQ8, HK2, S1024, D64)
    or a large grouped shape (B4, HQ32, HK8, S4096, D128); causal."""
    import torch

    import intent_amd as intent
    from intent_amd.examples import inputs
    from intent_amd.examples.programs.attention_backward import AttentionBackward

    b, hq, hk, s, d = (4, 32, 8, 4096, 128) if large else (2, 8, 2, 1024, 64)
    rng = np.random.default_rng(3)
    q = inputs.normal(rng, (b, hq, s, d), "f16")
    k = inputs.normal(rng, (b, hk, s, d), "f16")
    v = inputs.normal(rng, (b, hk, s, d), "f16")
    o = inputs.normal(rng, (b, hq, s, d), "f16")
    do = inputs.normal(rng, (b, hq, s, d), "f16")
    lse = (rng.standard_normal((b, hq, s)) * 0.5 + np.log(s)).astype(np.float32)
    scale = float(np.float32(1 / np.sqrt(d)))
    t = lambda a: torch.from_numpy(a).to(device)  # noqa: E731
    program = AttentionBackward.from_jit(lambda defn, **kw: intent.jit(defn, backend="hip", **kw),
                                         head_group=hq // hk, causal=True)
    call = program.prepare(t(q), t(k), t(v), t(o), t(do), t(lse), scale)
    ms = operator_ms(call.launch, flush)
    flops = 14 * b * hq * s * s * d // 2          # dQ: 3 products, dK/dV: 4 products, causal half
    out = {"config": f"causal attention backward f16 B{b} HQ{hq} HK{hk} S{s} D{d} (delta + dK/dV + dQ)",
           "median_ms": round(ms, 4), "achieved": round(flops / ms / 1e9, 1), "unit": "TFLOP/s",
           "roofline_frac": round(flops / ms / 1e9 / MFMA_PEAK_TFLOPS, 4), "flops": flops}
    if cpu:
        import oracle

        n = 512
        qs, ks, vs = (np.ascontiguousarray(a[:1, :1, :n]) for a in (q, k, v))
        os_, dos = np.ascontiguousarray(o[:1, :1, :n]), np.ascontiguousarray(do[:1, :1, :n])
        ls = np.ascontiguousarray(lse[:1, :1, :n])

        def run():
            delta = oracle.attention_bwd_delta(os_, dos)
            oracle.attention_bwd_dq(qs, ks, vs, dos, ls, delta, scale, True)
            oracle.attention_bwd_dkdv(qs, ks, vs, dos, ls, delta, scale, True)

        seconds = cpu_median_seconds(run)
        out["cpu"] = {"tflops": round(14 * n * n * d / 2 / seconds / 1e12, 5), "cores": oracle.default_workers(),
                      "kind": "port", "sample": f"one head, first {n} queries and keys"}
    return out


def op_attention_bwd(device, flush, cpu):
    return _op_attention_bwd(device, flush, cpu, False)


def op_attention_bwd_large(device, flush, cpu):
    return _op_attention_bwd(device, flush, cpu, True)


def op_paged_decode(device, flush, cpu):
    """Split-K paged grouped-query decode (programs/composition.py PagedDecode: partials + merge)
    at the paged_attention.py constants: B8, HQ32, HK8, D128, 64-token pages, 16 splits, sequence
    lengths 8191..6413, each sequence owning ceil(length / 64) shuffled pages."""
    import torch

    import intent_amd as intent
    from intent_amd.examples import inputs
    from intent_amd.examples.programs.composition import PagedDecode

    arrays = inputs.paged_decode(seed=4, layout="exact")
    q, key_cache, value_cache, page_offsets, page_indices, lengths, split_offsets = arrays
    batch, hq, d = q.shape
    hk, splits, page_size = key_cache.shape[2], 16, 64
    scale = float(np.float32(1 / np.sqrt(d)))
    t = lambda a: torch.from_numpy(a).to(device)  # noqa: E731
    program = PagedDecode.from_jit(lambda defn, **kw: intent.jit(defn, backend="hip", **kw), page_size=page_size,
                                   head_group=hq // hk, splits=splits)
    call = program.prepare(*(t(a) for a in arrays), scale)
    ms = operator_ms(call.launch, flush)
    partials, merge = call.calls
    partial_ms, merge_ms = sequence_kernel_ms(partials.launch, merge.launch, 50)
    tokens = int(lengths.astype(np.int64).sum())
    kv_bytes = tokens * hk * 2 * d * 2                       # K and V rows of every active token
    partial_bytes = batch * hq * splits * (d + 1) * 4          # written by the partials, read by the merge
    nbytes = kv_bytes + batch * hq * d * 2 + 2 * partial_bytes + batch * hq * d * 2 + 4 * (
        page_offsets.size + page_indices.size + lengths.size + split_offsets.size)
    out = {"config": f"paged GQA decode f16 B{batch} HQ{hq} HK{hk} D{d} page 64, {splits} splits, "
                     f"{tokens} cached tokens (partials + split-K merge)",
           "median_ms": round(ms, 4), "achieved": round(nbytes / ms / 1e6, 1), "unit": "GB/s",
           "roofline_frac": round(nbytes / ms / 1e6 / HBM_PEAK_GBS, 4), "bytes": nbytes,
           "partials_ms": round(partial_ms, 4), "merge_ms": round(merge_ms, 4),
           "partials_gbs": round((kv_bytes + partial_bytes) / partial_ms / 1e6, 1),
           "traffic": read_traffic("paged_decode_partials_b8_hq32_hk8_d128")}
    if cpu:
        import oracle

        def run():
            lse, part = oracle.paged_decode_partials(*arrays, scale, page_size=page_size, head_group=hq // hk,
                                                     splits=splits)
            oracle.splitk_reduce_f32_to_f16(part, lse)

        seconds = cpu_median_seconds(run)
        out["cpu"] = {"gbs": round(nbytes / seconds / 1e9, 3), "cores": oracle.default_workers(), "kind": "port",
                      "sample": "the whole workload"}
    return out


def op_continuous_decode(device, flush, cpu):
    """continuous_gqa_decode at the reference's GQA decode constants (streaming/attention.py:28-34):
    B32, HQ32 over HK8, K8192, D128, token-major f16 caches, every key admitted. HBM bytes: the K and
    V caches, the mask, q and the output, plus the split states written and read back."""
    import torch

    import intent_amd as intent
    from intent_amd.examples.kernels.streaming.attention import continuous_gqa_decode

    batch, hq, hk, keys, d = 32, 32, 8, 8192, 128
    generator = torch.Generator(device=device).manual_seed(12)     # 1 GiB of cache: drawn on the device
    draw = lambda shape: torch.randn(shape, generator=generator, device=device).to(torch.float16)  # noqa: E731
    q, k, v = draw((batch, hq, d)), draw((batch, keys, hk, d)), draw((batch, keys, hk, d))
    mask = torch.ones((batch, keys, hk), dtype=torch.uint8, device=device)
    scale = float(np.float32(1 / np.sqrt(d)))
    call = intent.jit(continuous_gqa_decode, backend="hip", constexprs={"HEAD_GROUP": hq // hk}).prepare(
        q, k, v, mask, scale)
    ms = operator_ms(call.launch, flush)
    splits = 8                                   # 2048 workgroups: 1024 keys per split at this shape
    state = batch * hq * splits * (d + 2) * 4
    nbytes = 2 * k.numel() * 2 + mask.numel() + q.numel() * 2 + batch * hq * d * 2 + 2 * state
    out = {"config": f"continuous GQA decode f16 B{batch} HQ{hq} HK{hk} K{keys} D{d}, token-major caches, all keys "
                     f"admitted (continuous_gqa_decode: partials + merge)",
           "median_ms": round(ms, 4), "achieved": round(nbytes / ms / 1e6, 1), "unit": "GB/s",
           "roofline_frac": round(nbytes / ms / 1e6 / HBM_PEAK_GBS, 4), "bytes": nbytes,
           "traffic": read_traffic("continuous_decode_partials_b32_hq32_hk8_k8192_d128")}
    if cpu:
        import oracle

        host = [a[:4].cpu().numpy() for a in (q, k, v, mask)]
        seconds = cpu_median_seconds(lambda: oracle.continuous_gqa_decode(*host, scale))
        out["cpu"] = {"gbs": round(nbytes / 8 / seconds / 1e9, 3), "cores": oracle.default_workers(), "kind": "port",
                      "sample": "the first 4 of the 32 batch rows"}
    return out


def op_grouped_decode(device, flush, cpu):
    """grouped_flash_decode_partials at the same constants in bf16 (head-major caches [B,HK,K,D]),
    P = 8 parts of SPLIT_SIZE 1024. HBM bytes: the K and V caches, q and the partials written."""
    import torch

    import intent_amd as intent
    from intent_amd.examples.kernels.streaming.attention import grouped_flash_decode_partials

    batch, hq, hk, keys, d, parts = 32, 32, 8, 8192, 128, 8
    generator = torch.Generator(device=device).manual_seed(13)
    draw = lambda shape: torch.randn(shape, generator=generator, device=device).to(torch.bfloat16)  # noqa: E731
    q, k, v = draw((batch, hq, 1, d)), draw((batch, hk, keys, d)), draw((batch, hk, keys, d))
    scale = float(np.float32(1 / np.sqrt(d)))
    call = intent.jit(grouped_flash_decode_partials, backend="hip",
                      constexprs={"HEAD_GROUP": hq // hk, "P": parts, "SPLIT_SIZE": keys // parts}).prepare(
        q, k, v, scale)
    ms = operator_ms(call.launch, flush)
    nbytes = 2 * k.numel() * 2 + q.numel() * 2 + batch * hq * parts * (d * 2 + 4)
    out = {"config": f"grouped flash decode partials bf16 B{batch} HQ{hq} HK{hk} K{keys} D{d}, P{parts} x "
                     f"{keys // parts} (grouped_flash_decode_partials)",
           "median_ms": round(ms, 4), "achieved": round(nbytes / ms / 1e6, 1), "unit": "GB/s",
           "roofline_frac": round(nbytes / ms / 1e6 / HBM_PEAK_GBS, 4), "bytes": nbytes,
           "traffic": read_traffic("grouped_decode_partials_b32_hq32_hk8_k8192_d128")}
    if cpu:
        import oracle

        host = [a[:4].float().cpu().numpy() for a in (q, k, v)]
        bf = [oracle.float_to_bf16_bits(a) for a in host]
        seconds = cpu_median_seconds(lambda: oracle.grouped_decode_partials(*bf, scale, parts=parts,
                                                                            split_size=keys // parts))
        out["cpu"] = {"gbs": round(nbytes / 8 / seconds / 1e9, 3), "cores": oracle.default_workers(), "kind": "port",
                      "sample": "the first 4 of the 32 batch rows"}
    return out


def op_varlen_decode(device, flush, cpu):
    """varlen_gqa_decode_with_sink_logits at the reference's constants (streaming/attention.py:18-27):
    8 packed sequences of 1..4096 keys (uniform, seed 14), HQ32 over HK8, D64, MAX_BLOCKS 64."""
    import torch

    import intent_amd as intent
    from intent_amd.examples import inputs
    from intent_amd.examples.kernels.streaming.attention import varlen_gqa_decode_with_sink_logits

    rng = np.random.default_rng(14)
    lengths = rng.integers(1, 4097, 8)
    cu = np.concatenate(([0], np.cumsum(lengths))).astype(np.int32)
    batch, hq, hk, d, rows = 8, 32, 8, 64, int(cu[-1])
    q = inputs.normal(rng, (batch, hq, d), "f16")
    k, v = inputs.normal(rng, (rows, hk, d), "f16"), inputs.normal(rng, (rows, hk, d), "f16")
    sink = rng.uniform(0.0, 2.0, hq).astype(np.float32)
    scale = float(np.float32(1 / np.sqrt(d)))
    t = lambda a: torch.from_numpy(a).to(device)  # noqa: E731
    call = intent.jit(varlen_gqa_decode_with_sink_logits, backend="hip",
                      constexprs={"HEAD_GROUP": hq // hk, "MAX_BLOCKS": 64}).prepare(
        t(q), t(k), t(v), t(cu), t(sink), scale)
    ms = operator_ms(call.launch, flush)
    nbytes = 2 * k.nbytes + q.nbytes + batch * hq * d * 2 + batch * hq * 64 * 4 * 2
    out = {"config": f"packed GQA decode with sink and block logits f16, {batch} sequences of 1..4096 keys ({rows} "
                     f"rows), HQ{hq} HK{hk} D{d} (varlen_gqa_decode_with_sink_logits)",
           "median_ms": round(ms, 4), "achieved": round(nbytes / ms / 1e6, 1), "unit": "GB/s",
           "roofline_frac": round(nbytes / ms / 1e6 / HBM_PEAK_GBS, 4), "bytes": nbytes,
           "traffic": read_traffic("varlen_decode_partials_8x1to4096_hq32_hk8_d64")}
    if cpu:
        import oracle

        seconds = cpu_median_seconds(lambda: oracle.varlen_decode_sink(q, k, v, cu, sink, scale, max_blocks=64))
        out["cpu"] = {"gbs": round(nbytes / seconds / 1e9, 3), "cores": oracle.default_workers(), "kind": "port",
                      "sample": "the whole workload"}
    return out


def op_spmm(device, flush, cpu):
    """csr_spmm at the sparse/csr_spmm.py:5-9 constants: 8192 x 8192, 32 nonzeros per row, 128 f32
    features. The dense operand (4 MB) is re-read per nonzero from L2/MALL; algorithmic HBM bytes
    are the CSR arrays, dense once and the output."""
    import torch

    import intent_amd as intent
    from intent_amd.examples import inputs
    from intent_amd.examples.kernels.sparse.csr_spmm import csr_spmm

    offsets, columns, values, dense = inputs.csr_spmm()
    t = lambda a: torch.from_numpy(a).to(device)  # noqa: E731
    call = intent.jit(csr_spmm, backend="hip").prepare(t(offsets), t(columns), t(values), t(dense))
    ms = operator_ms(call.launch, flush)
    rows, nnz = offsets.shape[0] - 1, int(offsets[-1])
    cols, features = dense.shape
    nbytes = 4 * (rows + 1) + 8 * nnz + 4 * cols * features + 4 * rows * features
    gathered = 4 * nnz * features
    out = {"config": f"CSR SpMM f32 {rows}x{cols}, {nnz} nnz (32 per row), {features} features",
           "median_ms": round(ms, 4), "achieved": round(nbytes / ms / 1e6, 1), "unit": "GB/s",
           "roofline_frac": round(nbytes / ms / 1e6 / HBM_PEAK_GBS, 4), "bytes": nbytes,
           "gathered_gbs": round(gathered / ms / 1e6, 1), "gflops": round(2 * nnz * features / ms / 1e6, 1),
           "traffic": read_traffic("csr_spmm_8192_f128")}
    if cpu:
        import oracle

        seconds = cpu_median_seconds(lambda: oracle.csr_spmm(offsets, columns, values, dense))
        out["cpu"] = {"gbs": round(nbytes / seconds / 1e9, 3), "cores": oracle.default_workers(), "kind": "port",
                      "sample": "the whole workload"}
    return out


OPERATORS = {"softmax_f32": op_softmax_f32, "gemm": op_gemm, "attention": op_attention, "spmv": op_spmv,
             "gemm_f16_relu": op_gemm_f16_relu, "gemm_f32": op_gemm_f32, "linear_f32": op_linear_f32,
             "gqa": op_gqa, "attention_bf16": op_attention_bf16, "attention_bwd": op_attention_bwd,
             "attention_bwd_large": op_attention_bwd_large, "paged_decode": op_paged_decode,
             "spmm": op_spmm, "varlen_prefill": op_varlen_prefill, "gemm_i8": op_gemm_i8,
             "quantized_gemm": op_quantized_gemm, "attention_bias": op_attention_bias,
             "continuous_decode": op_continuous_decode, "grouped_decode": op_grouped_decode,
             "varlen_decode": op_varlen_decode, "mla_prefill": op_mla_prefill,
             "mla_prefill_large": op_mla_prefill_large}


def read_traffic(name):
    """HBM bytes per launch measured with rocprofv3 --pmc (FETCH_SIZE + WRITE_SIZE, scaled by a
    copy-kernel calibration), recorded in profiles/<name>.traffic.txt as `traffic_bytes: N`."""
    path = ROOT / "profiles" / f"{name}.traffic.txt"
    if not path.exists():
        return None
    for line in path.read_text().splitlines():
        if line.startswith("traffic_bytes:"):
            return int(float(line.split(":", 1)[1]))
    return None


def main():
    args = parse()
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print("bench.py measures one GPU only: this build has no multi-GPU path "
              "(softmax, SpMV and attention would shard by rows or (batch, head) with no exchange, "
              "the GEMM by M-panels of A with B replicated)", file=sys.stderr)
        sys.exit(2)
    import numpy as np
    import torch

    if args.copy_calibration:
        src = torch.ones(512 << 20, dtype=torch.uint8, device="cuda:0")
        dst = torch.empty_like(src)
        for _ in range(20):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"copy_calibration": {"bytes_read": src.numel(), "bytes_written": dst.numel(),
                                               "launches": 20}}), flush=True)
        return
    if args.only == "box":
        import intent_amd  # noqa: F401

        device = torch.device("cuda", 0)
        print(json.dumps(box_reference(device, Flush(device))), flush=True)
        return
    if args.only == "sdpa":
        device = torch.device("cuda", 0)
        print(json.dumps(box_sdpa(device, Flush(device))), flush=True)
        return
    if args.only in OPERATORS:
        import intent_amd  # noqa: F401

        device = torch.device("cuda", 0)
        print(json.dumps(OPERATORS[args.only](device, Flush(device), False)), flush=True)
        return

    import intent_amd as intent
    from intent_amd.examples import inputs
    from intent_amd.examples.kernels.backward.softmax import softmax_backward_f16
    from intent_amd.examples.kernels.normalization.softmax import stable_softmax_f16

    device = torch.device("cuda", 0)
    rows, cols = 16384, 4096
    log("generating config 2 inputs")
    x_host, dy_host = inputs.softmax_f16_fwd_bwd(seed=0, rows=rows, cols=cols)
    x, dy = torch.from_numpy(x_host).to(device), torch.from_numpy(dy_host).to(device)
    fwd = intent.jit(stable_softmax_f16, backend="hip").prepare(x)
    bwd = intent.jit(softmax_backward_f16, backend="hip").prepare(fwd.result(), dy)

    def step():
        fwd.launch()
        bwd.launch()

    if args.only in ("softmax_fwd", "softmax_bwd"):
        fwd_ms, bwd_ms = sequence_kernel_ms(fwd.launch, bwd.launch, max(args.steps, 5))
        print(json.dumps({"kernel": args.only, "fwd_ms": fwd_ms, "bwd_ms": bwd_ms}), flush=True)
        return
    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    # Timed steps: K eager steps (prepared fwd and bwd launches, the surface's normal mode) between
    # HIP events on the launch stream, after W untimed warm-up steps.
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    for _ in range(args.steps):
        step()
    end.record()
    end.synchronize()
    ms_per_step = start.elapsed_time(end) / args.steps
    # The same step captured once in a hipGraph and replayed K times (the reference's GPU protocol
    # captures its call in a graph, runtime/triton/cuda.py:18-44), reported beside it.
    graph = torch.cuda.CUDAGraph()
    capture = torch.cuda.Stream()
    capture.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(capture):
        with torch.cuda.graph(graph, stream=capture):
            step()
    torch.cuda.current_stream().wait_stream(capture)
    for _ in range(args.warmup):
        graph.replay()
    torch.cuda.synchronize()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    for _ in range(args.steps):
        graph.replay()
    end.record()
    end.synchronize()
    torch.cuda.synchronize()
    graph_ms = start.elapsed_time(end) / args.steps
    fwd_bytes = FWD_BYTES_PER_ELEMENT * rows * cols
    bwd_bytes = BWD_BYTES_PER_ELEMENT * rows * cols
    value = (fwd_bytes + bwd_bytes) / ms_per_step / 1e6
    log(f"fwd+bwd step {ms_per_step:.4f} ms (eager; graph replay {graph_ms:.4f} ms) -> {value:.1f} GB/s")

    fwd_ms, bwd_ms = sequence_kernel_ms(fwd.launch, bwd.launch, max(args.steps, 20))
    achieved = bwd_bytes / bwd_ms / 1e6
    roofline = {"bound": "hbm", "kernel": "softmax_bwd_wave<f16,8,8> (softmax_backward_f16)",
                "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": read_traffic("softmax_bwd_f16_16384x4096"),
                "avg_launch_ms": round(bwd_ms, 5), "algorithmic_bytes": bwd_bytes,
                "fwd_kernel": {"avg_launch_ms": round(fwd_ms, 5), "achieved": round(fwd_bytes / fwd_ms / 1e6, 1),
                               "frac": round(fwd_bytes / fwd_ms / 1e6 / HBM_PEAK_GBS, 4),
                               "traffic": read_traffic("softmax_fwd_f16_16384x4096")}}
    log(f"bwd kernel {bwd_ms:.4f} ms ({achieved:.1f} GB/s), fwd kernel {fwd_ms:.4f} ms")
    # The same backward launch cold: a 512 MiB write-then-read flush of the MALL before each call, so
    # y and dy come from HBM rather than from the MALL lines the forward just wrote.
    cold_ms = operator_ms(bwd.launch, Flush(device))
    roofline["cold_backward"] = {"avg_launch_ms": round(cold_ms, 5), "achieved": round(bwd_bytes / cold_ms / 1e6, 1),
                                 "frac": round(bwd_bytes / cold_ms / 1e6 / HBM_PEAK_GBS, 4),
                                 "timing": "median of cold calls, 512 MiB flush before each"}
    log(f"bwd kernel cold {cold_ms:.4f} ms ({bwd_bytes / cold_ms / 1e6:.1f} GB/s)")

    operators = []
    if not args.no_operators:
        flush = Flush(device)
        for name in [n for n in args.operators.split(",") if n]:
            log(f"operator {name}")
            try:
                _LAST_CPU_ALL.clear()
                operators.append(OPERATORS[name](device, flush, not args.no_cpu_baseline))
                attach_all_cores(operators[-1])
                operator_graph_ms = _LAST_GRAPH_MS.pop("graph_ms", None)
                if operator_graph_ms is not None:
                    operators[-1]["graph_ms"] = round(operator_graph_ms, 5)
            except intent.CompilationStageError as error:
                operators.append({"config": name, "status": "unsupported", "error": str(error)})
            log(json.dumps(operators[-1]))
            torch.cuda.empty_cache()

    reference = None
    if not args.no_operators:
        log("box reference figures")
        reference = box_reference(device, Flush(device))
        torch.cuda.empty_cache()
        # Matrix operators also read against the MFMA rate this box sustains (the probe), beside
        # the published dense peak their roofline_frac uses.
        sustained = {"bf16": reference.get("mfma_bf16_probe_tflops"), "f16": reference.get("mfma_f16_probe_tflops")}
        for op in operators:
            config = op.get("config", "")
            if op.get("unit") == "TFLOP/s" and "achieved" in op and "f32" not in config.split(",")[0]:
                peak = sustained["bf16"] if "bf16" in config else sustained["f16"]
                if peak:
                    op["frac_of_box_mfma"] = round(op["achieved"] / peak, 4)

    cpu_baseline = None
    if not args.no_cpu_baseline:
        log("cpu baseline")
        cpu_baseline = headline_cpu_baseline(x_host, dy_host)

    record = {
        "metric": METRIC, "value": round(value, 1), "unit": "GB/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(ms_per_step, 5), "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "f16", "data": "synthetic",
        "config": {"workload": "softmax fwd+bwd f16 storage / f32 math, 16384x4096, x ~ N(0,1)*3, dy ~ N(0,1), "
                               "seed 0 (BASELINE config 2)", "rows": rows, "cols": cols,
                   "bytes_per_step": fwd_bytes + bwd_bytes, "parallelism": "single GPU",
                   "timing": "K eager steps (prepared fwd + bwd launches) between HIP events after W warm-ups",
                   "graph_ms_per_step": round(graph_ms, 5)},
        "roofline": roofline, "cpu_baseline": cpu_baseline, "operators": operators, "box_reference": reference,
    }
    print(json.dumps(record), flush=True)
    del np


if __name__ == "__main__":
    main()
