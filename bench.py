#!/usr/bin/env python3
"""Benchmark of the custom-op hot path on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu-baseline] [--quick]
                    [--configs 1,ceiling,reference,2,reduce,3,4,5,paged,tensorcore,fp8]

Prints ONE JSON line (the driver's contract). The workload behind `value` is
BASELINE.json's configs[1] - the memory-bound pair RMSNorm bf16 [16384, 4096]
(eps 1e-6, weight ~N(1, 0.02)) + causal-masked row softmax bf16 [1024, 2048]
(logits ~N(0, 4)) - and one step is one pass of both kernels over one buffer
set. `value` is the step's algorithmic bytes (read + write once) over its
wall time, with inputs resident in HBM; buffer sets rotate so the working set
(>= 1 GiB) exceeds the 256 MB Infinity Cache and every step reads from HBM.

`roofline` is the dominant kernel of the step (RMSNorm): algorithmic bytes per
launch over its average duration during the timed steps (every 8th launch),
against 8 TB/s. The duration comes from HIP events that the RMSNorm dispatch
itself records
(cf_time_next_launch -> hipExtLaunchKernel with start/stop events on the
launch stream): the kernel's own start and end timestamps, the figure a
rocprofv3 kernel trace reports, with no event packets queued around the
launch (an event pair around it also times the dispatch and completion
packets, ~2.5 us on a 45 us kernel). `traffic` is the HBM bytes
per launch from the rocprofv3 FETCH_SIZE/WRITE_SIZE summary committed under
profiles/ (null when absent). `cpu_baseline` times the reference's own CPU
operators (oracle/_ref, built from the reference source) on the same step,
each op for about --cpu-seconds of CPU work, on this host's cores.

The stdout line stays under 4 KB: besides the contract's fields it carries
`configs`, a few figures per configuration (C1 quantise/dequantise GB/s from
back-to-back launches, C2 RMSNorm GB/s from the kernels' own timestamps and the
softmax's microseconds per launch from a replayed HIP graph of back-to-back
launches, C3 fused LoRA TFLOP/s from its kernels' timestamps, its and
hipBLASLt's plain GEMM's microseconds per launch from back-to-back launches
(the same method for both), and the adapter backward GB/s, C4 tokens/s,
C5 aggregate GB/s). The full breakdown goes to the `--detail` file
(gpurun_out/bench_detail.json by default) and nowhere else.

`breakdown` reports every other configuration (`--configs` selects them):
median over 5 batches of back-to-back launches timed by HIP events, after at
least 0.3 s of warm-up, with cache-cold rotation (`median_ms`: launch-to-launch
time, which for kernels of a few microseconds is the host's launch rate), and
the median of 25 calls timed by their kernels' own start/end timestamps
(from the first kernel's start to the last one's end), launched back to back
(`kernel_median_ms`, the kernel-trace figure; `kernel_frac_*` is computed from
it): config 1
quantise/dequantise, `ceiling` the same two kernels and the streaming ceilings
of their traffic (read-only 64 MiB, write-only 16 MiB, both, a copy) launched
back to back over 2.6 GB of rotating buffers, `reference` every kernel the
reference publishes a figure for at its own benchmark shape (fp32, with the
reference's RTX 3090 figure beside it), config 2 per kernel, config 3 fused LoRA TFLOP/s (with
hipBLASLt's plain GEMM through torch for context) and its adapter backward,
`reduce` the two-stage sum (16M and 256M fp32) and per-row sums,
config 4 the Llama block forward (tokens/s end to end, per-operator event
times and TFLOP/s), `paged` the paged-attention decode at the reference's
benchmark shapes, `tensorcore` the fp32 matmul on the bf16 MFMA units, `fp8`
the fp8 MFMA matmul (with hipBLASLt's fp8 GEMM for context), config 5 bulk 7B
quantise/dequantise aggregate GB/s, and a plain copy's achieved bandwidth.
"""

from __future__ import annotations

import argparse
import json
import os
import re
import statistics
import subprocess
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

PEAK_HBM_GBS = 8000.0          # MI355X HBM3E
PEAK_BF16_TFLOPS = 2500.0      # dense bf16 MFMA
PEAK_FP8_TFLOPS = 5000.0       # dense fp8 MFMA
PEAK_FP32_TFLOPS = 157.3       # fp32 (the fp32 LoRA rows' reference point; they run as 3 bf16 MFMA products)
SUM_SINGLE_LAUNCH_BYTES = 256 * 1024  # cf_reduce_sum: one launch up to this input size
KERNEL_SAMPLES = 25            # breakdown: dispatches timed by their own timestamps
TIMER_STRIDE = 8               # main step: every 8th RMSNorm dispatch is timed
METRIC = "INT8 quant/RMSNorm/softmax GB/s (% HBM peak); fused LoRA-linear TFLOP/s"
CACHE_FLUSH_BYTES = 1 << 30    # rotate buffer sets until they exceed this


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


# ---------------------------------------------------------------------------
# Byte and FLOP models (algorithmic: each operand read once, each result
# written once; never cache re-reads).
# ---------------------------------------------------------------------------


def bytes_quant(n: int, in_size: int) -> int:
    return n * in_size + n + ((n + 63) // 64) * 4


def bytes_dequant(n: int, out_size: int) -> int:
    return n + ((n + 63) // 64) * 4 + n * out_size


def bytes_rmsnorm(rows: int, cols: int, size: int) -> int:
    return 2 * rows * cols * size + cols * size


def bytes_softmax(rows: int, cols: int, size: int) -> int:
    return 2 * rows * cols * size


def flops_lora(m: int, k: int, n: int, r: int) -> int:
    return 2 * m * k * n + 2 * m * k * r + 2 * m * r * n


# ---------------------------------------------------------------------------
# Timing helpers.
# ---------------------------------------------------------------------------


def sets_for(bytes_per_set: int, minimum: int = 2) -> int:
    return max(minimum, -(-CACHE_FLUSH_BYTES // max(bytes_per_set, 1)))


WARMUP_SECONDS = 0.3


def warm(torch, launches, warmup: int) -> None:
    """At least `warmup` launches and WARMUP_SECONDS of them, so the clocks
    have ramped before anything is timed."""
    started = time.perf_counter()
    i = 0
    while i < warmup or time.perf_counter() - started < WARMUP_SECONDS:
        launches[i % len(launches)]()
        i += 1
        if i % 16 == 0:
            torch.cuda.synchronize()
    torch.cuda.synchronize()


def time_launches(torch, launches, warmup: int, runs: int, batches: int = 5) -> list[float]:
    """Average launch duration (ms) of each of `batches` back-to-back batches
    of `runs` launches cycling over `launches`, timed by HIP events on the
    current stream (per-launch events would add their own overhead to short
    kernels)."""
    warm(torch, launches, warmup)
    out = []
    for _ in range(batches):
        start = torch.cuda.Event(enable_timing=True)
        stop = torch.cuda.Event(enable_timing=True)
        start.record()
        for i in range(runs):
            launches[i % len(launches)]()
        stop.record()
        torch.cuda.synchronize()
        out.append(start.elapsed_time(stop) / runs)
    return out


def graph_times(torch, launches, runs: int, batches: int = 5) -> list[float]:
    """Average launch duration (ms) of `runs` launches cycling over `launches`,
    captured once into a HIP graph and replayed `batches` times, each replay
    timed by HIP events: dispatches back to back with no host launch loop in
    between, for kernels shorter than the host's launch rate. Only for entry
    points that enqueue kernels and nothing else (no memset, no allocation)."""
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        for i in range(runs):
            launches[i % len(launches)]()
    out = []
    for i in range(batches + 2):  # two untimed replays first
        start = torch.cuda.Event(enable_timing=True)
        stop = torch.cuda.Event(enable_timing=True)
        start.record()
        graph.replay()
        stop.record()
        torch.cuda.synchronize()
        if i >= 2:
            out.append(start.elapsed_time(stop) / runs)
    del graph
    return out


def kernel_times(torch, cf, launches, count: int = KERNEL_SAMPLES) -> list[float]:
    """Execution time (ms) of `count` dispatches, cycling over `launches`,
    each timed by the start/end timestamps of its own dispatch
    (cf_time_next_launch), launched back to back. For kernels of ~15 us or
    less the median can read 10-30% long on some runs (the Python launch loop
    then falls behind the GPU and some dispatches start from an idle queue);
    the kernel-trace averages in profiles/ are the reference figures there.
    An entry point of several kernels is timed from its first kernel's start
    to its last kernel's end."""
    timers = [cf._lib.DispatchTimer() for _ in range(count)]
    torch.cuda.synchronize()
    for i, timer in enumerate(timers):
        timer.arm()
        launches[i % len(launches)]()
    torch.cuda.synchronize()
    samples = [timer.elapsed_ms() for timer in timers]
    for timer in timers:
        timer.close()
    return samples


def with_kernel_time(torch, cf, entry: dict, launches, nbytes: int | None = None,
                     flops: int | None = None, peak: float | None = None) -> dict:
    """Add the dispatch-timestamp median (and the rate it gives) to `entry`."""
    ms = statistics.median(kernel_times(torch, cf, launches))
    entry["kernel_median_ms"] = ms
    if nbytes is not None:
        entry["kernel_GB/s"] = gbs(nbytes, ms)
        entry["kernel_frac_hbm"] = gbs(nbytes, ms) / PEAK_HBM_GBS
    if flops is not None:
        tflops = flops / (ms * 1e-3) / 1e12
        entry["kernel_TFLOP/s"] = tflops
        entry["kernel_frac_peak"] = tflops / peak
    return entry


def summary(samples_ms: list[float]) -> dict:
    ordered = sorted(samples_ms)
    return {
        "median_ms": statistics.median(ordered),
        "mean_ms": statistics.fmean(ordered),
        "min_ms": ordered[0],
        "p95_ms": ordered[min(int(0.95 * len(ordered)), len(ordered) - 1)],
    }


def gbs(nbytes: int, ms: float) -> float:
    return nbytes / (ms * 1e-3) / 1e9


# ---------------------------------------------------------------------------
# Synthetic inputs (seeded, generated on the GPU).
# ---------------------------------------------------------------------------


def make_rmsnorm_set(torch, gen, rows, cols, dtype):
    x = torch.randn(rows, cols, generator=gen, device="cuda").to(dtype)
    return x, torch.empty_like(x)


def make_causal_logits(torch, gen, rows, cols, dtype):
    x = 2.0 * torch.randn(rows, cols, generator=gen, device="cuda")
    col = torch.arange(cols, device="cuda")[None, :]
    row = (torch.arange(rows, device="cuda") % cols)[:, None]
    x = x.masked_fill(col > row, float("-inf"))
    return x.to(dtype), torch.empty(rows, cols, dtype=dtype, device="cuda")


def with_outliers(torch, gen, x, fraction: float, factor: float):
    flat = x.view(-1)
    count = int(flat.numel() * fraction)
    idx = torch.randint(0, flat.numel(), (count,), generator=gen, device="cuda")
    flat[idx] *= factor
    return x


# ---------------------------------------------------------------------------
# Benchmarks.
# ---------------------------------------------------------------------------


def bench_main_step(torch, cf, steps: int, warmup: int) -> dict:
    """RMSNorm bf16 [16384, 4096] + causal softmax bf16 [1024, 2048]."""
    gen = torch.Generator(device="cuda").manual_seed(2)
    rows, cols = 16384, 4096
    s_rows, s_cols = 1024, 2048
    dtype = torch.bfloat16
    w = (1 + 0.02 * torch.randn(cols, generator=gen, device="cuda")).to(dtype)
    rms_bytes = bytes_rmsnorm(rows, cols, 2)
    sm_bytes = bytes_softmax(s_rows, s_cols, 2)
    nsets = sets_for(rms_bytes + sm_bytes, minimum=4)
    sets = []
    for _ in range(nsets):
        x, y = make_rmsnorm_set(torch, gen, rows, cols, dtype)
        lx, ly = make_causal_logits(torch, gen, s_rows, s_cols, dtype)
        sets.append((x, y, lx, ly))
    lib = cf._lib.load()
    CF_BF16 = cf._lib.CF_BF16

    def step(i: int, timer=None):
        x, y, lx, ly = sets[i % nsets]
        stream = torch.cuda.current_stream().cuda_stream
        if timer is not None:
            timer.arm()
        cf._lib.check(lib.cf_rmsnorm(x.data_ptr(), w.data_ptr(), y.data_ptr(), CF_BF16, rows, cols, 1e-6, stream))
        cf._lib.check(lib.cf_softmax(lx.data_ptr(), CF_BF16, ly.data_ptr(), CF_BF16, s_rows, s_cols, stream))

    # The untimed warm-up: at least `warmup` steps and WARMUP_SECONDS of them,
    # so the clocks have ramped before the timed steps (a step timed from an
    # idle GPU reads several percent slow).
    warm(torch, [lambda i=i: step(i) for i in range(nsets)], warmup)
    # Every TIMER_STRIDE-th RMSNorm launch of the timed region records its
    # own start and end timestamps on an event pair (cf_time_next_launch):
    # no extra packets enter the queue. A timed dispatch still costs its step
    # ~1.9 us of completion bookkeeping on MI355X, hence the sampling.
    timers = {i: cf._lib.DispatchTimer() for i in range(0, steps, TIMER_STRIDE)}
    torch.cuda.synchronize()
    started = time.perf_counter()
    for i in range(steps):
        step(i, timers.get(i))
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - started
    rms_ms = [timer.elapsed_ms() for timer in timers.values()]
    for timer in timers.values():
        timer.close()
    ms_per_step = elapsed * 1e3 / steps
    rms_avg = statistics.fmean(rms_ms)
    return {
        "ms_per_step": ms_per_step,
        "bytes_per_step": rms_bytes + sm_bytes,
        "rmsnorm_bytes": rms_bytes,
        "rmsnorm_avg_ms": rms_avg,
        "rmsnorm_median_ms": statistics.median(rms_ms),
        "buffer_sets": nsets,
    }


def bench_quant(torch, cf, warmup: int, runs: int) -> dict:
    """config 1: quantise fp32 [4096, 4096] (1% outliers x20), then dequantise; with the
    streaming ceiling of the quantiser's traffic mix (cf_stream_bytes) for context."""
    gen = torch.Generator(device="cuda").manual_seed(1)
    n = 4096 * 4096
    qb = bytes_quant(n, 4)
    nsets = sets_for(qb + n * 4)
    sets = []
    for _ in range(nsets):
        x = with_outliers(torch, gen, torch.randn(4096, 4096, generator=gen, device="cuda"), 0.01, 20.0)
        sets.append((x, torch.empty(n, dtype=torch.int8, device="cuda"),
                     torch.empty((n + 63) // 64, device="cuda"), torch.empty(n, device="cuda")))
    lib = cf._lib.load()

    def quant(s):
        return lambda: cf._lib.check(lib.cf_quantize_int8(
            s[0].data_ptr(), cf._lib.CF_F32, s[1].data_ptr(), s[2].data_ptr(), n,
            torch.cuda.current_stream().cuda_stream))

    def dequant(s):
        return lambda: cf._lib.check(lib.cf_dequantize_int8(
            s[1].data_ptr(), s[2].data_ptr(), s[3].data_ptr(), cf._lib.CF_F32, n,
            torch.cuda.current_stream().cuda_stream))

    q = summary(time_launches(torch, [quant(s) for s in sets], warmup, runs))
    with_kernel_time(torch, cf, q, [quant(s) for s in sets], nbytes=qb)
    # The streaming ceiling of the quantiser's own traffic mix at this size:
    # read 64 MiB, write a quarter of it, same load pattern, no arithmetic.
    def stream(s):
        return lambda: cf._lib.check(lib.cf_stream_bytes(
            s[0].data_ptr(), s[3].data_ptr(), n * 4, 4, torch.cuda.current_stream().cuda_stream))

    ceiling = summary(time_launches(torch, [stream(s) for s in sets], warmup, runs))
    with_kernel_time(torch, cf, ceiling, [stream(s) for s in sets], nbytes=n * 5)
    # Its two halves alone, same load and store patterns: read 64 MiB (one
    # word per 16 KiB written), and write 16 MiB (nothing read).
    def read_only(s):
        return lambda: cf._lib.check(lib.cf_stream_bytes(
            s[0].data_ptr(), s[3].data_ptr(), n * 4, 0, torch.cuda.current_stream().cuda_stream))

    def write_only(s):
        return lambda: cf._lib.check(lib.cf_stream_bytes(
            None, s[1].data_ptr(), n, -1, torch.cuda.current_stream().cuda_stream))

    reads = summary(time_launches(torch, [read_only(s) for s in sets], warmup, runs))
    with_kernel_time(torch, cf, reads, [read_only(s) for s in sets], nbytes=n * 4)
    writes = summary(time_launches(torch, [write_only(s) for s in sets], warmup, runs))
    with_kernel_time(torch, cf, writes, [write_only(s) for s in sets], nbytes=n)
    # Dequantisation reads only 17 MB per set and writes 64 MiB with
    # non-temporal stores, which leave the Infinity Cache to the codes: its
    # sets rotate until the codes alone exceed CACHE_FLUSH_BYTES, so no launch
    # finds its codes in the 256 MB cache. Each set's codes and scales are a
    # copy of the quantised first set.
    d_sets = [(None, sets[0][1].clone(), sets[0][2].clone(), torch.empty(n, device="cuda"))
              for _ in range(sets_for(n + 4 * ((n + 63) // 64)))]
    d = summary(time_launches(torch, [dequant(s) for s in d_sets], warmup, runs))
    with_kernel_time(torch, cf, d, [dequant(s) for s in d_sets], nbytes=bytes_dequant(n, 4))
    return {
        "quantize_f32_4096x4096": {**q, "GB/s": gbs(qb, q["median_ms"]), "bytes": qb,
                                   "frac_hbm": gbs(qb, q["median_ms"]) / PEAK_HBM_GBS},
        "dequantize_f32_4096x4096": {**d, "GB/s": gbs(bytes_dequant(n, 4), d["median_ms"]),
                                     "bytes": bytes_dequant(n, 4), "buffer_sets": len(d_sets),
                                     "frac_hbm": gbs(bytes_dequant(n, 4), d["median_ms"]) / PEAK_HBM_GBS},
        "stream_ceiling_read64MiB_write16MiB_context": {
            **ceiling, "bytes": n * 5, "GB/s": gbs(n * 5, ceiling["median_ms"]),
            "frac_hbm": gbs(n * 5, ceiling["median_ms"]) / PEAK_HBM_GBS},
        "stream_read_only_64MiB_context": {
            **reads, "bytes": n * 4, "GB/s": gbs(n * 4, reads["median_ms"]),
            "frac_hbm": gbs(n * 4, reads["median_ms"]) / PEAK_HBM_GBS},
        "stream_write_only_16MiB_context": {
            **writes, "bytes": n, "GB/s": gbs(n, writes["median_ms"]),
            "frac_hbm": gbs(n, writes["median_ms"]) / PEAK_HBM_GBS},
    }


def bench_ceiling(torch, cf, warmup: int, runs: int) -> dict:
    """Config 1's kernels next to the streaming ceilings of their traffic, all
    under the same conditions: 32 rotating buffer sets (2.6 GB, so no launch
    finds its input in the 256 MB Infinity Cache), one untimed pass over them,
    then two passes captured into a HIP graph and replayed (dispatches back
    to back, with no host launch loop, which kernels of a few microseconds
    outrun), each replay timed by a HIP event pair. Kernels: quantise and
    dequantise fp32 [4096, 4096]; reading the 64 MiB input alone; writing
    16 MiB alone (four stores per lane, and one store per lane under each
    cache policy: cf_stream_bytes divisors -1 .. -5); reading 64 MiB and
    writing 16 MiB with the quantiser's pattern (divisors 0 and 4); a 64 MiB
    copy; and config 5's 2 : 1 read/write mix at the size of one grouped
    launch. `median_ms` is the median over 3 replays of the per-launch
    time."""
    gen = torch.Generator(device="cuda").manual_seed(11)
    n = 4096 * 4096
    lib = cf._lib.load()
    nsets = 32
    xs = [with_outliers(torch, gen, torch.randn(n, generator=gen, device="cuda"), 0.01, 20.0)
          for _ in range(nsets)]
    qs = [torch.empty(n, dtype=torch.int8, device="cuda") for _ in range(nsets)]
    ss = [torch.empty((n + 63) // 64, device="cuda") for _ in range(nsets)]
    ys = [torch.empty(n, device="cuda") for _ in range(nsets)]
    xp, qp, sp, yp = ([t.data_ptr() for t in ts] for ts in (xs, qs, ss, ys))
    f32 = cf._lib.CF_F32
    # Each launch reads the current stream when it is made, so the same
    # closures run eagerly and under graph capture.
    def cur():
        return torch.cuda.current_stream().cuda_stream

    kinds = {
        "quantize_f32_4096x4096": (bytes_quant(n, 4),
                                   lambda i: lib.cf_quantize_int8(xp[i], f32, qp[i], sp[i], n, cur())),
        "dequantize_f32_4096x4096": (bytes_dequant(n, 4),
                                     lambda i: lib.cf_dequantize_int8(qp[i], sp[i], yp[i], f32, n, cur())),
        "read_only_64MiB": (n * 4, lambda i: lib.cf_stream_bytes(xp[i], sp[i], n * 4, 0, cur())),
        "write_only_16MiB": (n, lambda i: lib.cf_stream_bytes(None, qp[i], n, -1, cur())),
        # The same 16 MiB written with one 16-byte store per lane, under each
        # cache policy the stores can carry: the fastest of these is the best
        # this box writes 16 MiB in one launch.
        "write_only_16MiB_once_nt": (n, lambda i: lib.cf_stream_bytes(None, qp[i], n, -2, cur())),
        "write_only_16MiB_once_device_scope": (n, lambda i: lib.cf_stream_bytes(None, qp[i], n, -3, cur())),
        "write_only_16MiB_once_nt_device_scope": (n, lambda i: lib.cf_stream_bytes(None, qp[i], n, -4, cur())),
        "write_only_16MiB_once_plain": (n, lambda i: lib.cf_stream_bytes(None, qp[i], n, -5, cur())),
        "read_64MiB_write_16MiB": (n * 5, lambda i: lib.cf_stream_bytes(xp[i], qp[i], n * 4, 4, cur())),
        "copy_64MiB": (n * 8, lambda i: lib.cf_copy_bytes(xp[i], yp[i], n * 4, cur())),
    }
    # Config 5's bulk bf16 quantiser moves 2 bytes in per byte out in launches
    # of up to 48 tensors (~2.3 GB each): its traffic mix at that scale, one
    # launch reading 1.5 GiB and writing 0.75 GiB (divisor 2).
    big = 3 << 29
    big_in = torch.empty(big, dtype=torch.uint8, device="cuda")
    big_out = torch.empty(big // 2, dtype=torch.uint8, device="cuda")
    kinds["read_1536MiB_write_768MiB"] = (
        big + big // 2, lambda i: lib.cf_stream_bytes(big_in.data_ptr(), big_out.data_ptr(), big, 2, cur()))
    samples: dict[str, list[float]] = {}
    for label, (_, call) in kinds.items():
        for i in range(nsets):  # untimed pass, statuses checked
            cf._lib.check(call(i))
        torch.cuda.synchronize()
        # Two passes over the sets captured into one HIP graph (kernels only)
        # and replayed: dispatches back to back, with no host launch loop that
        # kernels of a few microseconds would outrun.
        samples[label] = graph_times(torch, [lambda i=i, call=call: call(i) for i in range(nsets)],
                                     runs=2 * nsets, batches=3)
    out = {}
    for label, (nbytes, _) in kinds.items():
        r = summary(samples[label])
        out[f"ceiling_{label}"] = {**r, "bytes": nbytes, "GB/s": gbs(nbytes, r["median_ms"]),
                                   "frac_hbm": gbs(nbytes, r["median_ms"]) / PEAK_HBM_GBS}
    return out


# The reference's published kernel table (README.md:400-451; RTX 3090, fp32,
# median of 100 event-timed launches): shape -> median ms, as context beside
# this build's figures at the same shapes.
REFERENCE_3090_MS = {
    "sum_f32_64K": 0.0082, "sum_f32_1M": 0.0102, "sum_f32_16M": 0.0922,
    "softmax_f32_128x8192": 0.0154, "rmsnorm_f32_4096x1024": 0.0440, "rmsnorm_f32_2048x4096": 0.0829,
    "silu_f32_16M": 0.1567, "swiglu_f32_16M": 0.2294, "fused_residual_rmsnorm_f32_2048x4096": 0.1597,
    "quantize_f32_16M": 0.1915, "dequantize_f32_16M": 0.1126,
    "lora_f32_32x1024x1024_r8": 0.0850, "lora_f32_64x2048x2048_r16": 0.3640,
    "lora_f32_128x4096x4096_r16": 2.0562,
}


def bench_reference_shapes(torch, cf, warmup: int, runs: int) -> dict:
    """Every kernel the reference publishes a figure for, at its benchmark shape
    (fp32; README.md:400-451). Every row reports the median of 25 calls timed
    by their kernels' own timestamps (`kernel_median_ms`, first kernel's start
    to last kernel's end) beside the launch-loop median (`median_ms`, which
    for calls of a few microseconds is the Python launch rate), over >= 1 GiB
    of rotating buffers; the sums' and LoRA's rates (GB/s, TFLOP/s) are from
    `kernel_median_ms`.
    Streaming rows add `graph_median_ms`: the same launches captured into one
    HIP graph and replayed, so short kernels run back to back on the GPU with
    no Python loop between them (`graph_frac_hbm` from it). Both figures
    bound the kernel's own time from above (a graph replay adds the gaps
    between dispatches; a dispatch's timestamps read long when it starts from
    an idle queue), and those rows' `GB/s` and `frac_hbm` take the smaller.
    `reference_3090_ms` is the reference's own figure (other hardware), an
    event pair around each launch (benchmarks/benchmark_kernels.cu:59-79)."""
    gen = torch.Generator(device="cuda").manual_seed(12)
    lib = cf._lib.load()
    f32 = cf._lib.CF_F32
    st = lambda: torch.cuda.current_stream().cuda_stream  # noqa: E731
    out = {}

    def record(label, entry):
        entry["reference_3090_ms"] = REFERENCE_3090_MS[label]
        out[label] = entry

    def streamed(label, nbytes, make, call):
        sets = [make() for _ in range(sets_for(nbytes))]
        launches = [lambda s=s: cf._lib.check(call(s)) for s in sets]
        r = summary(time_launches(torch, launches, warmup, runs))
        with_kernel_time(torch, cf, r, launches, nbytes=nbytes)
        r["graph_median_ms"] = statistics.median(graph_times(torch, launches, runs))
        r["graph_frac_hbm"] = gbs(nbytes, r["graph_median_ms"]) / PEAK_HBM_GBS
        best = min(r["kernel_median_ms"], r["graph_median_ms"])
        record(label, {**r, "bytes": nbytes, "GB/s": gbs(nbytes, best), "frac_hbm": gbs(nbytes, best) / PEAK_HBM_GBS})

    for n, label in ((1 << 16, "sum_f32_64K"), (1 << 20, "sum_f32_1M"), (1 << 24, "sum_f32_16M")):
        ws = torch.empty(max(lib.cf_reduce_sum_workspace_bytes(n), 16), dtype=torch.uint8, device="cuda")
        res = torch.empty(1, device="cuda")
        sets = [torch.randn(n, generator=gen, device="cuda") for _ in range(sets_for(4 * n))]
        launches = [lambda x=x, n=n, ws=ws: cf._lib.check(lib.cf_reduce_sum(
            x.data_ptr(), f32, res.data_ptr(), n, ws.data_ptr(), ws.numel(), 0, st())) for x in sets]
        r = summary(time_launches(torch, launches, warmup, runs))
        with_kernel_time(torch, cf, r, launches, nbytes=4 * n)
        record(label, {**r, "bytes": 4 * n, "launches": 1 if 4 * n <= SUM_SINGLE_LAUNCH_BYTES else 2,
                       "GB/s": r["kernel_GB/s"], "frac_hbm": r["kernel_frac_hbm"]})
    rows, cols = 128, 8192
    streamed("softmax_f32_128x8192", 2 * rows * cols * 4,
             lambda: (torch.randn(rows, cols, generator=gen, device="cuda"), torch.empty(rows, cols, device="cuda")),
             lambda s: lib.cf_softmax(s[0].data_ptr(), f32, s[1].data_ptr(), f32, rows, cols, st()))
    for rows, cols in ((4096, 1024), (2048, 4096)):
        w = torch.randn(cols, generator=gen, device="cuda")
        streamed(f"rmsnorm_f32_{rows}x{cols}", bytes_rmsnorm(rows, cols, 4),
                 lambda rows=rows, cols=cols: (torch.randn(rows, cols, generator=gen, device="cuda"),
                                               torch.empty(rows, cols, device="cuda")),
                 lambda s, rows=rows, cols=cols, w=w: lib.cf_rmsnorm(
                     s[0].data_ptr(), w.data_ptr(), s[1].data_ptr(), f32, rows, cols, 1e-6, st()))
    n = 1 << 24
    streamed("silu_f32_16M", 2 * n * 4,
             lambda: (torch.randn(n, generator=gen, device="cuda"), torch.empty(n, device="cuda")),
             lambda s: lib.cf_silu(s[0].data_ptr(), s[1].data_ptr(), f32, n, st()))
    streamed("swiglu_f32_16M", 3 * n * 4,
             lambda: tuple(torch.randn(n, generator=gen, device="cuda") for _ in range(3)),
             lambda s: lib.cf_swiglu(s[0].data_ptr(), s[1].data_ptr(), s[2].data_ptr(), f32, n, st()))
    rows, cols = 2048, 4096
    w = torch.randn(cols, generator=gen, device="cuda")
    streamed("fused_residual_rmsnorm_f32_2048x4096", 4 * rows * cols * 4,
             lambda: tuple(torch.randn(rows, cols, generator=gen, device="cuda") for _ in range(4)),
             lambda s: lib.cf_fused_residual_rmsnorm(s[0].data_ptr(), s[1].data_ptr(), w.data_ptr(), s[2].data_ptr(),
                                                     s[3].data_ptr(), f32, rows, cols, 1e-6, st()))
    streamed("quantize_f32_16M", bytes_quant(n, 4),
             lambda: (torch.randn(n, generator=gen, device="cuda"), torch.empty(n, dtype=torch.int8, device="cuda"),
                      torch.empty(n // 64, device="cuda")),
             lambda s: lib.cf_quantize_int8(s[0].data_ptr(), f32, s[1].data_ptr(), s[2].data_ptr(), n, st()))
    streamed("dequantize_f32_16M", bytes_dequant(n, 4),
             lambda: (torch.randint(-127, 128, (n,), generator=gen, device="cuda", dtype=torch.int8),
                      torch.rand(n // 64, generator=gen, device="cuda"), torch.empty(n, device="cuda")),
             lambda s: lib.cf_dequantize_int8(s[0].data_ptr(), s[1].data_ptr(), s[2].data_ptr(), f32, n, st()))
    for m, k, nn, r in ((32, 1024, 1024, 8), (64, 2048, 2048, 16), (128, 4096, 4096, 16)):
        label = f"lora_f32_{m}x{k}x{nn}_r{r}"
        flops = flops_lora(m, k, nn, r)
        set_bytes = 4 * (m * k + k * nn + k * r + r * nn + m * nn)
        sets = []
        for _ in range(sets_for(set_bytes)):
            sets.append((torch.randn(m, k, generator=gen, device="cuda"),
                         0.02 * torch.randn(k, nn, generator=gen, device="cuda"),
                         torch.randn(k, r, generator=gen, device="cuda") / 64,
                         0.02 * torch.randn(r, nn, generator=gen, device="cuda"),
                         torch.empty(m, nn, device="cuda"), torch.empty(m, r, device="cuda")))
        ws_bytes = lib.cf_lora_linear_ws_bytes(f32, m, k, nn, r)
        ws = torch.empty(max(ws_bytes, 16), dtype=torch.uint8, device="cuda")
        launches = [lambda s=s, m=m, k=k, nn=nn, r=r, ws_bytes=ws_bytes, ws=ws: cf._lib.check(lib.cf_lora_linear_ws(
            s[0].data_ptr(), s[1].data_ptr(), s[2].data_ptr(), s[3].data_ptr(), s[4].data_ptr(), s[5].data_ptr(),
            f32, m, k, nn, r, 2.0, ws.data_ptr() if ws_bytes else None, ws_bytes, st())) for s in sets]
        res = summary(time_launches(torch, launches, warmup, max(runs // 4, 8)))
        with_kernel_time(torch, cf, res, launches, flops=flops, peak=PEAK_FP32_TFLOPS)
        record(label, {**res, "flops": flops, "launches": 2 if ws_bytes else 1, "TFLOP/s": res["kernel_TFLOP/s"]})
        del sets
    return out


def bench_rowops(torch, cf, warmup: int, runs: int) -> dict:
    """config 2 per kernel, plus softmax at bandwidth scale (config 4's scores)."""
    gen = torch.Generator(device="cuda").manual_seed(3)
    lib = cf._lib.load()
    out = {}
    rows, cols = 16384, 4096
    w = (1 + 0.02 * torch.randn(cols, generator=gen, device="cuda")).to(torch.bfloat16)
    rb = bytes_rmsnorm(rows, cols, 2)
    sets = [make_rmsnorm_set(torch, gen, rows, cols, torch.bfloat16) for _ in range(sets_for(rb))]
    launches = [lambda s=s: cf._lib.check(lib.cf_rmsnorm(
        s[0].data_ptr(), w.data_ptr(), s[1].data_ptr(), cf._lib.CF_BF16, rows, cols, 1e-6,
        torch.cuda.current_stream().cuda_stream)) for s in sets]
    r = summary(time_launches(torch, launches, warmup, runs))
    with_kernel_time(torch, cf, r, launches, nbytes=rb)
    out["rmsnorm_bf16_16384x4096"] = {**r, "bytes": rb, "GB/s": gbs(rb, r["median_ms"]),
                                      "frac_hbm": gbs(rb, r["median_ms"]) / PEAK_HBM_GBS}
    del sets, launches
    for s_rows, s_cols, label in ((1024, 2048, "softmax_bf16_causal_1024x2048"),
                                  (131072, 512, "softmax_bf16_causal_131072x512")):
        sb = bytes_softmax(s_rows, s_cols, 2)
        sets = [make_causal_logits(torch, gen, s_rows, s_cols, torch.bfloat16) for _ in range(sets_for(sb))]
        launches = [lambda s=s, a=s_rows, b=s_cols: cf._lib.check(lib.cf_softmax(
            s[0].data_ptr(), cf._lib.CF_BF16, s[1].data_ptr(), cf._lib.CF_BF16, a, b,
            torch.cuda.current_stream().cuda_stream)) for s in sets]
        r = summary(time_launches(torch, launches, warmup, runs))
        with_kernel_time(torch, cf, r, launches, nbytes=sb)
        r["graph_median_ms"] = statistics.median(graph_times(torch, launches, runs))
        out[label] = {**r, "bytes": sb, "GB/s": gbs(sb, r["median_ms"]),
                      "frac_hbm": gbs(sb, r["median_ms"]) / PEAK_HBM_GBS}
        del sets, launches
    # Config 4's attention softmax as the block now runs it: softmax(scores /
    # sqrt(128) + causal) on [8 x 32 x 512, 512] bf16 scores in one pass
    # (cf_softmax_scaled). Algorithmic bytes: the visible scores read once
    # (row r of each head block keeps r + 1 columns) plus every output written.
    s_rows, s_cols = 131072, 512
    visible = sum((r % s_cols) + 1 for r in range(s_cols)) * (s_rows // s_cols)
    sb = (visible + s_rows * s_cols) * 2
    sets = []
    for _ in range(sets_for(2 * s_rows * s_cols * 2)):
        x = torch.randn(s_rows, s_cols, generator=gen, device="cuda").to(torch.bfloat16)
        sets.append((x, torch.empty_like(x)))
    launches = [lambda s=s: cf._lib.check(lib.cf_softmax_scaled(
        s[0].data_ptr(), cf._lib.CF_BF16, s[1].data_ptr(), cf._lib.CF_BF16, s_rows, s_cols,
        1 / 128 ** 0.5, s_cols, torch.cuda.current_stream().cuda_stream)) for s in sets]
    r = summary(time_launches(torch, launches, warmup, runs))
    with_kernel_time(torch, cf, r, launches, nbytes=sb)
    out["softmax_scaled_causal_bf16_131072x512"] = {**r, "bytes": sb, "GB/s": gbs(sb, r["median_ms"]),
                                                     "frac_hbm": gbs(sb, r["median_ms"]) / PEAK_HBM_GBS}
    del sets, launches
    # The row's neighbours in the same family: fused residual add +
    # RMSNorm at config 2's shape, and the activations over a Llama-7B MLP
    # activation ([16384, 11008]).
    res_bytes = 4 * rows * cols * 2
    sets = [tuple(torch.randn(rows, cols, generator=gen, device="cuda").to(torch.bfloat16) for _ in range(4))
            for _ in range(sets_for(res_bytes))]
    launches = [lambda s=s: cf._lib.check(lib.cf_fused_residual_rmsnorm(
        s[0].data_ptr(), s[1].data_ptr(), w.data_ptr(), s[2].data_ptr(), s[3].data_ptr(), cf._lib.CF_BF16,
        rows, cols, 1e-6, torch.cuda.current_stream().cuda_stream)) for s in sets]
    r = summary(time_launches(torch, launches, warmup, runs))
    with_kernel_time(torch, cf, r, launches, nbytes=res_bytes)
    out["fused_residual_rmsnorm_bf16_16384x4096"] = {**r, "bytes": res_bytes, "GB/s": gbs(res_bytes, r["median_ms"]),
                                                     "frac_hbm": gbs(res_bytes, r["median_ms"]) / PEAK_HBM_GBS}
    del sets, launches
    n = 16384 * 11008
    for name, operands in (("silu", 1), ("gelu", 1), ("swiglu", 2)):
        nbytes = (operands + 1) * n * 2
        sets = [tuple(torch.randn(n, generator=gen, device="cuda").to(torch.bfloat16) for _ in range(operands + 1))
                for _ in range(sets_for(nbytes))]
        if name == "swiglu":
            launches = [lambda s=s: cf._lib.check(lib.cf_swiglu(
                s[0].data_ptr(), s[1].data_ptr(), s[2].data_ptr(), cf._lib.CF_BF16, n,
                torch.cuda.current_stream().cuda_stream)) for s in sets]
        else:
            fn = getattr(lib, f"cf_{name}")
            launches = [lambda s=s, fn=fn: cf._lib.check(fn(
                s[0].data_ptr(), s[1].data_ptr(), cf._lib.CF_BF16, n,
                torch.cuda.current_stream().cuda_stream)) for s in sets]
        r = summary(time_launches(torch, launches, warmup, runs))
        with_kernel_time(torch, cf, r, launches, nbytes=nbytes)
        out[f"{name}_bf16_16384x11008"] = {**r, "bytes": nbytes, "GB/s": gbs(nbytes, r["median_ms"]),
                                          "frac_hbm": gbs(nbytes, r["median_ms"]) / PEAK_HBM_GBS}
        del sets, launches
    # A plain copy of the same size as the RMSNorm traffic: the achievable bound.
    nbytes = rows * cols * 2
    sets = [(torch.empty(nbytes, dtype=torch.uint8, device="cuda"),
             torch.empty(nbytes, dtype=torch.uint8, device="cuda")) for _ in range(sets_for(2 * nbytes))]
    launches = [lambda s=s: cf._lib.check(lib.cf_copy_bytes(
        s[0].data_ptr(), s[1].data_ptr(), nbytes, torch.cuda.current_stream().cuda_stream)) for s in sets]
    r = summary(time_launches(torch, launches, warmup, runs))
    with_kernel_time(torch, cf, r, launches, nbytes=2 * nbytes)
    out["copy_128MiB"] = {**r, "bytes": 2 * nbytes, "GB/s": gbs(2 * nbytes, r["median_ms"]),
                          "frac_hbm": gbs(2 * nbytes, r["median_ms"]) / PEAK_HBM_GBS}
    return out


def bench_reduce(torch, cf, warmup: int, runs: int) -> dict:
    """Rows a9-a11: the deterministic two-stage sum at the reference's benchmark
    size (16M fp32, README's reduction table) and at 256M, and per-row sums of a
    [16384, 4096] fp32 matrix. 4 bytes read per element; the output is a few bytes."""
    gen = torch.Generator(device="cuda").manual_seed(10)
    lib = cf._lib.load()
    out = {}
    for n, label in ((1 << 24, "sum_f32_16M"), (1 << 28, "sum_f32_256M")):
        nbytes = 4 * n
        sets = [torch.randn(n, generator=gen, device="cuda") for _ in range(sets_for(nbytes))]
        ws_bytes = lib.cf_reduce_sum_workspace_bytes(n)
        ws = torch.empty(max(ws_bytes, 16), dtype=torch.uint8, device="cuda")
        res = torch.empty(1, device="cuda")
        launches = [lambda x=x: cf._lib.check(lib.cf_reduce_sum(
            x.data_ptr(), cf._lib.CF_F32, res.data_ptr(), n, ws.data_ptr(), ws_bytes, 0,
            torch.cuda.current_stream().cuda_stream)) for x in sets]
        r = summary(time_launches(torch, launches, warmup, runs))
        with_kernel_time(torch, cf, r, launches, nbytes=nbytes)
        out[label] = {**r, "bytes": nbytes, "launches": 2, "GB/s": gbs(nbytes, r["median_ms"]),
                      "frac_hbm": gbs(nbytes, r["median_ms"]) / PEAK_HBM_GBS}
        del sets
        torch.cuda.empty_cache()
    rows, cols = 16384, 4096
    nbytes = rows * cols * 4 + rows * 4
    sets = [torch.randn(rows, cols, generator=gen, device="cuda") for _ in range(sets_for(nbytes))]
    res = torch.empty(rows, device="cuda")
    launches = [lambda x=x: cf._lib.check(lib.cf_row_sum(
        x.data_ptr(), cf._lib.CF_F32, res.data_ptr(), rows, cols,
        torch.cuda.current_stream().cuda_stream)) for x in sets]
    r = summary(time_launches(torch, launches, warmup, runs))
    with_kernel_time(torch, cf, r, launches, nbytes=nbytes)
    out["row_sum_f32_16384x4096"] = {**r, "bytes": nbytes, "GB/s": gbs(nbytes, r["median_ms"]),
                                     "frac_hbm": gbs(nbytes, r["median_ms"]) / PEAK_HBM_GBS}
    return out


def bench_lora(torch, cf, warmup: int, runs: int) -> dict:
    """config 3: fused LoRA bf16 8192x4096x4096 r16, alpha 32; adapter backward.
    Operand sets (x, W, A, B, y, dY, x@A) rotate until they exceed 1 GiB, so the
    forward and the backward read their operands from HBM, not from the 256 MB
    Infinity Cache; hipBLASLt's plain GEMM runs on the same sets. The forward
    goes through cf_lora_linear_ws with the workspace it asks for (x @ a shared
    between column tiles), the entry point the torch operator calls."""
    gen = torch.Generator(device="cuda").manual_seed(4)
    m, k, n, r = 8192, 4096, 4096, 16
    lib = cf._lib.load()
    flops = flops_lora(m, k, n, r)
    set_bytes = (m * k + k * n + 2 * m * n) * 2 + (k * r + r * n) * 2 + m * r * 4
    sets = []
    for _ in range(sets_for(set_bytes)):
        x = torch.randn(m, k, generator=gen, device="cuda").to(torch.bfloat16)
        W = (0.02 * torch.randn(n, k, generator=gen, device="cuda")).to(torch.bfloat16)
        A = (torch.randn(r, k, generator=gen, device="cuda") / 64).to(torch.bfloat16)
        B = (0.02 * torch.randn(n, r, generator=gen, device="cuda")).to(torch.bfloat16)
        sets.append({"x": x, "w": W.t().contiguous(), "a": A.t().contiguous(), "b": B.t().contiguous(),
                     "y": torch.empty(m, n, dtype=torch.bfloat16, device="cuda"),
                     "dy": torch.randn(m, n, generator=gen, device="cuda").to(torch.bfloat16),
                     "xa": torch.empty(m, r, device="cuda")})
        del W, A, B

    fwd_ws_bytes = lib.cf_lora_linear_ws_bytes(cf._lib.CF_BF16, m, k, n, r)
    fwd_ws = torch.empty(max(fwd_ws_bytes, 1), dtype=torch.uint8, device="cuda")

    def fused(s, xa_out=None):
        return lambda: cf._lib.check(lib.cf_lora_linear_ws(
            s["x"].data_ptr(), s["w"].data_ptr(), s["a"].data_ptr(), s["b"].data_ptr(), s["y"].data_ptr(),
            xa_out, cf._lib.CF_BF16, m, k, n, r, 2.0, fwd_ws.data_ptr() if fwd_ws_bytes else None,
            fwd_ws_bytes, torch.cuda.current_stream().cuda_stream))

    launches = [fused(s) for s in sets]
    f = summary(time_launches(torch, launches, warmup, runs))
    with_kernel_time(torch, cf, f, launches, flops=flops, peak=PEAK_BF16_TFLOPS)
    out = {"lora_bf16_8192x4096x4096_r16": {**f, "flops": flops, "buffer_sets": len(sets),
                                             "TFLOP/s": flops / (f["median_ms"] * 1e-3) / 1e12,
                                             "frac_mfma": flops / (f["median_ms"] * 1e-3) / 1e12 / PEAK_BF16_TFLOPS}}

    gemms = [lambda s=s: torch.matmul(s["x"], s["w"], out=s["y"]) for s in sets]
    lg = summary(time_launches(torch, gemms, warmup, runs))
    base = 2 * m * k * n
    out["hipblaslt_gemm_bf16_8192x4096x4096_context"] = {
        **lg, "TFLOP/s": base / (lg["median_ms"] * 1e-3) / 1e12}

    for s in sets:  # the forward's x @ A, which the backward reads
        fused(s, s["xa"].data_ptr())()
    ga = torch.empty(k, r, dtype=torch.bfloat16, device="cuda")
    gb = torch.empty(r, n, dtype=torch.bfloat16, device="cuda")
    nbytes = lib.cf_lora_backward_workspace_bytes(m, k, n, r)
    ws = torch.empty(nbytes, dtype=torch.uint8, device="cuda")

    def backward(s):
        return lambda: cf._lib.check(lib.cf_lora_backward(
            s["x"].data_ptr(), s["dy"].data_ptr(), s["b"].data_ptr(), s["xa"].data_ptr(), ga.data_ptr(),
            gb.data_ptr(), cf._lib.CF_BF16, m, k, n, r, 2.0, ws.data_ptr(), nbytes,
            torch.cuda.current_stream().cuda_stream))

    bw_launches = [backward(s) for s in sets]
    bw = summary(time_launches(torch, bw_launches, warmup, runs))
    bw_bytes = m * k * 2 + m * n * 2 + m * r * 4 + r * n * 2 + k * r * 2 + r * n * 2
    with_kernel_time(torch, cf, bw, bw_launches, nbytes=bw_bytes)
    out["lora_backward_bf16_8192x4096x4096_r16"] = {**bw, "bytes": bw_bytes, "buffer_sets": len(sets),
                                                    "GB/s": gbs(bw_bytes, bw["median_ms"]),
                                                    "frac_hbm": gbs(bw_bytes, bw["median_ms"]) / PEAK_HBM_GBS}
    return out


def bench_block(torch, cf, warmup: int, runs: int) -> dict:
    """config 4: one Llama block (8 x 512 tokens, hidden 4096, 32 heads, MLP 11008,
    LoRA r16 alpha 32 on every projection) through the custom operators."""
    from cuda_force_amd.transformer_block import BlockConfig, LlamaBlock, timed_forward

    gen = torch.Generator(device="cuda").manual_seed(6)
    config = BlockConfig()
    batch, seq = 8, 512
    block = LlamaBlock(config, "cuda", torch.bfloat16, gen)
    x = torch.randn(batch, seq, config.hidden, generator=gen, device="cuda").to(torch.bfloat16)
    residual = torch.randn(batch, seq, config.hidden, generator=gen, device="cuda").to(torch.bfloat16)
    tokens = batch * seq
    flops = block.gemm_flops(tokens, seq)
    total = summary(time_launches(torch, [lambda: block.forward(x, residual)], warmup, max(runs // 4, 5)))
    stages: dict[str, list[float]] = {}
    for _ in range(20):
        for name, ms in timed_forward(block, x, residual).items():
            stages.setdefault(name, []).append(ms)
    per_op = {}
    for name, samples in stages.items():
        ms = statistics.median(samples)
        entry = {"ms": ms}
        if name in flops:
            entry["TFLOP/s"] = flops[name] / (ms * 1e-3) / 1e12
        per_op[name] = entry
    gemm = sum(flops.values())
    # The same forward captured once into a HIP graph and replayed: the ~20
    # launches of a block go out as one submission.
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for _ in range(2):
            block.forward(x, residual)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        block.forward(x, residual)
    replay = summary(time_launches(torch, [graph.replay], warmup, max(runs // 4, 5)))
    return {"block_c4_bf16_8x512_h4096": {
        **total, "tokens": tokens, "tokens/s": tokens / (total["median_ms"] * 1e-3),
        "gemm_flops": gemm, "gemm_TFLOP/s_end_to_end": gemm / (total["median_ms"] * 1e-3) / 1e12,
        "graph_replay_ms": replay["median_ms"], "graph_tokens/s": tokens / (replay["median_ms"] * 1e-3),
        "per_op_events": per_op}}


def bench_paged(torch, cf, warmup: int, runs: int) -> dict:
    """Paged-attention decode at the reference's benchmark shapes
    (benchmarks/benchmark_kernels.cu:369-441: block size 16, fp32, identity
    and reversed block tables), plus bf16 caches. Algorithmic bytes: K and V
    once per (sequence, KV head) over the context, plus the query and output."""
    lib = cf._lib.load()
    gen = torch.Generator(device="cuda").manual_seed(7)
    stream = torch.cuda.current_stream().cuda_stream
    out = {}
    block = 16
    for seqs, heads, kv_heads, dim, ctx in ((16, 32, 32, 128, 512), (64, 32, 8, 128, 1024),
                                            (128, 32, 8, 128, 256)):
        per_seq = -(-ctx // block)
        blocks = seqs * per_seq
        for dtype, code, size in ((torch.float32, cf._lib.CF_F32, 4), (torch.bfloat16, cf._lib.CF_BF16, 2)):
            nbytes = 2 * seqs * kv_heads * ctx * dim * size + 2 * seqs * heads * dim * size
            sets = []
            for _ in range(sets_for(nbytes)):
                k = torch.randn(blocks, block, kv_heads, dim, generator=gen, device="cuda").to(dtype)
                v = torch.randn(blocks, block, kv_heads, dim, generator=gen, device="cuda").to(dtype)
                q = torch.randn(seqs, heads, dim, generator=gen, device="cuda").to(dtype)
                sets.append((q, k, v, torch.empty_like(q)))
            ctx_lens = torch.full((seqs,), ctx, dtype=torch.int32, device="cuda")
            ws_bytes = lib.cf_paged_attention_workspace_bytes(seqs, heads, kv_heads, dim, block, per_seq)
            ws = torch.empty(max(ws_bytes, 16), dtype=torch.uint8, device="cuda")
            identity = torch.arange(blocks, dtype=torch.int32, device="cuda").view(seqs, per_seq)
            for layout, table in (("contiguous", identity), ("scattered", identity.flip(0).flip(1).contiguous())):
                launches = [lambda s=s, t=table: cf._lib.check(lib.cf_paged_attention(
                    s[0].data_ptr(), s[1].data_ptr(), s[2].data_ptr(), t.data_ptr(), ctx_lens.data_ptr(),
                    s[3].data_ptr(), code, seqs, heads, kv_heads, dim, block, per_seq, dim ** -0.5,
                    ws.data_ptr() if ws_bytes else None, ws_bytes, stream)) for s in sets]
                r = summary(time_launches(torch, launches, warmup, runs))
                name = "f32" if size == 4 else "bf16"
                out[f"paged_attention_{name}_{seqs}seq_{ctx}ctx_h{heads}kv{kv_heads}_{layout}"] = {
                    **r, "bytes": nbytes, "GB/s": gbs(nbytes, r["median_ms"]),
                    "frac_hbm": gbs(nbytes, r["median_ms"]) / PEAK_HBM_GBS}
            del sets
            torch.cuda.empty_cache()
    return out


def bench_tensor_core(torch, cf, warmup: int, runs: int) -> dict:
    """fp32 matmul on the bf16 MFMA units (hi/lo split, three bf16 products in
    one GEMM) at the reference benchmark's largest square, and 4096^3; FLOP/s
    counts the fp32 product (2 m n k), with torch's fp32 matmul for context."""
    lib = cf._lib.load()
    gen = torch.Generator(device="cuda").manual_seed(8)
    stream = torch.cuda.current_stream().cuda_stream
    out = {}
    for n in (1024, 4096):
        a = torch.randn(n, n, generator=gen, device="cuda")
        b = torch.randn(n, n, generator=gen, device="cuda")
        c = torch.empty(n, n, device="cuda")
        nbytes = lib.cf_matmul_tensor_core_workspace_bytes(n, n, n)
        ws = torch.empty(nbytes, dtype=torch.uint8, device="cuda")

        def tc():
            cf._lib.check(lib.cf_matmul_tensor_core(a.data_ptr(), b.data_ptr(), c.data_ptr(), n, n, n,
                                                    ws.data_ptr(), nbytes, stream))

        r = summary(time_launches(torch, [tc], warmup, runs))
        flops = 2 * n ** 3
        out[f"tensor_core_matmul_f32_{n}"] = {**r, "TFLOP/s": flops / (r["median_ms"] * 1e-3) / 1e12}
        r = summary(time_launches(torch, [lambda: torch.matmul(a, b, out=c)], warmup, runs))
        out[f"torch_matmul_f32_{n}_context"] = {**r, "TFLOP/s": flops / (r["median_ms"] * 1e-3) / 1e12}
    return out


def bench_fp8(torch, cf, warmup: int, runs: int) -> dict:
    """fp8 (e4m3fn) MFMA matmul, bf16 output, at 8192^3 and 4096^3, with w
    row-major [K, N] (cf_matmul_fp8) and K-major as w_t [N, K]
    (cf_matmul_fp8_wt, the operand layout hipBLASLt's fp8 GEMM is given
    below); FLOP/s counts 2 m n k against the dense fp8 peak, with hipBLASLt's
    fp8 GEMM (torch._scaled_mm, per-tensor scales) for context where torch
    offers it."""
    lib = cf._lib.load()
    gen = torch.Generator(device="cuda").manual_seed(9)
    stream = torch.cuda.current_stream().cuda_stream
    out = {}
    for n in (8192, 4096):
        codes = torch.randint(0, 256, (2, n, n), generator=gen, device="cuda", dtype=torch.uint8)
        codes = (codes & 0xA7) | 0x18  # finite, moderate magnitudes
        x, w = codes[0], codes[1]
        y = torch.empty(n, n, dtype=torch.bfloat16, device="cuda")

        def fp8():
            cf._lib.check(lib.cf_matmul_fp8(x.data_ptr(), w.data_ptr(), y.data_ptr(), n, n, n, 1.0, stream))

        w_t = w.t().contiguous()

        def fp8_wt():
            cf._lib.check(lib.cf_matmul_fp8_wt(x.data_ptr(), w_t.data_ptr(), y.data_ptr(), n, n, n, 1.0, stream))

        flops = 2 * n ** 3
        for name, fn in ((f"matmul_fp8_{n}", fp8), (f"matmul_fp8_wt_{n}", fp8_wt)):
            r = summary(time_launches(torch, [fn], warmup, runs))
            with_kernel_time(torch, cf, r, [fn], flops=flops, peak=PEAK_FP8_TFLOPS)
            tflops = flops / (r["median_ms"] * 1e-3) / 1e12
            out[name] = {**r, "TFLOP/s": tflops, "frac_fp8_peak": tflops / PEAK_FP8_TFLOPS}
        try:
            xf = x.view(torch.float8_e4m3fn)
            wf = w.view(torch.float8_e4m3fn).t().contiguous().t()  # column-major right operand
            one = torch.ones((), device="cuda")
            torch._scaled_mm(xf, wf, scale_a=one, scale_b=one, out_dtype=torch.bfloat16)
            r = summary(time_launches(
                torch, [lambda: torch._scaled_mm(xf, wf, scale_a=one, scale_b=one, out_dtype=torch.bfloat16)],
                warmup, runs))
            out[f"torch_scaled_mm_fp8_{n}_context"] = {
                **r, "TFLOP/s": flops / (r["median_ms"] * 1e-3) / 1e12}
        except (RuntimeError, AttributeError) as exc:
            out[f"torch_scaled_mm_fp8_{n}_context"] = {"unavailable": str(exc).splitlines()[0][:160]}
        del codes, y, w_t
        torch.cuda.empty_cache()
    return out


def bench_bulk_quant(torch, cf, warmup: int) -> dict:
    """config 5: every weight of a 7B model, bf16 -> int8 + scales -> bf16, through the
    grouped entry points (aggregate) and one call per tensor (for comparison, and
    per-tensor rates)."""
    gen = torch.Generator(device="cuda").manual_seed(5)
    shapes = [(4096, 4096)] * 4 + [(11008, 4096)] * 2 + [(4096, 11008)]
    lib = cf._lib.load()
    per_shape = {}
    tensors = []
    for layer in range(32):
        for i, shape in enumerate(shapes):
            x = with_outliers(torch, gen, 0.02 * torch.randn(*shape, generator=gen, device="cuda"), 0.001, 50.0)
            tensors.append((f"{shape[0]}x{shape[1]}", x.to(torch.bfloat16)))
            del x
    total_n = sum(t.numel() for _, t in tensors)
    q_all = [torch.empty(t.numel(), dtype=torch.int8, device="cuda") for _, t in tensors]
    s_all = [torch.empty((t.numel() + 63) // 64, device="cuda") for _, t in tensors]
    y_all = [torch.empty_like(t) for _, t in tensors]
    stream = torch.cuda.current_stream().cuda_stream

    def quant_all():
        for (_, t), q, s in zip(tensors, q_all, s_all):
            cf._lib.check(lib.cf_quantize_int8(t.data_ptr(), cf._lib.CF_BF16, q.data_ptr(), s.data_ptr(), t.numel(), stream))

    def dequant_all():
        for (_, t), q, s, y in zip(tensors, q_all, s_all, y_all):
            cf._lib.check(lib.cf_dequantize_int8(q.data_ptr(), s.data_ptr(), y.data_ptr(), cf._lib.CF_BF16, t.numel(), stream))

    # The same weight set through the grouped entry points: up to 48 tensors
    # per launch (5 launches instead of 224).
    ptr = cf._lib.pointer_array
    x_ptrs = ptr([t.data_ptr() for _, t in tensors])
    q_ptrs = ptr([q.data_ptr() for q in q_all])
    s_ptrs = ptr([s.data_ptr() for s in s_all])
    y_ptrs = ptr([y.data_ptr() for y in y_all])
    counts = cf._lib.int64_array([t.numel() for _, t in tensors])

    def quant_group():
        cf._lib.check(lib.cf_quantize_int8_group(x_ptrs, cf._lib.CF_BF16, q_ptrs, s_ptrs, counts, len(tensors), stream))

    def dequant_group():
        cf._lib.check(lib.cf_dequantize_int8_group(q_ptrs, s_ptrs, y_ptrs, cf._lib.CF_BF16, counts, len(tensors),
                                                   stream))

    qt = summary(time_launches(torch, [quant_group], 1, 3))
    dt = summary(time_launches(torch, [dequant_group], 1, 3))
    qt1 = summary(time_launches(torch, [quant_all], 1, 3))
    dt1 = summary(time_launches(torch, [dequant_all], 1, 3))
    qb = sum(bytes_quant(t.numel(), 2) for _, t in tensors)
    db = sum(bytes_dequant(t.numel(), 2) for _, t in tensors)
    for label in sorted({lbl for lbl, _ in tensors}):
        t = next(tt for lbl, tt in tensors if lbl == label)
        q = next(q for (lbl, _), q in zip(tensors, q_all) if lbl == label)
        s = next(s for (lbl, _), s in zip(tensors, s_all) if lbl == label)
        y = next(y for (lbl, _), y in zip(tensors, y_all) if lbl == label)
        n = t.numel()
        tq = summary(time_launches(torch, [lambda: cf._lib.check(lib.cf_quantize_int8(
            t.data_ptr(), cf._lib.CF_BF16, q.data_ptr(), s.data_ptr(), n, stream))], warmup, 20))
        td = summary(time_launches(torch, [lambda: cf._lib.check(lib.cf_dequantize_int8(
            q.data_ptr(), s.data_ptr(), y.data_ptr(), cf._lib.CF_BF16, n, stream))], warmup, 20))
        per_shape[label] = {"quantize_GB/s": gbs(bytes_quant(n, 2), tq["median_ms"]),
                            "dequantize_GB/s": gbs(bytes_dequant(n, 2), td["median_ms"])}
    return {
        "bulk_7b_quantize_bf16": {"elements": total_n, "bytes": qb, "ms": qt["median_ms"], "entry": "grouped",
                                  "GB/s": gbs(qb, qt["median_ms"]), "frac_hbm": gbs(qb, qt["median_ms"]) / PEAK_HBM_GBS},
        "bulk_7b_dequantize_bf16": {"elements": total_n, "bytes": db, "ms": dt["median_ms"], "entry": "grouped",
                                    "GB/s": gbs(db, dt["median_ms"]), "frac_hbm": gbs(db, dt["median_ms"]) / PEAK_HBM_GBS},
        "bulk_7b_quantize_bf16_per_tensor_calls": {
            "ms": qt1["median_ms"], "GB/s": gbs(qb, qt1["median_ms"]), "frac_hbm": gbs(qb, qt1["median_ms"]) / PEAK_HBM_GBS},
        "bulk_7b_dequantize_bf16_per_tensor_calls": {
            "ms": dt1["median_ms"], "GB/s": gbs(db, dt1["median_ms"]), "frac_hbm": gbs(db, dt1["median_ms"]) / PEAK_HBM_GBS},
        "bulk_7b_per_tensor_warm": per_shape,
    }


def cpu_baseline(seconds: float) -> dict | None:
    """The reference's CPU operators (oracle/_ref) on configs[1]'s step, each op timed
    for about `seconds` of CPU work."""
    from oracle import ref_runner

    if not ref_runner.available():
        return None
    threads = int(os.environ.get("OMP_NUM_THREADS", os.cpu_count() or 1))
    results = {}
    for op, shape in (("rmsnorm", [16384, 4096]), ("softmax", [1024, 2048])):
        proc = subprocess.run(
            [sys.executable, "-m", "oracle.ref_runner", "time", op, "--shape", *map(str, shape),
             "--dtype", "bf16", "--seconds", str(seconds), "--threads", str(threads)],
            capture_output=True, text=True, cwd=str(ROOT), env={**os.environ, "PYTHONPATH": str(ROOT)},
        )
        if proc.returncode != 0:
            log(f"cpu baseline for {op} failed: {proc.stderr[-400:]}")
            return None
        results[op] = json.loads(proc.stdout.strip().splitlines()[-1])
    rms_bytes = bytes_rmsnorm(16384, 4096, 2)
    sm_bytes = bytes_softmax(1024, 2048, 2)
    total_s = results["rmsnorm"]["median_s"] + results["softmax"]["median_s"]
    return {
        "value": (rms_bytes + sm_bytes) / total_s / 1e9,
        "unit": "GB/s",
        "cores": results["rmsnorm"]["threads"],
        "kind": "reference",
        "sample": ("reference CPU operators (cpp/src/bindings.cpp rmsnorm_cpu + softmax_cpu via ATen) on "
                   "the configs[1] step itself: RMSNorm bf16 [16384, 4096] + softmax bf16 [1024, 2048] on "
                   "causal-masked N(0, 4) logits; "
                   f"median of the calls made in ~{seconds:.0f} s per op (at least 5)"),
        "rmsnorm_median_s": results["rmsnorm"]["median_s"],
        "softmax_median_s": results["softmax"]["median_s"],
        "host_cpu_count": results["rmsnorm"]["cpu_count"],
    }


def _sig(v, digits: int = 4):
    """A float rounded to `digits` significant digits (keeps the stdout line short)."""
    if isinstance(v, float):
        return float(f"{v:.{digits}g}")
    return v


# Summary fields of the stdout line: (config, field) -> (breakdown key, entry field).
# Kernel-timestamp medians for kernels of tens of microseconds and more; the ~15 us
# config-1 kernels take the launch-to-launch median of back-to-back batches (their
# per-dispatch timestamps read 10-30% long on some runs), as config 5 does.
SUMMARY_FIELDS = {
    "c1": {"quantize_GB/s": ("quantize_f32_4096x4096", "GB/s"),
           "quantize_frac_hbm": ("quantize_f32_4096x4096", "frac_hbm"),
           "dequantize_GB/s": ("dequantize_f32_4096x4096", "GB/s"),
           "dequantize_frac_hbm": ("dequantize_f32_4096x4096", "frac_hbm")},
    "c2": {"rmsnorm_GB/s": ("rmsnorm_bf16_16384x4096", "kernel_GB/s"),
           "rmsnorm_frac_hbm": ("rmsnorm_bf16_16384x4096", "kernel_frac_hbm"),
           "softmax_us": ("softmax_bf16_causal_1024x2048", "graph_median_ms")},
    "c3": {"fused_TFLOP/s": ("lora_bf16_8192x4096x4096_r16", "kernel_TFLOP/s"),
           "fused_frac_mfma": ("lora_bf16_8192x4096x4096_r16", "kernel_frac_peak"),
           "fused_us": ("lora_bf16_8192x4096x4096_r16", "median_ms"),
           "hipblaslt_gemm_us": ("hipblaslt_gemm_bf16_8192x4096x4096_context", "median_ms"),
           "hipblaslt_gemm_TFLOP/s": ("hipblaslt_gemm_bf16_8192x4096x4096_context", "TFLOP/s"),
           "backward_GB/s": ("lora_backward_bf16_8192x4096x4096_r16", "kernel_GB/s"),
           "backward_frac_hbm": ("lora_backward_bf16_8192x4096x4096_r16", "kernel_frac_hbm")},
    "c4": {"tokens/s": ("block_c4_bf16_8x512_h4096", "tokens/s")},
    "c5": {"quantize_GB/s": ("bulk_7b_quantize_bf16", "GB/s"),
           "quantize_frac_hbm": ("bulk_7b_quantize_bf16", "frac_hbm"),
           "dequantize_GB/s": ("bulk_7b_dequantize_bf16", "GB/s"),
           "dequantize_frac_hbm": ("bulk_7b_dequantize_bf16", "frac_hbm")},
}


def config_summary(breakdown: dict) -> dict:
    """One or a few numbers per configuration, picked from the full breakdown."""
    out = {}
    for config, fields in SUMMARY_FIELDS.items():
        picked = {}
        for name, (key, field) in fields.items():
            value = breakdown.get(key, {}).get(field)
            if value is None:
                continue
            if name.endswith("_us"):
                value = value * 1e3
            picked[name] = _sig(value)
        if picked:
            out[config] = picked
    return out


STDOUT_LINE_LIMIT = 4000  # bytes; the driver parses the last stdout line


def profiled_traffic() -> float | None:
    """HBM bytes per RMSNorm launch from the committed rocprofv3 counter summary."""
    path = ROOT / "profiles" / "rmsnorm_bf16_c2_traffic.md"
    if not path.exists():
        return None
    match = re.search(r"traffic_bytes_per_launch:\s*([0-9.eE+]+)", path.read_text(encoding="utf-8"))
    return float(match.group(1)) if match else None


def main(argv: list[str] | None = None) -> int:
    parser = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    parser.add_argument("--gpus", type=int, default=1)
    parser.add_argument("--steps", type=int, default=200)
    parser.add_argument("--warmup", type=int, default=400)
    parser.add_argument("--runs", type=int, default=40, help="launches per timed batch (5 batches) per breakdown kernel")
    parser.add_argument("--cpu-seconds", type=float, default=10.0)
    parser.add_argument("--no-cpu-baseline", action="store_true")
    parser.add_argument("--quick", action="store_true", help="skip the breakdown (main step only)")
    parser.add_argument("--configs", default="1,ceiling,reference,2,reduce,3,4,5,paged,tensorcore,fp8",
                        help="breakdown configs to run (comma-separated: 1-5, ceiling, reference, "
                             "reduce, paged, tensorcore, fp8)")
    parser.add_argument("--detail", default=str(ROOT / "gpurun_out" / "bench_detail.json"),
                        help="write the full result JSON, with every breakdown entry, here ('' for none)")
    args = parser.parse_args(argv)

    if args.gpus != 1:
        print(f"bench.py: --gpus {args.gpus} is not supported; this build measures one MI355X "
              "(the hot path has no cross-GPU component, see DESIGN.md on sharding)", file=sys.stderr)
        return 2

    import torch

    import cuda_force_amd as cf
    import cuda_force_amd._lib  # noqa: F401

    if not cf.backend_report().using_custom_kernels:
        raise SystemExit(f"HIP kernels are not active: {cf.backend_report()}")
    torch.cuda.set_device(0)
    log(f"device: {torch.cuda.get_device_name(0)}")

    main_step = bench_main_step(torch, cf, args.steps, args.warmup)
    log(f"main step: {main_step['ms_per_step']:.4f} ms, rmsnorm avg {main_step['rmsnorm_avg_ms']:.4f} ms")
    # One plain copy of known size (256 MiB read + 256 MiB written): the
    # calibration kernel for rocprofv3's FETCH_SIZE / WRITE_SIZE counters.
    calib = torch.empty(2, 1 << 28, dtype=torch.uint8, device="cuda")
    cf._lib.check(cf._lib.load().cf_copy_bytes(calib[0].data_ptr(), calib[1].data_ptr(), 1 << 28,
                                               torch.cuda.current_stream().cuda_stream))
    torch.cuda.synchronize()
    del calib
    breakdown = {}
    if not args.quick:
        wanted = {c.strip() if not c.strip().isdigit() else f"config{c.strip()}"
                  for c in args.configs.split(",") if c.strip()}
        for name, fn in (("config1", lambda: bench_quant(torch, cf, args.warmup, args.runs)),
                         ("ceiling", lambda: bench_ceiling(torch, cf, args.warmup, args.runs)),
                         ("reference", lambda: bench_reference_shapes(torch, cf, args.warmup, args.runs)),
                         ("config2", lambda: bench_rowops(torch, cf, args.warmup, args.runs)),
                         ("reduce", lambda: bench_reduce(torch, cf, args.warmup, args.runs)),
                         ("config3", lambda: bench_lora(torch, cf, args.warmup, args.runs)),
                         ("config4", lambda: bench_block(torch, cf, 20, args.runs)),
                         ("config5", lambda: bench_bulk_quant(torch, cf, 3)),
                         ("paged", lambda: bench_paged(torch, cf, args.warmup, args.runs)),
                         ("tensorcore", lambda: bench_tensor_core(torch, cf, 20, args.runs)),
                         ("fp8", lambda: bench_fp8(torch, cf, 20, args.runs))):
            if name not in wanted:
                continue
            log(f"breakdown {name}")
            breakdown.update(fn())
            torch.cuda.empty_cache()

    baseline = None if args.no_cpu_baseline else cpu_baseline(args.cpu_seconds)
    value = main_step["bytes_per_step"] / (main_step["ms_per_step"] * 1e-3) / 1e9
    achieved = main_step["rmsnorm_bytes"] / (main_step["rmsnorm_avg_ms"] * 1e-3) / 1e9
    line = {
        "metric": METRIC,
        "value": value,
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": main_step["ms_per_step"],
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (seeded torch.randn on the GPU; causal -inf mask on the logits)",
        "config": {
            "workload": "configs[1]: RMSNorm bf16 [16384,4096] eps 1e-6 + causal softmax bf16 [1024,2048], one pass each",
            "rmsnorm": [16384, 4096],
            "softmax": [1024, 2048],
            "bytes_per_step": main_step["bytes_per_step"],
            "buffer_sets": main_step["buffer_sets"],
            "parallelism": "single GPU",
        },
        "roofline": {
            "bound": "hbm",
            "kernel": "rmsnorm_tile_kernel<bf16, 512 vectors, 2 per lane, 256 threads>",
            "achieved": achieved,
            "peak": PEAK_HBM_GBS,
            "unit": "GB/s",
            "frac": achieved / PEAK_HBM_GBS,
            "traffic": profiled_traffic(),
        },
        "cpu_baseline": baseline,
        "configs": config_summary(breakdown),
    }
    if args.detail:
        try:
            Path(args.detail).parent.mkdir(parents=True, exist_ok=True)
            Path(args.detail).write_text(json.dumps({**line, "breakdown": breakdown}, indent=2) + "\n",
                                         encoding="utf-8")
            log(f"full breakdown written to {args.detail}")
        except OSError as exc:
            log(f"could not write {args.detail}: {exc}")
    for config, figures in line["configs"].items():
        log(f"{config}: {json.dumps(figures)}")
    text = json.dumps(line, separators=(",", ":"))
    if len(text) > STDOUT_LINE_LIMIT:
        log(f"summary line is {len(text)} bytes; dropping the per-config figures from it")
        line["configs"] = None
        text = json.dumps(line, separators=(",", ":"))
    print(text, flush=True)
    return 0


if __name__ == "__main__":
    raise SystemExit(main())
