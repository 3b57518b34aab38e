"""Event-timed benchmark loop (reference benchmarks/harness.py:11-70).

Warmup, then `samples` samples of `iterations_per_sample` back-to-back calls, each
sample bracketed by device events (host clock for CPU operations); the per-call
time of every sample feeds median, min, p10, p90 and max. Percentiles are the
nearest-rank values at index round((n - 1) * fraction) of the sorted samples, the
reference's definition, so the two harnesses report comparable statistics.

With `graph` set (an addition of this harness, off by default), the
`iterations_per_sample` calls are captured once in a HIP graph and every sample
replays it between the events: the calls then run back to back on the device with
no host launches between them, which measures the kernels where eager calls are
bound by the host's launch rate.
"""

from __future__ import annotations

import statistics
import time
from collections.abc import Callable
from dataclasses import dataclass

import torch


@dataclass(frozen=True)
class BenchmarkConfig:
    warmup_iterations: int = 25
    samples: int = 20
    iterations_per_sample: int = 100
    graph: bool = False


@dataclass(frozen=True)
class BenchmarkResult:
    kernel_name: str
    median_ms: float
    minimum_ms: float
    p10_ms: float
    p90_ms: float
    maximum_ms: float
    flops: float = 0.0

    @property
    def median_tflops(self) -> float:
        return self.flops / (self.median_ms * 1e-3) / 1e12 if self.median_ms > 0 else 0.0


def percentile(values: list[float], fraction: float) -> float:
    if not values:
        raise ValueError("percentile of an empty list")
    ordered = sorted(values)
    return ordered[round((len(ordered) - 1) * fraction)]


def _capture(operation: Callable[[], object], iterations: int) -> torch.cuda.CUDAGraph:
    # Lazy set-up (allocator, library handles) happens on a side stream before capture.
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        operation()
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        for _ in range(iterations):
            operation()
    graph.replay()
    torch.cuda.synchronize()
    return graph


def _time_samples(operation: Callable[[], object], config: BenchmarkConfig, on_device: bool) -> list[float]:
    times_ms: list[float] = []
    if on_device:
        start = torch.cuda.Event(enable_timing=True)
        end = torch.cuda.Event(enable_timing=True)
        graph = _capture(operation, config.iterations_per_sample) if config.graph else None
        for _ in range(config.samples):
            start.record()
            if graph is not None:
                graph.replay()
            else:
                for _ in range(config.iterations_per_sample):
                    operation()
            end.record()
            end.synchronize()
            times_ms.append(start.elapsed_time(end) / config.iterations_per_sample)
    else:
        for _ in range(config.samples):
            t0 = time.perf_counter()
            for _ in range(config.iterations_per_sample):
                operation()
            times_ms.append((time.perf_counter() - t0) * 1e3 / config.iterations_per_sample)
    return times_ms


def benchmark_operation(name: str, operation: Callable[[], object], config: BenchmarkConfig,
                        *, flops: float = 0.0, on_device: bool = True) -> BenchmarkResult:
    """Time `operation` (a device operation unless `on_device` is False)."""
    with torch.inference_mode():
        for _ in range(config.warmup_iterations):
            operation()
        if on_device:
            torch.cuda.synchronize()
        times_ms = _time_samples(operation, config, on_device)
    return BenchmarkResult(
        kernel_name=name,
        median_ms=statistics.median(times_ms),
        minimum_ms=min(times_ms),
        p10_ms=percentile(times_ms, 0.10),
        p90_ms=percentile(times_ms, 0.90),
        maximum_ms=max(times_ms),
        flops=flops,
    )
