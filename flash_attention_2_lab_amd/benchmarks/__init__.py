"""Benchmark harness for the attention entry points, mirroring the reference's
``benchmarks/`` package (workloads, kernel registry, event-timed harness and the
``benchmark_forward`` command line), with TFLOP/s and fraction-of-peak columns.

Run ``python -m flash_attention_2_lab_amd.benchmarks --help``.
"""

from .harness import BenchmarkConfig, BenchmarkResult, benchmark_operation, percentile
from .kernels import KERNELS, KernelSpec, find_kernel
from .workloads import AttentionInputs, AttentionWorkload, attention_flops, generate_attention_inputs

__all__ = [
    "AttentionInputs", "AttentionWorkload", "BenchmarkConfig", "BenchmarkResult", "KERNELS",
    "KernelSpec", "attention_flops", "benchmark_operation", "find_kernel",
    "generate_attention_inputs", "percentile",
]
