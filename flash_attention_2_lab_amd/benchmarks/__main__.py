"""Command line of the benchmark harness (reference benchmarks/benchmark_forward.py:23-134):
same flags and per-kernel median/p10/p90 lines, plus TFLOP/s, the fraction of the
FP16 dense MFMA peak, and the latency ratio against SDPA.

    python -m flash_attention_2_lab_amd.benchmarks --dtype float16 --query-length 1024 \\
        --kernels tensorcore_production_128x128 pytorch_sdpa
"""

from __future__ import annotations

import argparse
import json
import sys

import torch

from .harness import BenchmarkConfig, benchmark_operation
from .kernels import KERNELS
from .workloads import AttentionWorkload, attention_flops, generate_attention_inputs

DTYPES: dict[str, torch.dtype] = {
    "float32": torch.float32,
    "float16": torch.float16,
    "bfloat16": torch.bfloat16,
}

MI355X_FP16_DENSE_TFLOPS = 2516.6  # 256 CUs x 4 SIMDs x 1024 FLOP/clk x 2.4 GHz


def build_parser() -> argparse.ArgumentParser:
    parser = argparse.ArgumentParser(prog="python -m flash_attention_2_lab_amd.benchmarks")
    parser.add_argument("--batch", type=int, default=1)
    parser.add_argument("--heads", type=int, default=8)
    parser.add_argument("--query-length", type=int, default=512)
    parser.add_argument("--key-length", type=int, default=None)
    parser.add_argument("--head-dim", type=int, default=64)
    parser.add_argument("--causal", action="store_true")
    parser.add_argument("--dtype", type=str, choices=list(DTYPES), default="float32")
    parser.add_argument("--samples", type=int, default=20)
    parser.add_argument("--iterations", type=int, default=100)
    parser.add_argument("--warmup", type=int, default=25)
    parser.add_argument("--kernels", nargs="+", default=None,
                        help="Kernel names to benchmark (default: every supported kernel).")
    parser.add_argument("--peak-tflops", type=float, default=MI355X_FP16_DENSE_TFLOPS,
                        help="Peak used for the fraction-of-peak column.")
    parser.add_argument("--json", action="store_true", help="Also print one JSON line per kernel.")
    parser.add_argument("--graph", action="store_true",
                        help="Time replays of a HIP graph of each sample's calls (device kernels only).")
    return parser


def main(argv: list[str] | None = None) -> int:
    args = build_parser().parse_args(argv)
    workload = AttentionWorkload(
        batch=args.batch, heads=args.heads, query_length=args.query_length,
        key_length=args.key_length if args.key_length is not None else args.query_length,
        head_dimension=args.head_dim, dtype=DTYPES[args.dtype], causal=args.causal,
    )
    config = BenchmarkConfig(warmup_iterations=args.warmup, samples=args.samples,
                             iterations_per_sample=args.iterations, graph=args.graph)
    inputs = generate_attention_inputs(workload)
    flops = attention_flops(workload)

    print(f"GPU:      {torch.cuda.get_device_name()}")
    print(f"Workload: {workload.label}")
    print()
    unknown = set(args.kernels or ()) - {spec.name for spec in KERNELS}
    if unknown:
        print(f"unknown kernels: {', '.join(sorted(unknown))}", file=sys.stderr)
        return 2
    results = []
    for spec in KERNELS:
        if args.kernels is not None and spec.name not in args.kernels:
            continue
        if not spec.supported(workload):
            print(f"{spec.name:30s} unsupported")
            continue
        cpu_config = config if spec.on_device else BenchmarkConfig(1, max(1, min(args.samples, 3)), 1)
        result = benchmark_operation(spec.name, lambda spec=spec: spec.function(inputs, workload),
                                     cpu_config, flops=flops, on_device=spec.on_device)
        results.append(result)
        peak_frac = result.median_tflops / args.peak_tflops
        print(f"{result.kernel_name:30s} median={result.median_ms:9.4f} ms  "
              f"p10={result.p10_ms:9.4f} ms  p90={result.p90_ms:9.4f} ms  "
              f"{result.median_tflops:8.2f} TFLOP/s  {100 * peak_frac:5.1f}% of peak")
        if args.json:
            print(json.dumps({"kernel": result.kernel_name, "median_ms": result.median_ms,
                              "p10_ms": result.p10_ms, "p90_ms": result.p90_ms,
                              "min_ms": result.minimum_ms, "max_ms": result.maximum_ms,
                              "tflops": result.median_tflops, "peak_fraction": peak_frac,
                              "workload": workload.label, "graph": bool(args.graph and spec.on_device)}))
    baseline = next((r for r in results if r.kernel_name == "pytorch_sdpa"), None)
    if baseline is not None:
        print()
        for result in results:
            print(f"{result.kernel_name:30s} {result.median_ms / baseline.median_ms:8.2f}x SDPA latency")
    return 0


if __name__ == "__main__":
    sys.exit(main())
