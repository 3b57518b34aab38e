"""Re-measures the forward's kernel choice: at every routing threshold of
`choose_kernel` (csrc/fa2_forward.hip), times the kernel the plan picks and its
neighbours across the threshold on the same inputs, through fa2_forward_with_kernel,
and reports whether the pick is still the fastest.

    python -m flash_attention_2_lab_amd.benchmarks.routing [--json] [--reps 7] [--calls 20]

Each kernel is timed by replaying a HIP graph of `--calls` back-to-back calls (no host
launch cost between them), `--reps` times, interleaved across the kernels of a shape;
the median replay gives the per-call time. A row is flagged when a neighbour beats the
pick by more than `--margin` (default 3%, about the spread of repeated same-process
runs); box-to-box spread is larger, so a flag is a prompt to re-measure, not a verdict.
"""

from __future__ import annotations

import argparse
import json
import statistics
import sys
from dataclasses import dataclass

import torch

from .. import capi
from .workloads import AttentionWorkload, attention_flops

K = capi
KERNEL_NAMES = {
    K.FA2_KERNEL_256_QUERY: "256-query", K.FA2_KERNEL_256_QUERY_PAIRS: "256-query pairs",
    K.FA2_KERNEL_128_QUERY: "128-query", K.FA2_KERNEL_128_QUERY_SPLIT_PAIRS: "128-query split pairs",
    K.FA2_KERNEL_KEY_SPLIT_64: "key-split 64", K.FA2_KERNEL_KEY_SPLIT_32: "key-split 32",
    K.FA2_KERNEL_KEY_SPLIT_8_WAVES: "key-split 8 waves", K.FA2_KERNEL_KEY_SPLIT_PAIRS16: "paired 16-query",
    K.FA2_KERNEL_KEY_SPLIT_64_DMA_WAVES: "key-split DMA waves",
}


@dataclass(frozen=True)
class Case:
    """One shape next to a routing threshold and the kernels to compare there."""
    rule: str
    batch: int
    heads: int
    seq_len: int
    causal: bool
    kernels: tuple[int, ...]


# Both sides of every threshold of choose_kernel, each with the kernels the rule decides
# between (the plan's pick is always timed as well).
CASES = (
    Case("wide vs 128-query, noncausal: 512 wide workgroups", 1, 32, 4096, False, (K.FA2_KERNEL_256_QUERY, K.FA2_KERNEL_128_QUERY)),
    Case("wide vs 128-query, noncausal: sparse last round (576)", 1, 36, 4096, False, (K.FA2_KERNEL_256_QUERY, K.FA2_KERNEL_128_QUERY)),
    Case("wide vs 128-query, noncausal: half-full last round (768)", 1, 48, 4096, False, (K.FA2_KERNEL_256_QUERY, K.FA2_KERNEL_128_QUERY)),
    Case("wide vs 128-query, noncausal: whole rounds", 16, 16, 4096, False, (K.FA2_KERNEL_256_QUERY, K.FA2_KERNEL_128_QUERY)),
    Case("wide vs 128-query, causal: 256 workgroups", 1, 32, 4096, True, (K.FA2_KERNEL_256_QUERY, K.FA2_KERNEL_128_QUERY)),
    Case("wide vs 128-query, causal: 512 workgroups", 1, 64, 4096, True, (K.FA2_KERNEL_256_QUERY, K.FA2_KERNEL_128_QUERY)),
    Case("pairs vs head groups, causal: T = 4, 1024 tiles", 16, 16, 1024, True, (K.FA2_KERNEL_256_QUERY, K.FA2_KERNEL_256_QUERY_PAIRS)),
    Case("pairs vs head groups, causal: T = 4, 2048 tiles", 32, 16, 1024, True, (K.FA2_KERNEL_256_QUERY, K.FA2_KERNEL_256_QUERY_PAIRS)),
    Case("pairs vs head groups, causal: T = 8", 8, 16, 2048, True, (K.FA2_KERNEL_256_QUERY, K.FA2_KERNEL_256_QUERY_PAIRS)),
    Case("head groups vs pairs, causal: T = 16 (throughput shape)", 16, 16, 4096, True, (K.FA2_KERNEL_256_QUERY, K.FA2_KERNEL_256_QUERY_PAIRS)),
    Case("head groups vs pairs, causal: T = 64", 2, 32, 16384, True, (K.FA2_KERNEL_256_QUERY, K.FA2_KERNEL_256_QUERY_PAIRS)),
    Case("pairs vs head groups, causal: T = 2, 2048 tiles", 64, 16, 512, True, (K.FA2_KERNEL_256_QUERY, K.FA2_KERNEL_256_QUERY_PAIRS)),
    Case("pairs vs head groups, causal: T = 2, 4096 tiles", 128, 16, 512, True, (K.FA2_KERNEL_256_QUERY, K.FA2_KERNEL_256_QUERY_PAIRS)),
    Case("128-query vs split pairs, causal: 2048 keys", 1, 32, 2048, True, (K.FA2_KERNEL_128_QUERY_SPLIT_PAIRS, K.FA2_KERNEL_128_QUERY)),
    Case("split pairs vs 128-query, causal: 4096 keys, 320 groups", 1, 10, 4096, True, (K.FA2_KERNEL_128_QUERY_SPLIT_PAIRS, K.FA2_KERNEL_128_QUERY)),
    Case("split pairs vs 128-query, causal: 4096 keys, 512 groups", 1, 16, 4096, True, (K.FA2_KERNEL_128_QUERY_SPLIT_PAIRS, K.FA2_KERNEL_128_QUERY)),
    Case("key-split vs split pairs, causal: 4096 keys, 256 groups", 1, 8, 4096, True, (K.FA2_KERNEL_128_QUERY_SPLIT_PAIRS, K.FA2_KERNEL_KEY_SPLIT_32)),
    Case("split pairs vs 128-query, causal: 8192 keys", 1, 8, 8192, True, (K.FA2_KERNEL_128_QUERY_SPLIT_PAIRS, K.FA2_KERNEL_128_QUERY)),
    Case("split pairs vs 128-query, causal: 16384 keys", 1, 4, 16384, True, (K.FA2_KERNEL_128_QUERY_SPLIT_PAIRS, K.FA2_KERNEL_128_QUERY)),
    Case("128-query vs key-split, noncausal: 200 groups", 1, 25, 1024, False, (K.FA2_KERNEL_128_QUERY, K.FA2_KERNEL_KEY_SPLIT_32)),
    Case("key-split vs 128-query, noncausal: 192 groups", 1, 24, 1024, False, (K.FA2_KERNEL_128_QUERY, K.FA2_KERNEL_KEY_SPLIT_32)),
    Case("key-split vs 128-query, noncausal: 192 groups of 4096 keys", 1, 6, 4096, False, (K.FA2_KERNEL_128_QUERY, K.FA2_KERNEL_KEY_SPLIT_32)),
    Case("128-query vs key-split, causal: 320 groups", 1, 40, 1024, True, (K.FA2_KERNEL_128_QUERY, K.FA2_KERNEL_KEY_SPLIT_32)),
    Case("128-query vs key-split, causal: 256 groups", 1, 32, 1024, True, (K.FA2_KERNEL_128_QUERY, K.FA2_KERNEL_KEY_SPLIT_32)),
    Case("paired 16-query vs key-split, causal: 512 keys", 1, 8, 512, True, (K.FA2_KERNEL_KEY_SPLIT_PAIRS16, K.FA2_KERNEL_KEY_SPLIT_32)),
    Case("paired 16-query vs key-split, causal: 1024 keys (bench)", 1, 8, 1024, True, (K.FA2_KERNEL_KEY_SPLIT_PAIRS16, K.FA2_KERNEL_KEY_SPLIT_32, K.FA2_KERNEL_KEY_SPLIT_8_WAVES)),
    Case("8 waves vs paired 16-query, causal: 2048 keys", 1, 4, 2048, True, (K.FA2_KERNEL_KEY_SPLIT_PAIRS16, K.FA2_KERNEL_KEY_SPLIT_8_WAVES)),
    Case("key-split 32 vs 64, causal: below the paired kernel's 512 keys", 1, 8, 384, True, (K.FA2_KERNEL_KEY_SPLIT_32, K.FA2_KERNEL_KEY_SPLIT_64)),
    Case("DMA waves vs key-split 64, noncausal: 1024 keys (bench)", 1, 8, 1024, False, (K.FA2_KERNEL_KEY_SPLIT_64_DMA_WAVES, K.FA2_KERNEL_KEY_SPLIT_64, K.FA2_KERNEL_KEY_SPLIT_8_WAVES)),
    Case("DMA waves vs key-split 64, noncausal: 768 keys", 1, 8, 768, False, (K.FA2_KERNEL_KEY_SPLIT_64_DMA_WAVES, K.FA2_KERNEL_KEY_SPLIT_64)),
    Case("8 waves vs DMA waves, noncausal: 2048 keys", 1, 4, 2048, False, (K.FA2_KERNEL_KEY_SPLIT_8_WAVES, K.FA2_KERNEL_KEY_SPLIT_64_DMA_WAVES)),
    Case("key-split 64 vs 32 by tiles per wave: 640 keys", 1, 8, 640, False, (K.FA2_KERNEL_KEY_SPLIT_64, K.FA2_KERNEL_KEY_SPLIT_32)),
    Case("key-split 64 vs 32 by blocks: 288 blocks", 1, 9, 1024, False, (K.FA2_KERNEL_KEY_SPLIT_32, K.FA2_KERNEL_KEY_SPLIT_64_DMA_WAVES)),
)


def _graph(kernel, q, k, v, out, causal, calls):
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        capi.forward_with_kernel(kernel, q, k, v, causal, output=out)
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        for _ in range(calls):
            capi.forward_with_kernel(kernel, q, k, v, causal, output=out)
    graph.replay()
    return graph


def measure(case: Case, reps: int, calls: int) -> dict:
    plan = capi.forward_plan(case.batch, case.heads, case.seq_len, case.causal)
    kernels = list(dict.fromkeys((plan,) + case.kernels))
    gen = torch.Generator().manual_seed(0)
    shape = (case.batch, case.heads, case.seq_len, 64)
    q, k, v = (torch.randn(shape, generator=gen).half().cuda() for _ in range(3))
    outs = {kern: torch.empty_like(q) for kern in kernels}
    graphs = {kern: _graph(kern, q, k, v, outs[kern], case.causal, calls) for kern in kernels}
    times = {kern: [] for kern in kernels}
    for _ in range(reps):
        for kern in kernels:
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record()
            graphs[kern].replay()
            e1.record()
            torch.cuda.synchronize()
            times[kern].append(e0.elapsed_time(e1) * 1e3 / calls)
    del graphs
    us = {kern: statistics.median(t) for kern, t in times.items()}
    best = min(us, key=us.get)
    flops = attention_flops(AttentionWorkload(case.batch, case.heads, case.seq_len, case.seq_len, 64,
                                              torch.float16, case.causal))
    return {"rule": case.rule, "shape": [case.batch, case.heads, case.seq_len], "causal": case.causal,
            "plan": KERNEL_NAMES[plan], "best": KERNEL_NAMES[best],
            "us": {KERNEL_NAMES[kern]: round(t, 2) for kern, t in us.items()},
            "tflops": {KERNEL_NAMES[kern]: round(flops / t / 1e6, 1) for kern, t in us.items()},
            "plan_over_best": round(us[plan] / us[best], 4)}


def main(argv: list[str] | None = None) -> int:
    parser = argparse.ArgumentParser(prog="python -m flash_attention_2_lab_amd.benchmarks.routing")
    parser.add_argument("--reps", type=int, default=7)
    parser.add_argument("--calls", type=int, default=20)
    parser.add_argument("--margin", type=float, default=0.03)
    parser.add_argument("--json", action="store_true", help="one JSON line per case instead of the table")
    args = parser.parse_args(argv)
    if not torch.cuda.is_available():
        print("the routing check needs a GPU", file=sys.stderr)
        return 2
    flagged = 0
    if not args.json:
        print(f"GPU: {torch.cuda.get_device_name()}")
        print(f"{'rule':60s} {'B H N':>14s} {'mode':9s} {'plan':22s} us per kernel")
    for case in CASES:
        row = measure(case, args.reps, args.calls)
        flag = row["plan_over_best"] > 1.0 + args.margin
        flagged += flag
        row["flagged"] = flag
        if args.json:
            print(json.dumps(row), flush=True)
        else:
            kernels = ", ".join(f"{name} {t:.1f}" for name, t in row["us"].items())
            shape = "x".join(str(x) for x in row["shape"])
            mode = "causal" if case.causal else "noncausal"
            print(f"{case.rule:60s} {shape:>14s} {mode:9s} {row['plan']:22s} {kernels}"
                  f"{'  <- ' + row['best'] + ' faster' if flag else ''}", flush=True)
    if not args.json:
        print(f"{flagged} of {len(CASES)} picks beaten by more than {args.margin:.0%}")
    return 0


if __name__ == "__main__":
    sys.exit(main())
