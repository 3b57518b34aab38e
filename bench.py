"""Benchmark of the MI355X FlashAttention-2 forward (FP16, D=64).

Prints ONE JSON line. The measured workload is the reference's headline
configuration, B=1 H=8 N=1024 D=64 FP16 (reference README.md:9-42): one step is
one noncausal forward plus one causal forward through the product entry point
`flash_attention_cuda.tensorcore_attention_forward_production_128x128`, on
synthetic inputs already resident in HBM.

Inside the timed region the K steps run as four batches of back-to-back calls in
mirrored order - K/2 noncausal, K/2 causal, the other K/2 causal, the other K/2
noncausal (the same work as K interleaved steps, with neither mode always first) -
with HIP events on the launch stream between the batches: the reference harness's
method (benchmarks/harness.py:34-71: events around back-to-back calls). Those events
give each kernel's average launch duration for the `roofline` object (the region's
first call, which the device starts from idle, is left out of that average);
wall-clock time between two device synchronisations, over all K steps, gives
`ms_per_step`.

Also reported (extra keys, each timed the same way after the main region):
`north_star` - B16 H16 N4096 noncausal and causal (the >=50%-of-MFMA-peak target)
and B2 H32 N16384 causal with sigma=2 logits; `cpu_baseline` - the oracle's FP32
CPU restatement of the reference (oracle.attention_reference) timed on this host's
cores (os.cpu_count() torch threads) on a bounded sample of the same workload, with
the other BASELINE configurations' CPU rates under `configs`; `graph_us` - the same
K calls per mode captured once in a HIP graph and replayed (per-call time, median of
three replays), for callers that capture launch-bound loops.

FLOPs: 4*B*H*N^2*D per forward, halved for causal. Bytes: 8*B*H*N*D (read Q, K, V
and write O once, FP16).
"""

from __future__ import annotations

import argparse
import json
import os
import sys
import time

MI355X_FP16_DENSE_TFLOPS = 2516.6  # 256 CUs x 4 SIMDs x 1024 FLOP/clk x 2.4 GHz
MI355X_HBM_GBPS = 8000.0

# Reference's published medians on an RTX 4070 Laptop GPU (reference README.md:21-42):
# N=1024 noncausal 65.7 us (runs 65.7/65.4/65.7), causal 53.4 us (53.1/55.4/53.4).
REFERENCE_US = {"noncausal": 65.7, "causal": 53.4}

METRIC = "fwd attention TFLOP/s + µs, B1 H8 N1024 D64 fp16, causal & noncausal"


def attention_flops(batch, heads, seq_len, head_dim, causal):
    flops = 4.0 * batch * heads * seq_len * seq_len * head_dim
    return flops / 2 if causal else flops


def attention_bytes(batch, heads, seq_len, head_dim):
    return 8.0 * batch * heads * seq_len * head_dim


def make_inputs(batch, heads, seq_len, *, seed=0, sigma=1.0, device="cpu"):
    import torch

    gen = torch.Generator().manual_seed(seed)
    shape = (batch, heads, seq_len, 64)
    q = torch.randn(shape, generator=gen)
    k = torch.randn(shape, generator=gen)
    v = torch.randn(shape, generator=gen)
    return tuple(t.half().to(device) for t in (q * sigma, k * sigma, v))


def time_kernel_batches(entry, inputs, modes, steps, warmup):
    """Runs `warmup` untimed rounds, then times `steps` calls per mode between HIP
    events on the current stream. With two modes the calls run as four back-to-back
    batches in mirrored order - first half of mode A, first half of mode B, second
    half of B, second half of A - so neither mode is always the one timed right after
    the warmup. Returns (wall_s, {mode: avg_s}).

    The wall clock covers all `steps` calls per mode. The per-call averages leave out
    the region's first call: after the opening synchronisation the device waits idle
    for the host to launch it, and that wait is not the kernel's duration. An event
    recorded right after that call is reached when it completes, and from there on the
    host launches ahead of the device, so the events time back-to-back kernels."""
    import torch

    q, k, v = inputs
    for _ in range(warmup):
        for causal in modes:
            entry(q, k, v, causal)
    first = steps // 2
    halves = [(causal, first) for causal in modes] + [(causal, steps - first) for causal in reversed(modes)]
    halves = [(causal, n) for causal, n in halves if n > 0]
    skip_first = steps > 1  # the first mode keeps at least one timed call
    stream = torch.cuda.current_stream()
    start = torch.cuda.Event(enable_timing=True)
    events = [torch.cuda.Event(enable_timing=True) for _ in range(len(halves) + 1)]
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    start.record(stream)
    for i, (causal, n) in enumerate(halves):
        for j in range(n):
            entry(q, k, v, causal)
            if i == 0 and j == 0:
                events[0].record(stream)
        events[i + 1].record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    per_kernel, calls = {}, {}
    for i, (causal, n) in enumerate(halves):
        mode = "causal" if causal else "noncausal"
        begin = events[i] if i > 0 or skip_first else start
        timed = n - 1 if i == 0 and skip_first else n
        per_kernel[mode] = per_kernel.get(mode, 0.0) + begin.elapsed_time(events[i + 1]) / 1e3
        calls[mode] = calls.get(mode, 0) + timed
    return wall, {mode: total / calls[mode] for mode, total in per_kernel.items()}


def time_in_graph(entry, inputs, modes, steps, replays=3):
    """Captures `steps` back-to-back calls per mode in one HIP graph each and times
    replays with HIP events. Returns {mode: median per-call seconds}."""
    import torch

    q, k, v = inputs
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):  # capture needs the lazy setup done off the capture stream
        for causal in modes:
            entry(q, k, v, causal)
    torch.cuda.current_stream().wait_stream(side)
    result = {}
    for causal in modes:
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            for _ in range(steps):
                entry(q, k, v, causal)
        graph.replay()
        times = []
        for _ in range(replays):
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record()
            graph.replay()
            e1.record()
            torch.cuda.synchronize()
            times.append(e0.elapsed_time(e1) / 1e3 / steps)
        result["causal" if causal else "noncausal"] = sorted(times)[len(times) // 2]
        del graph
    return result


REPO = os.path.dirname(os.path.abspath(__file__))
TRAFFIC_FILE = os.path.join(REPO, "profiles", "hbm_traffic.json")
# The kernel source the traffic figures were measured on: the committed summary records
# its SHA-256, and a summary taken on another version of the source is not reported.
KERNEL_SOURCE = os.path.join(REPO, "flash_attention_2_lab_amd", "csrc", "fa2_forward.hip")


def kernel_source_digest():
    import hashlib

    with open(KERNEL_SOURCE, "rb") as f:
        return hashlib.sha256(f.read()).hexdigest()


def measured_traffic(key):
    """(HBM bytes per launch, status) from the committed rocprofv3 FETCH_SIZE/WRITE_SIZE
    summary (calibrated on a plain copy). Bytes are None, with status "not profiled" or
    "stale", when that workload was not profiled or the summary was taken on another
    version of the kernel source."""
    try:
        with open(TRAFFIC_FILE) as f:
            summary = json.load(f)
        entry = summary["kernels"].get(key)
    except (OSError, ValueError, KeyError):
        return None, "not profiled"
    if entry is None:
        return None, "not profiled"
    if summary.get("source_sha256") != kernel_source_digest():
        return None, "stale"
    return entry["hbm_bytes"], "current"


def roofline(flops, avg_s, traffic_key=None):
    achieved = flops / avg_s / 1e12
    traffic, status = measured_traffic(traffic_key) if traffic_key else (None, "not profiled")
    return {"bound": "mfma", "achieved": round(achieved, 3), "peak": MI355X_FP16_DENSE_TFLOPS,
            "unit": "TFLOP/s", "frac": round(achieved / MI355X_FP16_DENSE_TFLOPS, 5),
            "traffic": traffic, "traffic_status": status}


# Workloads of the benchmark configurations: (batch, heads, seq_len, sigma).
WORKLOADS = {
    "b1h8n1024": (1, 8, 1024, 1.0),
    "b16h16n4096": (16, 16, 4096, 1.0),
    "b2h32n16384": (2, 32, 16384, 2.0),
}


# North-star workloads timed after the headline: (workload key, modes).
NORTH_STAR = (("b16h16n4096", (False, True)), ("b2h32n16384", (True,)))


def traffic_keys():
    """The rocprof traffic entries the bench line's roofline objects read."""
    keys = [f"b1h8n1024/{m}" for m in ("noncausal", "causal")]
    for workload, ns_modes in NORTH_STAR:
        keys += [f"{workload}/{'causal' if c else 'noncausal'}" for c in ns_modes]
    return keys


# Plain device-to-device copy of a known size: calibrates the FETCH_SIZE and
# WRITE_SIZE counters (each should read this many bytes per dispatch).
COPY_CALIBRATION_BYTES = 256 << 20
COPY_KERNEL = "__amd_rocclr_copyBuffer"


def _counter_kib(csv_path, kernel_prefix):
    """Median per-dispatch value (KiB) of the one counter in a rocprofv3 counter CSV, over
    the dispatches whose kernel name starts with `kernel_prefix`; also returns the name."""
    import csv

    values, names = [], set()
    with open(csv_path, newline="") as f:
        for row in csv.DictReader(f):
            if row["Kernel_Name"].startswith(kernel_prefix):
                values.append(float(row["Counter_Value"]))
                names.add(row["Kernel_Name"])
    if not values or len(names) != 1:
        raise ValueError(f"{csv_path}: expected one kernel named {kernel_prefix}*, found {sorted(names)}")
    values.sort()
    return values[len(values) // 2], names.pop()


def write_traffic_summary(run_dir):
    """Builds profiles/hbm_traffic.json from rocprofv3 counter runs under `run_dir`, one
    counter and one mode per run:
        rocprofv3 --pmc <C> -f csv -d <run_dir>/<W>_<M>_<C> -o run -- python3 bench.py --only <W> --mode <M>
    for C in FETCH_SIZE, WRITE_SIZE, each traffic key <W>/<M>, and <W>_<M> = copy_both. Each
    counter is scaled by what it reads for the plain copy of known size; the summary
    records the SHA-256 of the kernel source it was measured on."""
    def csv_of(stem, counter):
        return os.path.join(run_dir, f"{stem}_{counter}", "run_counter_collection.csv")

    fetch_copy, _ = _counter_kib(csv_of("copy_both", "FETCH_SIZE"), COPY_KERNEL)
    write_copy, _ = _counter_kib(csv_of("copy_both", "WRITE_SIZE"), COPY_KERNEL)
    copy_kib = COPY_CALIBRATION_BYTES / 1024
    fetch_factor, write_factor = copy_kib / fetch_copy, copy_kib / write_copy
    summary = {"source_sha256": kernel_source_digest(),
               "calibration": {"kernel": COPY_KERNEL, "bytes": COPY_CALIBRATION_BYTES,
                               "fetch_kib": round(fetch_copy, 1), "write_kib": round(write_copy, 1),
                               "fetch_factor": round(fetch_factor, 4), "write_factor": round(write_factor, 4)},
               "kernels": {}}
    for key in traffic_keys():
        workload, mode = key.split("/")
        batch, heads, seq_len, _ = WORKLOADS[workload]
        stem = f"{workload}_{mode}"
        fetch, name = _counter_kib(csv_of(stem, "FETCH_SIZE"), "_ZN12_GLOBAL__N_1")
        write, name_w = _counter_kib(csv_of(stem, "WRITE_SIZE"), "_ZN12_GLOBAL__N_1")
        if name != name_w:
            raise ValueError(f"{key}: FETCH_SIZE run profiled {name}, WRITE_SIZE run {name_w}")
        hbm = 1024 * (fetch * fetch_factor + write * write_factor)
        algorithmic = attention_bytes(batch, heads, seq_len, 64)
        qkv = 6 * batch * heads * seq_len * 64
        summary["kernels"][key] = {
            "kernel": name, "fetch_kib_raw": round(fetch, 1), "write_kib_raw": round(write, 1),
            "hbm_bytes": int(round(hbm)), "algorithmic_bytes": int(algorithmic),
            "ratio": round(hbm / algorithmic, 3),
            "fetch_vs_qkv": round(1024 * fetch * fetch_factor / qkv, 3),
            "write_vs_o": round(1024 * write * write_factor / (qkv / 3), 3)}
    with open(TRAFFIC_FILE, "w") as f:
        json.dump(summary, f, indent=1)
        f.write("\n")
    print(json.dumps({"traffic_summary": TRAFFIC_FILE, "keys": sorted(summary["kernels"])}))
    return 0


def run_copy_calibration(args):
    import torch

    src = torch.empty(COPY_CALIBRATION_BYTES, dtype=torch.uint8, device="cuda").fill_(1)
    dst = torch.empty_like(src)
    for _ in range(args.warmup):
        dst.copy_(src)
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(args.steps):
        dst.copy_(src)
    e1.record()
    torch.cuda.synchronize()
    avg = e0.elapsed_time(e1) / 1e3 / args.steps
    print(json.dumps({"workload": "copy", "bytes_per_copy": COPY_CALIBRATION_BYTES,
                      "us": round(avg * 1e6, 3),
                      "GBps": round(2 * COPY_CALIBRATION_BYTES / avg / 1e9, 1)}), flush=True)
    return 0


# The vendor GEMM at the FP16 rate the attention kernels are priced against: one
# 8192^3 product (the vendor BLAS through torch.matmul, FP32 accumulation), on N(0,1) and on
# all-zero operands. It shows what the MFMA pipes sustain on random data at the board's
# power limit, with no softmax.
GEMM_SIZE = 8192


def run_gemm_ceiling(args):
    import torch

    gen = torch.Generator(device="cuda").manual_seed(0)
    out = {"workload": "gemm", "m_n_k": GEMM_SIZE, "dtype": "fp16", "steps": args.steps}
    for name in ("randn", "zeros"):
        a = torch.randn(GEMM_SIZE, GEMM_SIZE, device="cuda", dtype=torch.float16, generator=gen)
        b = torch.randn(GEMM_SIZE, GEMM_SIZE, device="cuda", dtype=torch.float16, generator=gen)
        if name == "zeros":
            a.zero_()
            b.zero_()
        c = torch.empty(GEMM_SIZE, GEMM_SIZE, device="cuda", dtype=torch.float16)
        for _ in range(args.warmup):
            torch.matmul(a, b, out=c)
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(args.steps):
            torch.matmul(a, b, out=c)
        e1.record()
        torch.cuda.synchronize()
        avg = e0.elapsed_time(e1) / 1e3 / args.steps
        tflops = 2 * GEMM_SIZE**3 / avg / 1e12
        out[name] = {"us": round(avg * 1e6, 1), "tflops": round(tflops, 1),
                     "frac": round(tflops / MI355X_FP16_DENSE_TFLOPS, 4)}
        del a, b, c
    print(json.dumps(out), flush=True)
    return 0


def run_single(entry, args):
    """Times one workload (used under rocprofv3); prints one JSON line."""
    if args.only == "copy":
        return run_copy_calibration(args)
    if args.only == "gemm":
        return run_gemm_ceiling(args)
    batch, heads, seq_len, sigma = WORKLOADS[args.only]
    modes = {"noncausal": (False,), "causal": (True,), "both": (False, True)}[args.mode]
    inputs = make_inputs(batch, heads, seq_len, sigma=sigma, device="cuda")
    _, per_kernel = time_kernel_batches(entry, inputs, modes, args.steps, args.warmup)
    out = {"workload": args.only, "steps": args.steps}
    for mode, avg in per_kernel.items():
        f = attention_flops(batch, heads, seq_len, 64, mode == "causal")
        out[mode] = {"us": round(avg * 1e6, 3), "tflops": round(f / avg / 1e12, 2)}
    print(json.dumps(out), flush=True)
    return 0


def _cpu_rate(batch, heads, seq_len, causal, sigma, budget_s, chunk=None, max_heads=None):
    """Times the oracle (FP32 torch on the CPU) on one workload: whole calls, or - for
    configurations whose score tensor does not fit (chunk set) - one (batch, head) at a
    time with the queries in chunks of `chunk` rows, over at most `max_heads` heads or
    until `budget_s` is spent. Returns (algorithmic FLOP/s, description)."""
    from oracle import attention_reference, attention_rows_fp32

    q, k, v = make_inputs(batch, heads, seq_len, sigma=sigma)
    if chunk is None:
        attention_reference(q, k, v, causal=causal)  # warmup
        runs, t0 = 0, time.perf_counter()
        while runs < 3 or time.perf_counter() - t0 < budget_s:
            attention_reference(q, k, v, causal=causal)
            runs += 1
        elapsed = time.perf_counter() - t0
        flops = runs * attention_flops(batch, heads, seq_len, 64, causal)
        return flops / elapsed, f"{runs} calls"
    done, t0 = 0, time.perf_counter()
    for bh in range(batch * heads):
        b, h = divmod(bh, heads)
        for i0 in range(0, seq_len, chunk):
            rows = [(b, h, i) for i in range(i0, min(seq_len, i0 + chunk))]
            attention_rows_fp32(q, k, v, rows, causal=causal)
        done += 1
        if (max_heads and done >= max_heads) or time.perf_counter() - t0 >= budget_s:
            break
    elapsed = time.perf_counter() - t0
    flops = done * attention_flops(1, 1, seq_len, 64, causal)
    return flops / elapsed, f"{done} of {batch * heads} heads, queries in chunks of {chunk}"


def cpu_baseline(budget_s):
    """Oracle (FP32 torch restatement of the reference) on this host's CPU cores, with
    torch using os.cpu_count() threads. `value` is the headline workload (one
    noncausal plus one causal B1 H8 N1024 call per step); `configs` holds the same
    rate for the other BASELINE configurations on bounded samples. The CPU computes
    every score even when causal; TFLOP/s use the algorithmic FLOPs (causal halved),
    as the GPU figures do."""
    import torch

    from oracle import attention_reference

    threads = os.cpu_count() or 1
    torch.set_num_threads(threads)
    q, k, v = make_inputs(1, 8, 1024)
    flops = 0.0
    runs = 0
    attention_reference(q, k, v, causal=False)  # warmup
    t0 = time.perf_counter()
    while time.perf_counter() - t0 < budget_s or runs < 2:
        for causal in (False, True):
            attention_reference(q, k, v, causal=causal)
            flops += attention_flops(1, 8, 1024, 64, causal)
        runs += 1
    elapsed = time.perf_counter() - t0
    configs = {}
    for n in (128, 256, 512, 1024):
        for causal in (False, True):
            rate, how = _cpu_rate(1, 8, n, causal, 1.0, budget_s / 16)
            configs[f"B1H8N{n}_{'causal' if causal else 'noncausal'}"] = {"tflops": round(rate / 1e12, 5),
                                                                            "sample": how}
    for causal in (False, True):
        rate, how = _cpu_rate(16, 16, 4096, causal, 1.0, budget_s / 2, chunk=4096, max_heads=8)
        configs[f"B16H16N4096_{'causal' if causal else 'noncausal'}"] = {"tflops": round(rate / 1e12, 5),
                                                                           "sample": how}
    rate, how = _cpu_rate(2, 32, 16384, True, 2.0, budget_s, chunk=2048, max_heads=2)
    configs["B2H32N16384_causal_sigma2"] = {"tflops": round(rate / 1e12, 5), "sample": how}
    return {"value": round(flops / elapsed / 1e12, 5), "unit": "TFLOP/s", "cores": threads,
            "kind": "port",
            "sample": f"{runs} steps of B1 H8 N1024 D64 (one noncausal + one causal "
                      f"oracle.attention_reference call each, FP32 CPU), {elapsed:.1f} s; "
                      f"configs: the other BASELINE configurations on the samples named",
            "ms_per_step": round(elapsed / runs * 1e3, 3),
            "affinity_cpus": len(os.sched_getaffinity(0)),
            "configs": configs}


def main() -> int:
    parser = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    parser.add_argument("--gpus", type=int, default=1)
    parser.add_argument("--steps", type=int, default=200)
    parser.add_argument("--warmup", type=int, default=30)
    parser.add_argument("--north-star-steps", type=int, default=20)
    parser.add_argument("--cpu-seconds", type=float, default=10.0)
    parser.add_argument("--skip-north-star", action="store_true")
    parser.add_argument("--skip-cpu", action="store_true")
    parser.add_argument("--only", choices=sorted(WORKLOADS) + ["copy", "gemm"],
                        help="time one workload only (for profilers); prints its own JSON line")
    parser.add_argument("--mode", choices=("noncausal", "causal", "both"), default="both")
    parser.add_argument("--traffic-from", metavar="DIR",
                        help="write profiles/hbm_traffic.json from the rocprofv3 counter runs in DIR "
                             "(no GPU work)")
    args = parser.parse_args()

    if args.traffic_from:
        return write_traffic_summary(args.traffic_from)

    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU only: the attention forward shards over "
              "batch*heads with no communication, so N>1 is not run here.", file=sys.stderr)
        return 2

    import torch

    import flash_attention_2_lab_amd as fa

    if not torch.cuda.is_available():
        print("bench.py needs a GPU", file=sys.stderr)
        return 2
    entry = fa.flash_attention_cuda.tensorcore_attention_forward_production_128x128

    if args.only:
        return run_single(entry, args)

    modes = (False, True)
    inputs = make_inputs(1, 8, 1024, device="cuda")
    wall, per_kernel = time_kernel_batches(entry, inputs, modes, args.steps, args.warmup)
    step_flops = sum(attention_flops(1, 8, 1024, 64, c) for c in modes)
    ms_per_step = wall / args.steps * 1e3
    value = step_flops / (wall / args.steps) / 1e12
    ref_step_s = sum(REFERENCE_US.values()) * 1e-6
    flops_by_mode = {"noncausal": attention_flops(1, 8, 1024, 64, False),
                     "causal": attention_flops(1, 8, 1024, 64, True)}
    dominant = max(per_kernel, key=lambda m: per_kernel[m])
    line = {
        "metric": METRIC,
        "value": round(value, 4),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": round(value / (step_flops / ref_step_s / 1e12), 4),
        "dtype": "f16",
        "data": "synthetic",
        "config": {"workload": "B1 H8 N1024 D64 fp16; one step = one noncausal + one causal forward",
                   "batch": 1, "heads": 8, "seq_len": 1024, "head_dim": 64,
                   "baseline_hardware": "RTX 4070 Laptop (reference README.md:21-42)"},
        "us": {m: round(t * 1e6, 3) for m, t in per_kernel.items()},
        "roofline": dict(roofline(flops_by_mode[dominant], per_kernel[dominant], f"b1h8n1024/{dominant}"),
                         kernel=dominant,
                         hbm_frac=round(attention_bytes(1, 8, 1024, 64) / per_kernel[dominant]
                                        / 1e9 / MI355X_HBM_GBPS, 5)),
    }
    graph = time_in_graph(entry, inputs, modes, args.steps)
    line["graph_us"] = {m: round(t * 1e6, 3) for m, t in graph.items()}
    del inputs

    if not args.skip_north_star:
        # Each north-star workload: 3 untimed calls per mode, then five timed batches of
        # --north-star-steps calls (mirrored halves per mode, as above); the median batch
        # gives `us`, and `us_batches` lists all five.
        north = {}
        for workload, ns_modes in NORTH_STAR:
            batch, heads, seq_len, sigma = WORKLOADS[workload]
            steps = args.north_star_steps if len(ns_modes) > 1 else max(2, args.north_star_steps // 4)
            name = workload.upper()
            data = make_inputs(batch, heads, seq_len, sigma=sigma, device="cuda")
            batches = []
            for rep in range(5):
                _, t = time_kernel_batches(entry, data, ns_modes, steps, 3 if rep == 0 else 0)
                batches.append(t)
            del data
            for mode in t:
                per_call = sorted(b[mode] for b in batches)
                avg = per_call[len(per_call) // 2]
                f = attention_flops(batch, heads, seq_len, 64, mode == "causal")
                key = f"{name}_{mode}" + ("_sigma2" if sigma != 1.0 else "")
                north[key] = {"us": round(avg * 1e6, 2), "tflops": round(f / avg / 1e12, 2),
                              "us_batches": [round(b[mode] * 1e6, 1) for b in batches],
                              "roofline": roofline(f, avg, f"{workload}/{mode}")}
        line["north_star"] = north

    if not args.skip_cpu:
        line["cpu_baseline"] = cpu_baseline(args.cpu_seconds)
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
