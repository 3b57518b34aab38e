"""CPU tests of the benchmark harness (mirror of reference benchmarks/)."""

from __future__ import annotations

import pytest
import torch

from flash_attention_2_lab_amd import benchmarks as bm
from flash_attention_2_lab_amd.benchmarks.__main__ import build_parser


def test_percentile_is_nearest_rank_of_round_index():
    values = [5.0, 1.0, 4.0, 2.0, 3.0]
    assert bm.percentile(values, 0.0) == 1.0
    assert bm.percentile(values, 1.0) == 5.0
    assert bm.percentile(values, 0.5) == 3.0
    assert bm.percentile(values, 0.10) == 1.0   # round(0.4) = 0
    assert bm.percentile(values, 0.90) == 5.0   # round(3.6) = 4
    with pytest.raises(ValueError):
        bm.percentile([], 0.5)


def test_workload_shapes_label_and_flops():
    w = bm.AttentionWorkload(2, 3, 128, 256, 64, dtype=torch.float16, causal=False)
    assert w.query_shape == (2, 3, 128, 64)
    assert w.key_value_shape == (2, 3, 256, 64)
    assert w.label == "B=2, H=3, Nq=128, Nk=256, D=64, dtype=float16, causal=False"
    assert bm.attention_flops(w) == 4 * 2 * 3 * 128 * 256 * 64
    wc = bm.AttentionWorkload(1, 8, 1024, 1024, 64, dtype=torch.float16, causal=True)
    assert bm.attention_flops(wc) == 4 * 8 * 1024 * 1024 * 64 / 2


def test_inputs_are_seeded_and_drawn_in_q_k_v_order():
    w = bm.AttentionWorkload(1, 2, 32, 32, 64, dtype=torch.float16, seed=7)
    a = bm.generate_attention_inputs(w, device="cpu")
    b = bm.generate_attention_inputs(w, device="cpu")
    assert torch.equal(a.query, b.query) and torch.equal(a.value, b.value)
    gen = torch.Generator().manual_seed(7)
    q = torch.randn(w.query_shape, dtype=torch.float16, generator=gen)
    k = torch.randn(w.key_value_shape, dtype=torch.float16, generator=gen)
    assert torch.equal(a.query, q) and torch.equal(a.key, k)


@pytest.mark.parametrize("n, causal, expected", [
    (1024, False, {"tensorcore_attention", "tensorcore_attention_bc32", "tensorcore_bc32_raw_pv",
                   "tensorcore_bc32_raw_qk_raw_pv", "tensorcore_production_128x128"}),
    (1024, True, {"tensorcore_production_128x128"}),
    (80, False, {"tensorcore_attention"}),
    (96, False, {"tensorcore_attention", "tensorcore_attention_bc32", "tensorcore_bc32_raw_pv",
                 "tensorcore_bc32_raw_qk_raw_pv"}),
])
def test_support_predicates_follow_the_reference(n, causal, expected):
    # Reference benchmarks/kernels.py:186-239.
    w = bm.AttentionWorkload(1, 8, n, n, 64, dtype=torch.float16, causal=causal)
    ours = {s.name for s in bm.KERNELS if s.supported(w) and s.name.startswith("tensorcore")}
    assert ours == expected
    fp32 = bm.AttentionWorkload(1, 8, n, n, 64, dtype=torch.float32, causal=causal)
    assert not any(s.supported(fp32) for s in bm.KERNELS if s.name.startswith("tensorcore"))


@pytest.mark.parametrize("dtype, n, d, causal, expected", [
    (torch.float32, 100, 64, False, {"naive_online", "block_online", "tiled_simt", "tilewise_simt"}),
    (torch.float32, 100, 128, False, {"naive_online", "block_online"}),
    (torch.float32, 100, 64, True, set()),
    (torch.float32, 96, 32, False, set()),
    (torch.float16, 128, 64, False, set()),
])
def test_simt_support_predicates_follow_the_reference(dtype, n, d, causal, expected):
    # Reference benchmarks/kernels.py:137-183: FP32, square, D in {64, 128} (naive,
    # block) or 64 (tiled, tilewise), noncausal.
    w = bm.AttentionWorkload(1, 8, n, n, d, dtype=dtype, causal=causal)
    simt = {"naive_online", "block_online", "tiled_simt", "tilewise_simt"}
    assert {s.name for s in bm.KERNELS if s.name in simt and s.supported(w)} == expected
    rectangular = bm.AttentionWorkload(1, 8, n, n + 1, 64, dtype=torch.float32)
    assert not any(bm.find_kernel(name).supported(rectangular) for name in simt)


def test_device_sdpa_is_not_offered_in_bfloat16():
    w = bm.AttentionWorkload(1, 8, 128, 128, 64, dtype=torch.bfloat16)
    assert not bm.find_kernel("pytorch_sdpa").supported(w)
    assert bm.find_kernel("pytorch_sdpa_cpu").supported(w)


def test_cli_defaults_match_the_reference():
    # Reference benchmarks/benchmark_forward.py:26-52.
    args = build_parser().parse_args([])
    assert (args.batch, args.heads, args.query_length, args.key_length, args.head_dim) == (1, 8, 512, None, 64)
    assert (args.dtype, args.samples, args.iterations, args.warmup, args.causal) == ("float32", 20, 100, 25, False)
    # This harness's additions are off by default: eager timing, as the reference's.
    assert args.graph is False and args.json is False
    assert build_parser().parse_args(["--graph"]).graph is True


def test_host_timing_path_and_cpu_comparator():
    w = bm.AttentionWorkload(1, 2, 64, 64, 64, dtype=torch.float16)
    inputs = bm.generate_attention_inputs(w, device="cpu")
    spec = bm.find_kernel("pytorch_sdpa_cpu")
    out = spec.function(inputs, w)
    assert out.shape == w.query_shape and out.dtype == torch.float32
    result = bm.benchmark_operation(spec.name, lambda: spec.function(inputs, w),
                                    bm.BenchmarkConfig(1, 3, 2), flops=bm.attention_flops(w),
                                    on_device=False)
    assert result.minimum_ms <= result.median_ms <= result.maximum_ms
    assert result.p10_ms <= result.p90_ms
    assert result.median_tflops > 0


def test_bench_traffic_keys_are_measured():
    # Every roofline object of bench.py's line names its HBM traffic from the committed
    # rocprofv3 FETCH_SIZE/WRITE_SIZE summary; a missing entry would report null.
    import importlib.util
    from pathlib import Path

    root = Path(__file__).resolve().parents[1]
    spec = importlib.util.spec_from_file_location("bench_module", root / "bench.py")
    bench = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(bench)
    keys = set(bench.traffic_keys())
    assert {"b1h8n1024/noncausal", "b1h8n1024/causal", "b16h16n4096/noncausal", "b16h16n4096/causal",
            "b2h32n16384/causal"} <= keys
    import json

    summary = json.loads(Path(bench.TRAFFIC_FILE).read_text())
    assert len(summary["source_sha256"]) == 64  # the kernel source it was measured on
    for key in sorted(keys):
        entry = summary["kernels"][key]
        assert isinstance(entry["hbm_bytes"], int) and entry["hbm_bytes"] > 0, key
        # Reported only while the kernel source is the profiled one (else null, "stale").
        traffic, status = bench.measured_traffic(key)
        assert (traffic, status) in ((entry["hbm_bytes"], "current"), (None, "stale")), key
