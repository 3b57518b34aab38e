"""GPU test of the benchmark harness command line on this library's entry points."""

from __future__ import annotations

import json

import pytest

from flash_attention_2_lab_amd.benchmarks.__main__ import main

pytestmark = pytest.mark.gpu


def test_cli_times_the_tensorcore_entries(capsys):
    status = main(["--dtype", "float16", "--heads", "2", "--query-length", "256",
                   "--samples", "3", "--iterations", "2", "--warmup", "1", "--json",
                   "--kernels", "tensorcore_production_128x128", "tensorcore_attention",
                   "tensorcore_attention_bc32", "naive_online"])
    out = capsys.readouterr().out
    assert status == 0
    assert "Workload: B=1, H=2, Nq=256, Nk=256, D=64, dtype=float16, causal=False" in out
    assert "naive_online" in out and "unsupported" in out  # an FP32 kernel on FP16 inputs
    rows = [json.loads(line) for line in out.splitlines() if line.startswith("{")]
    assert {r["kernel"] for r in rows} == {"tensorcore_production_128x128", "tensorcore_attention",
                                          "tensorcore_attention_bc32"}
    for r in rows:
        assert 0 < r["p10_ms"] <= r["median_ms"] <= r["p90_ms"]
        assert r["tflops"] > 0 and 0 < r["peak_fraction"] < 1


def test_cli_times_graph_replays(capsys):
    # --graph: each sample's calls captured once in a HIP graph and replayed between the
    # events; the result is a positive per-call time for the production entry and for
    # the device SDPA comparator.
    status = main(["--dtype", "float16", "--heads", "8", "--query-length", "256", "--causal",
                   "--samples", "3", "--iterations", "20", "--warmup", "2", "--json", "--graph",
                   "--kernels", "tensorcore_production_128x128", "pytorch_sdpa"])
    out = capsys.readouterr().out
    assert status == 0
    rows = {r["kernel"]: r for r in (json.loads(line) for line in out.splitlines() if line.startswith("{"))}
    assert set(rows) == {"tensorcore_production_128x128", "pytorch_sdpa"}
    for r in rows.values():
        assert r["graph"] is True
        assert 0 < r["p10_ms"] <= r["median_ms"] <= r["p90_ms"]


def test_cli_reports_unsupported_and_unknown_kernels(capsys):
    assert main(["--dtype", "float16", "--query-length", "80", "--samples", "1", "--iterations", "1",
                 "--warmup", "0", "--kernels", "tensorcore_production_128x128"]) == 0
    assert "tensorcore_production_128x128" in capsys.readouterr().out
    assert main(["--kernels", "no_such_kernel"]) == 2


def test_cli_times_the_fp32_simt_entries(capsys):
    status = main(["--dtype", "float32", "--heads", "2", "--query-length", "200", "--head-dim", "64",
                   "--samples", "3", "--iterations", "2", "--warmup", "1", "--json",
                   "--kernels", "naive_online", "block_online", "tiled_simt", "tilewise_simt",
                   "tensorcore_attention"])
    out = capsys.readouterr().out
    assert status == 0
    rows = [json.loads(line) for line in out.splitlines() if line.startswith("{")]
    assert {r["kernel"] for r in rows} == {"naive_online", "block_online", "tiled_simt", "tilewise_simt"}
    assert "tensorcore_attention" in out and "unsupported" in out
