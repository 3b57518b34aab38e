"""CPU tests of bench.py's host logic: the timed-region bookkeeping and the one-GPU rule.

The device is replaced by a simulated clock: each fake launch advances it by the
kernel's duration (plus an idle gap before the region's first call, as after a device
synchronisation), and each fake event reads it when recorded. No GPU is used.
"""

from __future__ import annotations

import subprocess
import sys
from pathlib import Path

import pytest
import torch

import bench

REPO_ROOT = Path(__file__).resolve().parents[1]


class _Clock:
    def __init__(self, durations, idle_before_first):
        self.now = 0.0
        self.calls = []
        self.durations = durations
        self.idle = idle_before_first

    def entry(self, q, k, v, causal):
        if not self.calls:
            self.now += self.idle
        self.calls.append(causal)
        self.now += self.durations[causal]


@pytest.fixture
def fake_device(monkeypatch):
    clock = _Clock({False: 7e-6, True: 6e-6}, idle_before_first=20e-6)

    class Event:
        def __init__(self, enable_timing=False):
            self.t = None

        def record(self, stream=None):
            self.t = clock.now

        def elapsed_time(self, other):  # milliseconds, as torch.cuda.Event
            return (other.t - self.t) * 1e3

    monkeypatch.setattr(torch.cuda, "Event", Event)
    monkeypatch.setattr(torch.cuda, "current_stream", lambda: None)
    monkeypatch.setattr(torch.cuda, "synchronize", lambda: None)
    return clock


@pytest.mark.parametrize("steps", [2, 3, 20, 200])
def test_per_call_averages_leave_out_the_idle_start(fake_device, steps):
    _, per_mode = bench.time_kernel_batches(fake_device.entry, (None,) * 3, (False, True), steps, warmup=0)
    assert per_mode["noncausal"] == pytest.approx(7e-6)
    assert per_mode["causal"] == pytest.approx(6e-6)
    # Every call of the region ran: `steps` per mode, in mirrored halves.
    assert fake_device.calls.count(False) == steps and fake_device.calls.count(True) == steps
    first = steps // 2
    expected = [False] * first + [True] * first + [True] * (steps - first) + [False] * (steps - first)
    assert fake_device.calls == expected


def test_one_mode_and_warmup(fake_device):
    _, per_mode = bench.time_kernel_batches(fake_device.entry, (None,) * 3, (True,), 5, warmup=3)
    assert per_mode == {"causal": pytest.approx(6e-6)}
    assert len(fake_device.calls) == 8


def test_a_single_step_keeps_its_only_call(fake_device):
    # With one step per mode there is nothing to leave out: the first mode's average then
    # includes the idle start (documented behaviour; the driver runs many steps).
    _, per_mode = bench.time_kernel_batches(fake_device.entry, (None,) * 3, (False, True), 1, warmup=0)
    assert per_mode["causal"] == pytest.approx(26e-6)
    assert per_mode["noncausal"] == pytest.approx(7e-6)


def test_flop_and_byte_counts():
    assert bench.attention_flops(1, 8, 1024, 64, False) == 4 * 8 * 1024**2 * 64
    assert bench.attention_flops(1, 8, 1024, 64, True) == 2 * 8 * 1024**2 * 64
    assert bench.attention_bytes(1, 8, 1024, 64) == 8 * 8 * 1024 * 64


def test_more_than_one_gpu_is_refused():
    result = subprocess.run([sys.executable, str(REPO_ROOT / "bench.py"), "--gpus", "2"],
                            capture_output=True, text=True, cwd=REPO_ROOT, timeout=300)
    assert result.returncode == 2
    assert "one GPU only" in result.stderr
    assert result.stdout == ""


def test_traffic_keys_are_in_the_committed_summary():
    for key in bench.traffic_keys():
        _, status = bench.measured_traffic(key)
        assert status in ("current", "stale"), (key, status)


def _write_counter_csv(path, rows):
    path.parent.mkdir(parents=True, exist_ok=True)
    header = ("Correlation_Id,Dispatch_Id,Kernel_Name,Counter_Name,Counter_Value\n")
    body = "".join(f'{i},{i},"{name}","C",{value}\n' for i, (name, value) in enumerate(rows))
    path.write_text(header + body)


def test_traffic_summary_is_calibrated_and_stamped(tmp_path, monkeypatch):
    # Synthetic rocprofv3 counter CSVs: the copy reads half its bytes in FETCH_SIZE (factor
    # 2) and all of them in WRITE_SIZE; every attention key fetches 1.5x Q+K+V and writes O.
    summary_file = tmp_path / "hbm_traffic.json"
    monkeypatch.setattr(bench, "TRAFFIC_FILE", str(summary_file))
    copy_kib = bench.COPY_CALIBRATION_BYTES / 1024
    _write_counter_csv(tmp_path / "copy_both_FETCH_SIZE" / "run_counter_collection.csv",
                       [(bench.COPY_KERNEL, copy_kib / 2)] * 3)
    _write_counter_csv(tmp_path / "copy_both_WRITE_SIZE" / "run_counter_collection.csv",
                       [(bench.COPY_KERNEL, copy_kib)] * 3)
    expected = {}
    for key in bench.traffic_keys():
        workload, mode = key.split("/")
        b, h, n, _ = bench.WORKLOADS[workload]
        qkv_kib = 6 * b * h * n * 64 / 1024
        kernel = f"_ZN12_GLOBAL__N_1kernel_{mode}"
        # a torch helper kernel in the same run is ignored; the median dispatch is taken
        _write_counter_csv(tmp_path / f"{workload}_{mode}_FETCH_SIZE" / "run_counter_collection.csv",
                           [("torch_fill", 1e9), (kernel, 0.75 * qkv_kib), (kernel, 0.75 * qkv_kib), (kernel, 9e9)])
        _write_counter_csv(tmp_path / f"{workload}_{mode}_WRITE_SIZE" / "run_counter_collection.csv",
                           [(kernel, qkv_kib / 3)] * 2)
        expected[key] = int(round(1024 * (1.5 * qkv_kib + qkv_kib / 3)))
    assert bench.write_traffic_summary(str(tmp_path)) == 0
    for key, hbm in expected.items():
        assert bench.measured_traffic(key) == (hbm, "current")
    # A summary taken on another version of the kernel source is reported as stale.
    monkeypatch.setattr(bench, "kernel_source_digest", lambda: "0" * 64)
    for key in expected:
        assert bench.measured_traffic(key) == (None, "stale")
    assert bench.roofline(1e12, 1.0, bench.traffic_keys()[0])["traffic"] is None
