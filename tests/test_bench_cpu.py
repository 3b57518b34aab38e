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
        assert bench.measured_traffic(key) is not None, key
