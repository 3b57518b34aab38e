"""The C ABI from a plain C program (tests/c_abi/caller.c, built by gcc against the
HIP runtime's C API with the package build): closed-form outputs for Q = K = 0 in
both modes, argument rejection, the empty problem and fa2_forward_plan."""

from __future__ import annotations

import subprocess
from pathlib import Path

import pytest

pytestmark = pytest.mark.gpu

CALLER = Path(__file__).resolve().parent / "c_abi" / "caller"


def test_plain_c_caller():
    assert CALLER.exists(), f"{CALLER} is not built (run flash_attention_2_lab_amd/_build.py)"
    proc = subprocess.run([str(CALLER)], capture_output=True, text=True, timeout=120)
    assert proc.returncode == 0, proc.stdout + proc.stderr
    assert proc.stdout.strip().splitlines()[-1] == "ok", proc.stdout
