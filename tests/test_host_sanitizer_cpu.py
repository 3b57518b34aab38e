"""The C ABI's host-side paths under AddressSanitizer and UndefinedBehaviorSanitizer.

`tests/c_abi/host_checks.c` calls every entry point only with arguments it rejects (or
with an empty problem), plus `fa2_status_string` and `fa2_forward_plan`, so nothing is
launched and no GPU is needed. The library is rebuilt here from `fa2_forward.hip` and
`fa2_aux.hip` with the sanitizers on their host code only (`-Xarch_host`), and the
checker is built by clang so that both use clang's sanitizer runtime. Any sanitizer
report aborts the run (`-fno-sanitize-recover=all`).
"""

from __future__ import annotations

import shutil
import subprocess
from pathlib import Path

import pytest

REPO_ROOT = Path(__file__).resolve().parents[1]
ROCM = Path("/opt/rocm")
HIPCC = ROCM / "bin" / "hipcc"
CLANG = ROCM / "llvm" / "bin" / "clang"
CSRC = REPO_ROOT / "flash_attention_2_lab_amd" / "csrc"
SOURCES = [CSRC / "fa2_forward.hip", CSRC / "fa2_aux.hip"]
CHECKS = REPO_ROOT / "tests" / "c_abi" / "host_checks.c"
INCLUDE = REPO_ROOT / "include"
SANITIZE = ["-fsanitize=address", "-fsanitize=undefined", "-fno-sanitize-recover=all",
            "-fno-omit-frame-pointer"]


def _run(cmd: list[str], **kwargs) -> subprocess.CompletedProcess:
    return subprocess.run(cmd, capture_output=True, text=True, timeout=300, **kwargs)


@pytest.mark.skipif(not (HIPCC.exists() and CLANG.exists()), reason="needs ROCm hipcc and clang")
def test_host_paths_are_clean_under_sanitizers(tmp_path: Path) -> None:
    library = tmp_path / "libfa2_host_sanitized.so"
    host_flags = [flag for option in SANITIZE for flag in ("-Xarch_host", option)]
    build = _run([str(HIPCC), "--offload-arch=gfx950", "-O1", "-g", "-std=c++17", "-fPIC", "-shared",
                  "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops", *host_flags,
                  f"-I{INCLUDE}", *(str(p) for p in SOURCES), "-o", str(library)])
    assert build.returncode == 0, build.stdout + build.stderr

    checker = tmp_path / "host_checks"
    link = _run([str(CLANG), "-std=c11", "-O1", "-g", "-Wall", "-Wextra", "-Werror", *SANITIZE,
                 "-D__HIP_PLATFORM_AMD__", f"-I{INCLUDE}", str(CHECKS), "-o", str(checker),
                 f"-L{tmp_path}", "-lfa2_host_sanitized", f"-L{ROCM / 'lib'}", "-lamdhip64",
                 f"-Wl,-rpath,{tmp_path}", f"-Wl,-rpath,{ROCM / 'lib'}"])
    assert link.returncode == 0, link.stdout + link.stderr

    # The sanitized library must really carry the instrumentation.
    nm = shutil.which("nm")
    if nm:
        symbols = _run([nm, "-D", str(library)]).stdout
        assert "__asan_" in symbols and "__ubsan_" in symbols

    proc = _run([str(checker)])
    assert proc.returncode == 0, proc.stdout + proc.stderr
    assert "Sanitizer" not in proc.stderr, proc.stderr
    assert proc.stdout.strip().splitlines()[-1] == "ok", proc.stdout
