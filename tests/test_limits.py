"""The host-side predicates behind the entry points' argument checks and the
GEMM kernel routing (csrc/limits.hpp), compiled with the host compiler and
checked at their boundaries (no GPU, no HIP)."""

import shutil
import subprocess
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent


@pytest.mark.skipif(shutil.which("g++") is None, reason="needs the host C++ compiler")
def test_limits_predicates(tmp_path):
    exe = tmp_path / "limits_check"
    subprocess.run(["g++", "-std=c++17", "-O1", "-Wall", "-Werror",
                    "-I", str(ROOT / "transformer_optimization_amd" / "csrc"),
                    str(ROOT / "tests" / "cpp" / "limits_check.cpp"), "-o", str(exe)],
                   check=True, capture_output=True, text=True)
    out = subprocess.run([str(exe)], capture_output=True, text=True)
    assert out.returncode == 0 and out.stdout.strip() == "ok", out.stdout + out.stderr
