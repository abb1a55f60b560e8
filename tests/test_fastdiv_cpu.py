"""The kernels' grid decode divides by launch constants with a host-precomputed multiply-shift
(``fa::FastDiv`` in csrc/fa_internal.h). This builds a small checker against the real header with
the host compiler and runs it: every divisor 1..20000 with edge and random numerators below 2^31,
and a few large divisors, against plain integer division."""

from __future__ import annotations

import shutil
import subprocess
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]


def test_fastdiv_matches_integer_division(tmp_path):
    cxx = shutil.which("g++")
    if cxx is None or not Path("/opt/rocm/include/hip/hip_runtime_api.h").exists():
        pytest.skip("needs g++ and the ROCm headers")
    exe = tmp_path / "fastdiv_check"
    subprocess.run([cxx, "-O2", "-std=c++17", "-D__HIP_PLATFORM_AMD__", "-I/opt/rocm/include",
                    f"-I{ROOT / 'include'}", f"-I{ROOT / 'fused-attention-cuda_amd' / 'csrc'}",
                    str(ROOT / "tests" / "fastdiv_check.cpp"), "-o", str(exe)], check=True)
    res = subprocess.run([str(exe)], capture_output=True, text=True, timeout=120)
    assert res.returncode == 0, res.stdout + res.stderr
    assert "all exact" in res.stdout
