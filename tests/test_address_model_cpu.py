"""Memory safety of the kernels' address arithmetic, on the CPU.

tests/address_model.cpp replays, from the kernels' own layout functions (csrc/tile_layout.h),
every LDS-DMA load and MFMA operand read of every workgroup of the stage-4/5 kernels -- for each
tile variant in the kernel tables of csrc/attn_mfma16.h, over a sweep of sequence lengths (full
and partial tiles, including N = 288 where the reference ran compute-sanitizer,
ref:scripts/gpu_run.sh:157-181), causal and not, split walks of 1-16 parts, dense and strided rows
-- plus decode's split kernel, and checks that every read lies inside its tensor and every LDS
access inside its buffer. The variants are read from the table source, so a tile added there is
covered without touching this test.
"""

from __future__ import annotations

import re
import shutil
import subprocess
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
CSRC = ROOT / "fused-attention-cuda_amd" / "csrc"


def table_variants() -> list[tuple[int, int, int, int]]:
    """(D, RG, KS, BCW) of every stage-5 and stage-4 variant instantiated in attn_mfma16.h."""
    src = (CSRC / "attn_mfma16.h").read_text()
    rows = src[src.index("struct S5Rows"):src.index("};", src.index("struct S5Rows"))]
    generic = re.findall(r"variant<STAGE, T, D, (\d+), (\d+), (\d+)>", rows)
    found = {(d, *map(int, g)) for d in (64, 128) for g in generic}
    for m in re.finditer(r"variant<(?:[45]|STAGE), T, (\d+), (\d+), (\d+), (\d+)>", src):
        found.add(tuple(map(int, m.groups())))
    return sorted(found)


def test_the_table_parse_sees_the_default_tiles():
    v = table_variants()
    assert (64, 4, 2, 64) in v and (128, 4, 2, 32) in v and (128, 4, 1, 32) in v
    assert (64, 2, 2, 32) in v and (64, 8, 1, 64) in v
    assert (128, 8, 1, 64) not in v  # the spilling D = 128 BR 256 tile is not built
    assert len(v) >= 17


def test_every_kernel_read_stays_in_bounds(tmp_path):
    cxx = shutil.which("g++")
    if cxx is None:
        pytest.skip("needs g++")
    exe = tmp_path / "address_model"
    subprocess.run([cxx, "-O2", "-std=c++17", f"-I{CSRC}", str(ROOT / "tests" / "address_model.cpp"),
                    "-o", str(exe)], check=True)
    args = [",".join(map(str, v)) for v in table_variants()]
    res = subprocess.run([str(exe), *args], capture_output=True, text=True, timeout=600)
    assert res.returncode == 0, res.stdout[-3000:] + res.stderr[-2000:]
    assert "all in bounds" in res.stdout, res.stdout


def test_the_model_catches_a_missing_clamp(tmp_path):
    """Planted mistake, on the CPU: with the row clamp of partial tiles removed (the bug the clamp
    exists to prevent) the model must report a read past the end of a head."""
    cxx = shutil.which("g++")
    if cxx is None:
        pytest.skip("needs g++")
    exe = tmp_path / "address_model"
    subprocess.run([cxx, "-O2", "-std=c++17", f"-I{CSRC}", str(ROOT / "tests" / "address_model.cpp"),
                    "-o", str(exe)], check=True)
    res = subprocess.run([str(exe), "--plant-no-clamp", "64,4,2,64"], capture_output=True,
                         text=True, timeout=600)
    assert res.returncode != 0 and "VIOLATION" in res.stdout, res.stdout[-2000:]
