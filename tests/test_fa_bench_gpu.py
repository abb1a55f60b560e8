"""fa_bench on the GPU (marker ``gpu``): it checks its own output against fp64 rows before it
writes a row, writes rows of the frozen schema, and reports unsupported stages with exit code 3
(ref:bench/bench_main.cu:25-26). One process per case; each is a short run (--iters small)."""

from __future__ import annotations

import csv
import subprocess
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
BIN = ROOT / "fused-attention-cuda_amd" / "bench" / "fa_bench"
pytestmark = pytest.mark.gpu


def run(*args, timeout=120):
    if not BIN.exists():
        pytest.fail(f"{BIN} is not built")
    print("fa_bench", *args, flush=True)
    return subprocess.run([str(BIN), *args], capture_output=True, text=True, timeout=timeout)


@pytest.mark.parametrize("dtype,causal,extra", [("fp16", 0, []), ("bf16", 1, ["--hkv", "2"]),
                                                ("fp16", 1, [])],
                         ids=["fp16-full", "bf16-causal-gqa", "fp16-causal"])
def test_row_after_passing_check(tmp_path, dtype, causal, extra):
    out = tmp_path / "rows.csv"
    r = run("--stage", "5", "--cfg", "B2_H4_N512_D64", "--dtype", dtype, "--causal", str(causal),
            "--iters", "10", "--warmup", "2", "--out", str(out), "--commit", "test", *extra)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "CHECK_OK" in r.stdout
    rows = list(csv.DictReader(open(out)))
    assert len(rows) == 1
    row = rows[0]
    assert row["commit"] == "test" and row["impl"] == "tuned" and row["stage"] == "5"
    assert row["dtype"] == dtype and row["causal"] == str(causal)
    assert (row["B"], row["H"], row["N"], row["D"]) == ("2", "4", "512", "64")
    assert float(row["ms_median"]) > 0 and float(row["tflops"]) > 0 and float(row["gbps"]) > 0
    assert float(row["ms_p10"]) <= float(row["ms_median"]) <= float(row["ms_p90"])
    assert int(row["clock_mhz"]) > 500
    notes = row["notes"].split(";")
    assert "iters=10" in notes and "check=rows128" in notes
    assert ("flops=causal_half" in notes) == bool(causal)


def test_second_run_appends_without_a_second_header(tmp_path):
    out = tmp_path / "rows.csv"
    for _ in range(2):
        r = run("--stage", "3", "--cfg", "B1_H2_N128_D64", "--dtype", "fp32", "--iters", "5",
                "--warmup", "1", "--out", str(out))
        assert r.returncode == 0, r.stdout + r.stderr
    lines = out.read_text().splitlines()
    assert len(lines) == 3 and lines[0].startswith("commit,gpu,driver")


@pytest.mark.parametrize("stage,dtype", [(1, "fp32"), (2, "fp16"), (5, "fp32")])
def test_unimplemented_stage_exits_3(stage, dtype):
    r = run("--stage", str(stage), "--cfg", "B1_H1_N64_D64", "--dtype", dtype, "--iters", "3")
    assert r.returncode == 3, r.stdout + r.stderr
    assert "not implemented" in r.stdout


def test_list_reports_the_build():
    r = run("--list")
    assert r.returncode == 0
    assert "stage 5 tuned  fp16  D= 64 : yes" in r.stdout
    assert "stage 1 naive  fp32  D= 64 : no" in r.stdout


def test_smoke_mode_checks_and_writes_no_row(tmp_path):
    r = run("--smoke", "--stage", "4")
    assert r.returncode == 0, r.stdout + r.stderr
    assert "CHECK_OK" in r.stdout and "appended" not in r.stdout
