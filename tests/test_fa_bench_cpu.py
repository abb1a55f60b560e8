"""The torch-free bench binary and its profile tooling, without a GPU: the binary is built and
parses its command line like the reference's fa_bench (ref:bench/bench_main.cu:106-166), its CSV
header is the reference's frozen schema (ref:CONTRACT.md:25-27), and the profile summariser turns
rocprofv3 CSVs into the numbers it claims."""

from __future__ import annotations

import csv
import re
import subprocess
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
BENCH_DIR = ROOT / "fused-attention-cuda_amd" / "bench"
BIN = BENCH_DIR / "fa_bench"
# The frozen schema, verbatim from ref:CONTRACT.md:26.
SCHEMA = ("commit,gpu,driver,nvcc,torch,ncu,clock_mhz,impl,stage,dtype,B,H,N,D,causal,ms_median,"
          "ms_p10,ms_p90,tflops,gbps,notes")


def require_bin():
    if not BIN.exists():
        pytest.fail(f"{BIN} is not built (python fused-attention-cuda_amd/build.py)")


def test_help_exits_zero_and_prints_usage():
    require_bin()
    r = subprocess.run([str(BIN), "--help"], capture_output=True, text=True, timeout=60)
    assert r.returncode == 0
    assert "--stage N" in r.stdout and "--cfg" in r.stdout and "--list" in r.stdout


@pytest.mark.parametrize("args", [["--bogus"], ["--stage"], ["--iters", "0"], ["--causal", "x"]])
def test_bad_arguments_exit_with_usage_code(args):
    require_bin()
    r = subprocess.run([str(BIN), *args], capture_output=True, text=True, timeout=60)
    assert r.returncode == 2, r.stderr
    assert "fa_bench --stage N" in r.stderr


def test_csv_header_is_the_frozen_schema():
    src = (BENCH_DIR / "fa_bench.hip").read_text()
    m = re.search(r'kCsvHeader =\s*((?:"[^"]*"\s*)+);', src)
    assert m, "kCsvHeader not found"
    header = "".join(re.findall(r'"([^"]*)"', m.group(1)))
    assert header == SCHEMA


def test_prof_summary_on_synthetic_rocprof_output(tmp_path):
    """Known inputs: a 20 us C64 kernel is 17179869184 / 20000 ns = 859.0 TFLOP/s; the MFMA-busy
    share is busy / (GRBM_GUI_ACTIVE / 8 x 1024 SIMDs)."""
    name = "_ZN2fa3m1611fa_s5_tunedIDF16_Li64ELi4ELi2ELi64EEEvNS_5KArgsE"
    (tmp_path / "trace").mkdir()
    with open(tmp_path / "trace" / "trace_kernel_stats.csv", "w", newline="") as f:
        w = csv.writer(f)
        w.writerow(["Name", "Calls", "TotalDurationNs", "AverageNs", "Percentage", "MinNs",
                    "MaxNs", "StdDev"])
        w.writerow([name, 10, 200000, 20000, 99.0, 19000, 21000, 1.0])
        w.writerow(["some_fill_kernel", 10, 1000, 100, 1.0, 90, 110, 1.0])

    def counters(sub, values):
        (tmp_path / sub).mkdir()
        with open(tmp_path / sub / f"{sub}_counter_collection.csv", "w", newline="") as f:
            w = csv.writer(f)
            w.writerow(["Kernel_Name", "Counter_Name", "Counter_Value"])
            for k, v in values:
                w.writerow([name, k, v])
                w.writerow(["some_fill_kernel", k, 1e9])

    counters("fetch", [("FETCH_SIZE", 8000), ("FETCH_SIZE", 8400)])
    counters("write", [("WRITE_SIZE", 4096)])
    counters("sq", [("SQ_VALU_MFMA_BUSY_CYCLES", 1024 * 1000.0), ("GRBM_GUI_ACTIVE", 8 * 4000.0)])
    counters("lds", [("SQ_LDS_BANK_CONFLICT", 30.0), ("SQ_LDS_IDX_ACTIVE", 120.0)])
    r = subprocess.run([sys.executable, str(BENCH_DIR / "prof_summary.py"), str(tmp_path),
                        "--stage", "5", "--cfg", "C64", "--dtype", "fp16"],
                       capture_output=True, text=True, timeout=60, check=True)
    out = r.stdout
    assert "| 20000 | 859.0 |" in out
    assert "some_fill_kernel" not in out
    assert "| FETCH_SIZE (KiB per dispatch, raw counter) | 8200 |" in out
    assert "| WRITE_SIZE (KiB per dispatch, raw counter) | 4096 |" in out
    assert "| MFMA busy share (derived) | 25.0 % |" in out
    assert "| LDS bank-conflict share (derived) | 25.0 % |" in out


def test_profile_script_passes_bash_syntax_and_keeps_counter_limits():
    script = BENCH_DIR / "profile.sh"
    subprocess.run(["bash", "-n", str(script)], check=True, timeout=60)
    text = script.read_text()
    for line in re.findall(r"^pass \w+ --pmc (.*(?:\\\n.*)*)", text, flags=re.M):
        counters = line.replace("\\\n", " ").split()
        assert sum(c.startswith("SQ_") for c in counters) <= 8
        tcc = sum(c in ("FETCH_SIZE", "WRITE_SIZE") for c in counters)
        assert tcc <= 1, "FETCH_SIZE and WRITE_SIZE each need a pass of their own"
    assert "--sys-trace" not in text and "--runtime-trace" not in text
