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


@pytest.mark.parametrize("args", [["--bogus"], ["--stage"], ["--iters", "0"], ["--causal", "x"],
                                  ["--flush", "2"]])
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


KERNEL = "_ZN2fa3m1611fa_s5_tunedIDF16_Li64ELi4ELi2ELi64EEEvNS_5KArgsE"
TRACE_COLS = ["Kind", "Kernel_Name", "Start_Timestamp", "End_Timestamp", "LDS_Block_Size",
              "Scratch_Size", "VGPR_Count", "Accum_VGPR_Count", "SGPR_Count", "Workgroup_Size_X",
              "Workgroup_Size_Y", "Workgroup_Size_Z", "Grid_Size_X", "Grid_Size_Y", "Grid_Size_Z"]


def synthetic_capture(root: Path, durations_ns, meta: dict, counters: dict) -> Path:
    """A profile.sh output folder: kernel trace rows of the C64 default tile (grid 131072
    threads in 512-thread workgroups, 104 VGPRs, 64 KiB LDS) with the given durations, a fill
    kernel that must be ignored, and counter passes."""
    root.mkdir(parents=True)
    (root / "meta.txt").write_text("".join(f"{k}={v}\n" for k, v in meta.items()))
    (root / "trace").mkdir()
    with open(root / "trace" / "trace_kernel_trace.csv", "w", newline="") as f:
        w = csv.writer(f)
        w.writerow(TRACE_COLS)
        t = 1_000_000
        for d in durations_ns:
            w.writerow(["KERNEL_DISPATCH", "fill_uniform", t, t + 500, 0, 0, 8, 0, 16, 256, 1, 1,
                        4096, 1, 1])
            t += 1000
            w.writerow(["KERNEL_DISPATCH", KERNEL, t, t + d, 65536, 0, 104, 0, 112, 512, 1, 1,
                        131072, 1, 1])
            t += d + 1000
    for sub, values in counters.items():
        (root / sub).mkdir()
        with open(root / sub / f"{sub}_counter_collection.csv", "w", newline="") as f:
            w = csv.writer(f)
            w.writerow(["Kernel_Name", "Counter_Name", "Counter_Value"])
            for k, v in values:
                w.writerow([KERNEL, k, v])
                w.writerow(["fill_uniform", k, 1e9])
    return root


def table(out: str) -> dict:
    rows = {}
    for line in out.splitlines():
        cells = [c.strip() for c in line.strip().strip("|").split("|")]
        if line.startswith("| ") and len(cells) >= 3:
            rows[cells[0]] = cells[1:-1]
    return rows


def test_prof_summary_derives_its_quantities_from_known_inputs(tmp_path):
    """Known answers: a 20 us C64 forward is 17179869184 FLOP / 20000 ns = 859.0 TFLOP/s, 34.4 %
    of 2.5 PFLOP/s; 2048 waves; the counters below give 256 MFMA and 2000 VALU per wave (7.81 per
    MFMA), 25.0 % co-issue, 2.00 resident waves per busy SIMD, 25.0 % / 30.0 % of the
    wave-cycles waiting on a dependency / for issue, 25.0 % LDS bank conflicts, and
    (8200 x 2 + 4096) KiB = 20987904 B of HBM traffic, 1.241 x the 16908288 algorithmic bytes.
    Only the last `last` dispatches count toward the duration."""
    cap = synthetic_capture(
        tmp_path / "cap", [10000, 10000, 20000, 20000],
        {"stage": 5, "cfg": "C64", "dtype": "fp16", "causal": 0, "workload": "", "forced": "",
         "last": 2},
        {"fetch": [("FETCH_SIZE", 8000), ("FETCH_SIZE", 8400)],
         "write": [("WRITE_SIZE", 4096)],
         "sq": [("SQ_INSTS_MFMA", 2048 * 256.0), ("SQ_INSTS_VALU", 2048 * 2000.0),
                ("SQ_VALU_MFMA_BUSY_CYCLES", 1000.0), ("SQ_VALU_MFMA_COEXEC_CYCLES", 250.0),
                ("SQ_WAVES", 2048.0)],
         "stall": [("SQ_WAVE_CYCLES", 400.0), ("SQ_BUSY_CU_CYCLES", 200.0),
                   ("SQ_WAIT_ANY", 100.0), ("SQ_WAIT_INST_ANY", 120.0)],
         "lds": [("SQ_LDS_BANK_CONFLICT", 30.0), ("SQ_LDS_IDX_ACTIVE", 120.0)]})
    r = subprocess.run([sys.executable, str(BENCH_DIR / "prof_summary.py"), str(cap)],
                       capture_output=True, text=True, timeout=60, check=True)
    t = table(r.stdout)
    assert "fill_uniform" not in r.stdout
    assert t["kernel"] == ["stage 5, D 64, BR 128 x BC 128 (4 row groups x 2 key splits of 64)"]
    assert t["kernel mean duration"][0].startswith("20.00 us over 2 dispatches")
    assert t["achieved"][0].startswith("859.0 TFLOP/s = 34.4 %")
    assert t["grid"][0].startswith("256 workgroups x 8 waves")
    # 104 VGPRs as rocprofv3 reports them are 208 allocated: two waves per SIMD.
    assert t["registers / LDS"][0].startswith("208 VGPR")
    assert t["occupancy allowed"][0] == "2 waves/SIMD (VGPR 2, LDS 4, grid 2)"
    assert t["MFMA / VALU per wave"][0] == "256 / 2000 (7.81 VALU per MFMA)"
    assert t["VALU co-issued with MFMA"][0].startswith("25.0 %")
    assert t["resident waves per busy SIMD"][0] == "2.00"
    assert t["wave-cycles waiting on a dependency"][0] == "25.0 %"
    assert t["wave-cycles waiting for issue"][0] == "30.0 %"
    assert t["LDS bank conflicts"][0].startswith("25.0 %")
    assert t["HBM / algorithmic bytes"][0].startswith("1.241 (20.99 / 16.91 MB)")
    assert "profile.sh 5 C64 fp16" in r.stdout


def test_prof_summary_compares_captures_side_by_side(tmp_path):
    meta = {"stage": 5, "cfg": "C64", "dtype": "fp16", "causal": 0, "workload": "", "last": 0}
    a = synthetic_capture(tmp_path / "a", [20000] * 3, {**meta, "forced": ""}, {})
    b = synthetic_capture(tmp_path / "b", [25000] * 3, {**meta, "forced": "FA_FORCE_BC=64 "}, {})
    r = subprocess.run([sys.executable, str(BENCH_DIR / "prof_summary.py"), "--compare",
                        f"chosen={a}", f"with S=1={b}"],
                       capture_output=True, text=True, timeout=60, check=True)
    t = table(r.stdout)
    assert t["kernel mean duration"][:2] == ["20.00 us over 3 dispatches",
                                             "25.00 us over 3 dispatches"]
    assert t["forced"][:2] == ["", "FA_FORCE_BC=64"]
    assert "chosen 1.000, with S=1 1.250" in r.stdout
    assert f"FA_FORCE_BC=64 bash fused-attention-cuda_amd/bench/profile.sh 5 C64 fp16 {b}" in r.stdout


def test_profile_script_passes_bash_syntax_and_keeps_counter_limits():
    script = BENCH_DIR / "profile.sh"
    subprocess.run(["bash", "-n", str(script)], check=True, timeout=60)
    text = script.read_text()
    passes = re.findall(r"^pass \w+ \w+ --pmc (.*(?:\\\n.*)*)", text, flags=re.M)
    assert len(passes) == 5
    for line in passes:
        counters = line.replace("\\\n", " ").split()
        assert sum(c.startswith("SQ_") for c in counters) <= 8
        assert sum(c.startswith("GRBM_") for c in counters) <= 2
        tcc = sum(c in ("FETCH_SIZE", "WRITE_SIZE") for c in counters)
        assert tcc <= 1, "FETCH_SIZE and WRITE_SIZE each need a pass of their own"
    assert "--sys-trace" not in text and "--runtime-trace" not in text
    # rocprofv3 is a Python script: the interpreter runs it directly, with no launcher between
    # the profiler and the program it profiles.
    assert 'python3 "$ROCPROFV3"' in text and "/usr/bin/env" not in text.split("\n", 1)[1]
