#!/usr/bin/env python3
"""Summarise the rocprofv3 CSVs that profile.sh wrote into one markdown report.

For the attention kernels of the run (names starting ``fa_s``): average duration and achieved
TFLOP/s from the kernel trace, HBM KiB per dispatch from FETCH_SIZE / WRITE_SIZE, and the SQ and
LDS counters per dispatch, with the derived MFMA-busy share (SQ_VALU_MFMA_BUSY_CYCLES over the
SIMD-cycles of the dispatch: GRBM_GUI_ACTIVE / XCDs x SIMDs) and LDS bank-conflict share.

Usage: prof_summary.py <outdir> --stage 5 --cfg C64 --dtype fp16 [--causal 0]
"""

from __future__ import annotations

import argparse
import csv
import glob
import os
import re
import statistics

SIMDS = 1024  # MI355X: 256 CUs x 4 SIMDs
XCDS = 8      # GRBM_GUI_ACTIVE sums the XCDs' busy clocks


def shape_of(cfg: str) -> tuple[int, int, int, int]:
    if cfg.upper() == "C64":
        return 2, 8, 2048, 64
    if cfg.upper() == "C128":
        return 2, 8, 2048, 128
    m = re.fullmatch(r"B(\d+)_H(\d+)_N(\d+)_D(\d+)", cfg)
    if not m:
        raise SystemExit(f"bad cfg {cfg!r}")
    return tuple(int(x) for x in m.groups())  # type: ignore[return-value]


def kernel_stats(outdir: str) -> list[dict]:
    rows = []
    for f in glob.glob(os.path.join(outdir, "trace", "**", "*kernel_stats.csv"), recursive=True):
        rows += [r for r in csv.DictReader(open(f)) if "fa_s" in r["Name"]]
    return rows


def counters(outdir: str, name: str) -> dict[str, float]:
    vals: dict[str, list[float]] = {}
    for f in glob.glob(os.path.join(outdir, name, "**", "*counter_collection.csv"), recursive=True):
        for r in csv.DictReader(open(f)):
            if "fa_s" in r["Kernel_Name"]:
                vals.setdefault(r["Counter_Name"], []).append(float(r["Counter_Value"]))
    return {k: statistics.mean(v) for k, v in vals.items()}


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("outdir")
    ap.add_argument("--stage", type=int, required=True)
    ap.add_argument("--cfg", required=True)
    ap.add_argument("--dtype", required=True)
    ap.add_argument("--causal", type=int, default=0)
    a = ap.parse_args()
    b, h, n, d = shape_of(a.cfg)
    flops = 4.0 * b * h * n * n * d * (0.5 if a.causal else 1.0)
    print(f"# stage {a.stage}, {a.cfg} (B{b} H{h} N{n} D{d}) {a.dtype}, causal={a.causal}\n")
    cmds = os.path.join(a.outdir, "commands.txt")
    if os.path.exists(cmds):
        print("Commands (each pass its own run, from /tmp):\n")
        for line in open(cmds):
            print("    " + line.rstrip())
        print()
    print("| kernel | calls | average ns | TFLOP/s at the average |")
    print("|---|---|---|---|")
    for r in kernel_stats(a.outdir):
        avg = float(r["AverageNs"])
        print(f"| `{r['Name'][:90]}` | {r['Calls']} | {avg:.0f} | {flops / avg / 1e3:.1f} |")
    print()
    rows = []
    fetch = counters(a.outdir, "fetch").get("FETCH_SIZE")
    write = counters(a.outdir, "write").get("WRITE_SIZE")
    if fetch is not None:
        rows.append(("FETCH_SIZE (KiB per dispatch, raw counter)", f"{fetch:.0f}"))
    if write is not None:
        rows.append(("WRITE_SIZE (KiB per dispatch, raw counter)", f"{write:.0f}"))
    sq = counters(a.outdir, "sq")
    lds = counters(a.outdir, "lds")
    for k, v in sorted({**sq, **lds}.items()):
        rows.append((k, f"{v:.6g}"))
    if "SQ_VALU_MFMA_BUSY_CYCLES" in sq and "GRBM_GUI_ACTIVE" in sq:
        simd_cycles = sq["GRBM_GUI_ACTIVE"] / XCDS * SIMDS
        rows.append(("MFMA busy share (derived)", f"{100 * sq['SQ_VALU_MFMA_BUSY_CYCLES'] / simd_cycles:.1f} %"))
    if "SQ_LDS_BANK_CONFLICT" in lds and lds.get("SQ_LDS_IDX_ACTIVE"):
        rows.append(("LDS bank-conflict share (derived)",
                     f"{100 * lds['SQ_LDS_BANK_CONFLICT'] / lds['SQ_LDS_IDX_ACTIVE']:.1f} %"))
    if rows:
        print("| counter (mean per dispatch) | value |")
        print("|---|---|")
        for k, v in rows:
            print(f"| {k} | {v} |")
    return 0


if __name__ == "__main__":
    raise SystemExit(main())
