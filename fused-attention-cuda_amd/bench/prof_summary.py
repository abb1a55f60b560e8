#!/usr/bin/env python3
"""Summarise the rocprofv3 CSVs that profile.sh wrote into a markdown report.

One capture:     prof_summary.py <outdir>
Side by side:    prof_summary.py --compare LABEL=<outdir> LABEL=<outdir> ... [--title T]

For the attention kernels of the run (``fa_s*`` and ``fa_decode*``), per capture:

* duration: the mean kernel duration from the kernel trace (the last ``last`` dispatches when
  the program was bench.py's timed launches), TFLOP/s and share of the 2.5 PFLOP/s dense fp16/bf16
  MFMA peak (157.3 TFLOP/s for fp32); split walks add the combine kernel's mean;
* launch: workgroups, waves per workgroup, VGPRs (architectural + accumulation), LDS bytes,
  scratch, and the occupancy they allow (waves per SIMD: 512 VGPRs per lane, 160 KiB of LDS per
  CU, at most one workgroup slot per 256 CUs per grid wave);
* instruction mix per wave (SQ_INSTS_* / waves): MFMA, VALU, transcendental, LDS, SALU;
  co-execution = SQ_VALU_MFMA_COEXEC_CYCLES / SQ_VALU_MFMA_BUSY_CYCLES;
* wave states: mean resident waves per busy SIMD = SQ_WAVE_CYCLES / SQ_BUSY_CU_CYCLES (it reads
  1.94 for a grid of one 8-wave workgroup per CU, 2 waves on each SIMD for the whole launch, and
  1.00 for one 2-wave workgroup per CU, whose two SIMDs hold one wave each), and the
  shares of resident wave-cycles spent waiting on a dependency (SQ_WAIT_ANY: s_waitcnt, barrier)
  and waiting for issue (SQ_WAIT_INST_ANY) -- all three in quad-cycles;
* LDS: bytes read per CU and bank-conflict share;
* HBM: FETCH_SIZE x 2.0 and WRITE_SIZE x 1.0 (the factors a plain 256 MiB copy reads on the same
  counters: FETCH_SIZE counts half the bytes a copy reads), against the algorithmic bytes (Q, K,
  V read once, O written once, fp32 LSE written).
"""

from __future__ import annotations

import argparse
import csv
import glob
import math
import os
import re
import statistics

SIMDS_PER_CU = 4
CUS = 256
VGPRS_PER_LANE = 512      # unified architectural + accumulation file per SIMD lane (wave64)
LDS_PER_CU = 160 * 1024
MAX_WAVES_PER_SIMD = 8
FETCH_SCALE, WRITE_SCALE = 2.0, 1.0
PEAK = {"fp16": 2500.0, "bf16": 2500.0, "fp32": 157.3}  # dense MFMA TFLOP/s

_TILE = re.compile(r"fa_s([45])_\w+?I(DF16_|DF16b)Li(\d+)ELi(\d+)ELi(\d+)ELi(\d+)E")


def shape_of(cfg: str) -> tuple[int, int, int, int]:
    if cfg.upper() == "C64":
        return 2, 8, 2048, 64
    if cfg.upper() == "C128":
        return 2, 8, 2048, 128
    m = re.fullmatch(r"B(\d+)_H(\d+)_N(\d+)_D(\d+)", cfg)
    if not m:
        raise SystemExit(f"bad cfg {cfg!r}")
    return tuple(int(x) for x in m.groups())  # type: ignore[return-value]


def read_meta(outdir: str) -> dict[str, str]:
    meta = {}
    path = os.path.join(outdir, "meta.txt")
    if os.path.exists(path):
        for line in open(path):
            if "=" in line:
                k, v = line.rstrip("\n").split("=", 1)
                meta[k] = v
    return meta


def is_attn(name: str) -> bool:
    return "fa_s" in name or "fa_decode" in name


def trace_rows(outdir: str) -> list[dict]:
    rows = []
    for f in glob.glob(os.path.join(outdir, "trace", "**", "*kernel_trace.csv"), recursive=True):
        rows += [r for r in csv.DictReader(open(f)) if is_attn(r["Kernel_Name"])]
    rows.sort(key=lambda r: int(r["Start_Timestamp"]))
    return rows


def counters(outdir: str, name: str, kernel: str) -> dict[str, float]:
    vals: dict[str, list[float]] = {}
    for f in glob.glob(os.path.join(outdir, name, "**", "*counter_collection.csv"), recursive=True):
        for r in csv.DictReader(open(f)):
            if r["Kernel_Name"] == kernel:
                vals.setdefault(r["Counter_Name"], []).append(float(r["Counter_Value"]))
    return {k: statistics.mean(v) for k, v in vals.items()}


def collect(outdir: str) -> dict:
    """The quantities of one capture, as an ordered list of (quantity, value, source)."""
    meta = read_meta(outdir)
    b, h, n, d = shape_of(meta.get("cfg", "C64"))
    causal = meta.get("causal", "0") == "1"
    dtype = meta.get("dtype", "fp16")
    last = int(meta.get("last", "0") or 0)
    flops = 4.0 * b * h * n * n * d * (0.5 if causal else 1.0)
    es = 4 if dtype == "fp32" else 2
    algo_bytes = 4 * b * h * n * d * es + 4 * b * h * n
    rows = trace_rows(outdir)
    if not rows:
        raise SystemExit(f"{outdir}: no attention kernel in the kernel trace")
    by_name: dict[str, list[dict]] = {}
    for r in rows:
        by_name.setdefault(r["Kernel_Name"], []).append(r)
    dur = {k: [int(r["End_Timestamp"]) - int(r["Start_Timestamp"]) for r in v]
           for k, v in by_name.items()}
    main = max(dur, key=lambda k: sum(dur[k]))
    main_d = dur[main][-last:] if last else dur[main]
    avg_main = statistics.mean(main_d)
    others = {k: statistics.mean(v[-last:] if last else v) for k, v in dur.items() if k != main}
    fwd_ns = avg_main + sum(others.values())
    r0 = by_name[main][0]
    grid_threads = int(r0["Grid_Size_X"]) * int(r0["Grid_Size_Y"]) * int(r0["Grid_Size_Z"])
    wg = int(r0["Workgroup_Size_X"]) * int(r0["Workgroup_Size_Y"]) * int(r0["Workgroup_Size_Z"])
    wgs = grid_threads // wg
    waves = grid_threads // 64
    waves_per_wg = max(1, wg // 64)
    # rocprofv3 reports gfx950's register counts as 4 x ceil(v / 8) for a kernel the compiler
    # gives v VGPRs (its kernel-resource-usage report: 196 -> 100, 238 -> 120, 150 -> 76), while
    # the hardware allocates them in granules of 8: the allocation is twice the reported count.
    vgpr = 2 * (int(r0["VGPR_Count"]) + int(r0["Accum_VGPR_Count"]))
    lds = int(r0["LDS_Block_Size"])
    occ_vgpr = min(MAX_WAVES_PER_SIMD, VGPRS_PER_LANE // max(vgpr, 1))
    wg_lds = LDS_PER_CU // lds if lds else 10**9
    occ_lds = wg_lds * waves_per_wg / SIMDS_PER_CU
    occ_grid = math.ceil(wgs / CUS) * waves_per_wg / SIMDS_PER_CU
    occ = min(occ_vgpr, occ_lds, occ_grid)
    q: list[tuple[str, str, str]] = []
    m = _TILE.search(main)
    if m:
        stage, _, dd, rg, ks, bcw = m.groups()
        tile = (f"stage {stage}, D {dd}, BR {32 * int(rg)} x BC {int(ks) * int(bcw)} "
                f"({rg} row groups x {ks} key splits of {bcw})")
    else:
        tile = re.sub(r"^_ZN\d+\w+?(fa_\w+?)I.*", r"\1", main)
    q.append(("kernel", tile, "kernel name"))
    if meta.get("forced"):
        q.append(("forced", meta["forced"].strip(), "environment"))
    q.append(("kernel mean duration", f"{avg_main / 1e3:.2f} us over {len(main_d)} dispatches",
              "kernel trace" + (f", last {last} dispatches (the last timed loop)" if last else "")))
    for k, v in others.items():
        short = re.sub(r"^_ZN\d+\w+?(fa_\w+?)I.*", r"\1", k)
        q.append((f"+ {short}", f"{v / 1e3:.2f} us", "kernel trace"))
    if others:
        q.append(("forward (all kernels)", f"{fwd_ns / 1e3:.2f} us", "sum of the means"))
    tflops = flops / fwd_ns / 1e3
    q.append(("achieved", f"{tflops:.1f} TFLOP/s = {100 * tflops / PEAK[dtype]:.1f} % of "
              f"{PEAK[dtype]:g}", "4 B H N^2 D FLOP (halved causal) / forward time"))
    q.append(("grid", f"{wgs} workgroups x {waves_per_wg} waves ({wgs / CUS:.2f} per CU)",
              "kernel trace"))
    q.append(("registers / LDS", f"{vgpr} VGPR, {lds} B LDS, {r0['Scratch_Size']} B scratch",
              "kernel trace"))
    q.append(("occupancy allowed", f"{occ:g} waves/SIMD (VGPR {occ_vgpr}, LDS {occ_lds:g}, "
              f"grid {occ_grid:g})", "512 VGPRs, 160 KiB LDS, workgroups / 256 CUs"))
    sq = counters(outdir, "sq", main)
    st = counters(outdir, "stall", main)
    ld = counters(outdir, "lds", main)
    fe = counters(outdir, "fetch", main).get("FETCH_SIZE")
    wr = counters(outdir, "write", main).get("WRITE_SIZE")
    if sq:
        mf = sq.get("SQ_INSTS_MFMA", 0.0)
        va = sq.get("SQ_INSTS_VALU", 0.0)
        per = lambda c: sq.get(c, 0.0) / waves  # noqa: E731
        q.append(("MFMA / VALU per wave", f"{per('SQ_INSTS_MFMA'):.0f} / {per('SQ_INSTS_VALU'):.0f}"
                  f" ({va / mf if mf else 0:.2f} VALU per MFMA)", "SQ_INSTS_MFMA, SQ_INSTS_VALU"))
        q.append(("transcendental / LDS / SALU per wave",
                  f"{per('SQ_INSTS_VALU_TRANS_F32'):.0f} / {per('SQ_INSTS_LDS'):.0f} / "
                  f"{per('SQ_INSTS_SALU'):.0f}",
                  "SQ_INSTS_VALU_TRANS_F32, SQ_INSTS_LDS, SQ_INSTS_SALU"))
        if sq.get("SQ_VALU_MFMA_BUSY_CYCLES"):
            q.append(("VALU co-issued with MFMA",
                      f"{100 * sq.get('SQ_VALU_MFMA_COEXEC_CYCLES', 0) / sq['SQ_VALU_MFMA_BUSY_CYCLES']:.1f}"
                      " % of MFMA-busy cycles",
                      "SQ_VALU_MFMA_COEXEC_CYCLES / SQ_VALU_MFMA_BUSY_CYCLES"))
        if sq.get("SQ_WAVES"):
            q.append(("waves counted", f"{sq['SQ_WAVES']:.0f} (grid: {waves})", "SQ_WAVES"))
    if st.get("SQ_WAVE_CYCLES") and st.get("SQ_BUSY_CU_CYCLES"):
        wc = st["SQ_WAVE_CYCLES"]
        q.append(("resident waves per busy SIMD", f"{wc / st['SQ_BUSY_CU_CYCLES']:.2f}",
                  "SQ_WAVE_CYCLES / SQ_BUSY_CU_CYCLES"))
        q.append(("wave-cycles waiting on a dependency", f"{100 * st.get('SQ_WAIT_ANY', 0) / wc:.1f} %",
                  "SQ_WAIT_ANY / SQ_WAVE_CYCLES"))
        q.append(("wave-cycles waiting for issue", f"{100 * st.get('SQ_WAIT_INST_ANY', 0) / wc:.1f} %",
                  "SQ_WAIT_INST_ANY / SQ_WAVE_CYCLES"))
        q.append(("of which LDS issue", f"{100 * st.get('SQ_WAIT_INST_LDS', 0) / wc:.1f} %",
                  "SQ_WAIT_INST_LDS / SQ_WAVE_CYCLES"))
        for c in ("SQ_ACTIVE_INST_ANY", "SQ_ACTIVE_INST_VALU", "SQ_ACTIVE_INST_LDS"):
            if c in st:
                q.append((c.lower().replace("sq_active_inst_", "active instruction cycles, "),
                          f"{st[c] / waves:.0f} per wave", c + " (raw, per wave)"))
    if ld:
        if "SQ_INSTS_LDS_LOAD_BANDWIDTH" in ld:
            q.append(("LDS read per CU", f"{ld['SQ_INSTS_LDS_LOAD_BANDWIDTH'] * 64 / CUS / 1e6:.2f} MB",
                      "SQ_INSTS_LDS_LOAD_BANDWIDTH x 64 B / 256 CUs"))
        if ld.get("SQ_LDS_IDX_ACTIVE"):
            q.append(("LDS bank conflicts",
                      f"{100 * ld.get('SQ_LDS_BANK_CONFLICT', 0) / ld['SQ_LDS_IDX_ACTIVE']:.1f} % of "
                      "LDS-active cycles", "SQ_LDS_BANK_CONFLICT / SQ_LDS_IDX_ACTIVE"))
    if fe is not None and wr is not None:
        hbm = (fe * FETCH_SCALE + wr * WRITE_SCALE) * 1024
        q.append(("HBM read / written", f"{fe * FETCH_SCALE / 1024:.2f} / {wr * WRITE_SCALE / 1024:.2f}"
                  " MiB per launch", "FETCH_SIZE x 2.0, WRITE_SIZE x 1.0"))
        q.append(("HBM / algorithmic bytes", f"{hbm / algo_bytes:.3f} ({hbm / 1e6:.2f} / "
                  f"{algo_bytes / 1e6:.2f} MB)", "algorithmic: Q, K, V read, O and LSE written"))
    title = (f"B{b} H{h} N{n} D{d} {dtype} {'causal' if causal else 'non-causal'}"
             + (f", bench.py workload {meta['workload']}" if meta.get("workload") else ""))
    cmds = []
    cpath = os.path.join(outdir, "commands.txt")
    if os.path.exists(cpath):
        cmds = [line.rstrip() for line in open(cpath) if line.strip()]
    invocation = (f"{meta.get('forced', '')}bash fused-attention-cuda_amd/bench/profile.sh "
                  f"{meta.get('stage', '5')} {meta.get('cfg', 'C64')} {dtype} {outdir.rstrip('/')} "
                  f"{meta.get('causal', '0')} {meta.get('workload', '')}").rstrip()
    return {"title": title, "q": q, "commands": cmds, "fwd_ns": fwd_ns, "invocation": invocation}


def render(items: list[tuple[str, dict]], title: str, argv: list[str]) -> str:
    out = [f"# {title}", ""]
    out.append("Made on the GPU box from the repository root (one profile.sh run per capture), then "
               "summarised by")
    out += ["", "    python3 fused-attention-cuda_amd/bench/prof_summary.py " + " ".join(argv), ""]
    for label, c in items:
        inv = re.sub(r"/\S*?/repo/", "", c["invocation"])
        out.append(f"- {label + ': ' if label else ''}{c['title']}: `{inv}`")
    out.append("")
    out.append("The rocprofv3 passes of " + (items[0][0] if items[0][0] else "the capture") +
               " (each its own run; the other captures differ only in their program arguments, "
               "output folder and FA_FORCE_* settings; `$REPO` is the repository root):")
    out.append("")
    for line in items[0][1]["commands"]:
        out.append("    " + re.sub(r"/\S*?/repo/", "$REPO/", line))
    out.append("")
    if len(items) == 1:
        out += ["| Quantity | Value | From |", "|---|---|---|"]
        out += [f"| {k} | {v} | {s} |" for k, v, s in items[0][1]["q"]]
    else:
        keys: list[str] = []
        src: dict[str, str] = {}
        for _, c in items:
            for k, _, s in c["q"]:
                if k not in keys:
                    keys.append(k)
                    src[k] = s
        out.append("| Quantity | " + " | ".join(label for label, _ in items) + " | From |")
        out.append("|---|" + "---|" * len(items) + "---|")
        for k in keys:
            vals = [dict((kk, vv) for kk, vv, _ in c["q"]).get(k, "") for _, c in items]
            out.append(f"| {k} | " + " | ".join(vals) + f" | {src[k]} |")
        base = items[0][1]["fwd_ns"]
        out.append("")
        out.append("Forward time relative to " + items[0][0] + ": " + ", ".join(
            f"{label} {c['fwd_ns'] / base:.3f}" for label, c in items) + ".")
    out.append("")
    return "\n".join(out)


def main() -> int:
    import shlex
    import sys

    argv = [shlex.quote(x) for x in sys.argv[1:]]
    ap = argparse.ArgumentParser()
    ap.add_argument("outdir", nargs="?")
    ap.add_argument("--compare", nargs="+", metavar="LABEL=DIR")
    ap.add_argument("--title")
    a = ap.parse_args()
    if a.compare:
        items = []
        for spec in a.compare:
            label, _, path = spec.rpartition("=")
            items.append((label, collect(path)))
        print(render(items, a.title or items[0][1]["title"], argv))
    elif a.outdir:
        c = collect(a.outdir)
        print(render([("", c)], a.title or c["title"], argv))
    else:
        ap.error("give an outdir or --compare")
    return 0


if __name__ == "__main__":
    raise SystemExit(main())
