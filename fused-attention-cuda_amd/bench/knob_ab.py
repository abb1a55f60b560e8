"""A/B timing of the library's per-call environment knobs (FA_FORCE_ROTATE, FA_FORCE_BC, ...)
over bench.py's workloads or ad-hoc shapes, in one process: the library reads these knobs on
every call.

For every workload and each knob setting, twice in alternation: bench.py's gate and 50 launches
over 4 cache-resident sets (warm), then 100 host-issued launches over cache-cold sets, the median
of three loops (cold, the protocol of bench.py's ``value``). Prints one line per measurement and a
summary of the minimum over the two repetitions.

KNOB names one knob or several joined by '+'; each setting gives one value per knob, joined the
same way ("64+64" for FA_FORCE_BR+FA_FORCE_BC), or "rule", which unsets them all so that the
library's own rules decide. A workload is a bench.py workload name or a shape written
B<b>H<h>N<n>D<d>, then "c" for causal and "bf" for bf16 (fp16 otherwise), e.g. B8H12N1024D64c;
ad-hoc shapes take unit-variance inputs.

usage (from the repository root):
  python fused-attention-cuda_amd/bench/knob_ab.py KNOB setting0 setting1 [workload ...]
"""
import os
import re
import sys
from pathlib import Path

ROOT = Path(__file__).resolve().parents[2]
sys.path.insert(0, str(ROOT))
import bench  # noqa: E402
import torch  # noqa: E402
from fused_attn import capi  # noqa: E402

SHAPE = re.compile(r"B(\d+)H(\d+)N(\d+)D(\d+)(c?)(bf)?$")


def workload(name):
    """Registers an ad-hoc shape in bench.WORKLOADS under its own name."""
    if name not in bench.WORKLOADS:
        m = SHAPE.match(name)
        if m is None:
            sys.exit(f"unknown workload {name!r}: a bench.py workload or B<b>H<h>N<n>D<d>[c][bf]")
        b, h, n, d = (int(x) for x in m.group(1, 2, 3, 4))
        bench.WORKLOADS[name] = (b, h, n, d, "bf16" if m.group(6) else "fp16", m.group(5) == "c",
                                 1.0)
    return name


knobs = sys.argv[1].split("+")
vals = sys.argv[2:4]
names = [workload(n) for n in sys.argv[4:]] or [
    "C64", "C128", "C64_causal", "C128_causal", "GPT_attn", "LONG_N1024", "LONG"]
for val in vals:
    if val != "rule" and len(val.split("+")) != len(knobs):
        sys.exit(f"setting {val!r} does not give one value per knob of {sys.argv[1]!r}")
capi.load()
res = {}
for rep in range(2):
    for val in vals:
        for knob, v in zip(knobs, val.split("+") if val != "rule" else [None] * len(knobs)):
            if v is None:
                os.environ.pop(knob, None)
            else:
                os.environ[knob] = v
        for name in names:
            stage = bench.stage_of(name)
            r, s2, st, c, sc = bench.bench_workload(torch, capi, name, stage, 50, 50, replay=False)
            del s2
            torch.cuda.empty_cache()
            cold, _, nsets = bench.cold_timing(torch, capi, name, stage, 100, 50, graph=False)
            res.setdefault((name, val), []).append((cold * 1e3, r["eager_ms"] * 1e3, r["gate_max_err_o"]))
            print(f"rep{rep} {sys.argv[1]}={val} {name}: cold {cold*1e3:.2f} us warm {r['eager_ms']*1e3:.2f} us err {r['gate_max_err_o']:.2e}", flush=True)
print(f"summary (min of reps): name | " + " | ".join(f"{sys.argv[1]}={v} cold/warm" for v in vals))
for name in names:
    cells = []
    for v in vals:
        xs = res[(name, v)]
        cells.append(f"{min(x[0] for x in xs):.2f} / {min(x[1] for x in xs):.2f}")
    print(name, "|", " | ".join(cells))
