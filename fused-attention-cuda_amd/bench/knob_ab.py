"""A/B timing of one of the library's per-call environment knobs (FA_FORCE_ROTATE, FA_FORCE_BC,
...) over bench.py's workloads, in one process: the library reads these knobs on every call.

For every workload and each knob value (a value of "rule" unsets the knob, so the library's own
rule decides), twice in alternation: bench.py's gate and 50 launches over 4 cache-resident sets
(warm), then 100 host-issued launches over cache-cold sets, the median of three loops (cold, the
protocol of bench.py's ``value``). Prints one line per measurement and a summary of the minimum
over the two repetitions.

usage (from the repository root): python fused-attention-cuda_amd/bench/knob_ab.py KNOB v0 v1 [workload ...]
"""
import os
import sys
from pathlib import Path

ROOT = Path(__file__).resolve().parents[2]
sys.path.insert(0, str(ROOT))
import bench  # noqa: E402
import torch  # noqa: E402
from fused_attn import capi  # noqa: E402

knob, vals = sys.argv[1], sys.argv[2:4]
names = sys.argv[4:] or ["C64", "C128", "C64_causal", "C128_causal", "GPT_attn", "LONG_N1024", "LONG"]
capi.load()
res = {}
for rep in range(2):
    for val in vals:
        if val == "rule":
            os.environ.pop(knob, None)
        else:
            os.environ[knob] = val
        for name in names:
            stage = bench.stage_of(name)
            r, s2, st, c, sc = bench.bench_workload(torch, capi, name, stage, 50, 50, replay=False)
            del s2
            torch.cuda.empty_cache()
            cold, _, nsets = bench.cold_timing(torch, capi, name, stage, 100, 50, graph=False)
            res.setdefault((name, val), []).append((cold * 1e3, r["eager_ms"] * 1e3, r["gate_max_err_o"]))
            print(f"rep{rep} {knob}={val} {name}: cold {cold*1e3:.2f} us warm {r['eager_ms']*1e3:.2f} us err {r['gate_max_err_o']:.2e}", flush=True)
print("summary (min of reps): name | " + " | ".join(f"{knob}={v} cold/warm" for v in vals))
for name in names:
    cells = []
    for v in vals:
        xs = res[(name, v)]
        cells.append(f"{min(x[0] for x in xs):.2f} / {min(x[1] for x in xs):.2f}")
    print(name, "|", " | ".join(cells))
