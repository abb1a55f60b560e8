"""FA_S5_PREFETCH (ref:src/stage5_tuned.cu:763-775): "0" turns stage 5's pipelined K/V staging off.

Stage 5 then launches, for the tile its rules pick, the synchronous instantiation of the same
kernel body -- stage 4's loop (load, barrier, compute, barrier) -- so on stage 4's own tile
(BR 128 at the default width) its outputs must equal stage 4's bit for bit, while stage 5 with the
knob unset runs the pipelined loop. A tile stage 4 does not build (BR 64) still runs under the
knob, on the synchronous table that mirrors every stage-5 tile, and meets the fp64 oracle.

The library reads the variable once per process, so each case runs in a child process (one at a
time, on the one GPU) that prints its findings as JSON.
"""

from __future__ import annotations

import json
import os
import subprocess
import sys
from pathlib import Path

import pytest

pytestmark = pytest.mark.gpu

ROOT = Path(__file__).resolve().parents[1]

CHILD = r"""
import json, sys
sys.path[:0] = [sys.argv[1], sys.argv[1] + "/fused-attention-cuda_amd"]
import torch
import fused_attn
from oracle.oracle import math_reference
b, h, n, d, causal, dt = int(sys.argv[2]), int(sys.argv[3]), int(sys.argv[4]), int(sys.argv[5]), \
    sys.argv[6] == "1", {"fp16": torch.float16, "bf16": torch.bfloat16}[sys.argv[7]]
g = torch.Generator().manual_seed(5)
q, k, v = (torch.randn(b, h, n, d, generator=g).to("cuda", dt) for _ in range(3))
o5, l5 = fused_attn.forward_stage(q, k, v, 5, is_causal=causal)
o4, l4 = fused_attn.forward_stage(q, k, v, 4, is_causal=causal)
torch.cuda.synchronize()
ref, lse64 = math_reference(q, k, v, is_causal=causal)
err = float(abs(o5.double().cpu().numpy() - ref).max())
lerr = float(abs(l5.double().cpu().numpy() - lse64).max())
print(json.dumps({"equal_s4": bool(torch.equal(o5, o4) and torch.equal(l5, l4)),
                  "err_o": err, "err_lse": lerr, "ref_max": float(abs(ref).max())}))
"""


def _child(env_extra: dict[str, str], *shape) -> dict:
    env = {k: v for k, v in os.environ.items()
           if k not in ("FA_S5_PREFETCH", "FA_FORCE_BR", "FA_FORCE_BC", "FA_FORCE_SPLITS")}
    env.update(env_extra)
    args = [sys.executable, "-c", CHILD, str(ROOT), *map(str, shape)]
    print("case:", env_extra, shape, flush=True)
    r = subprocess.run(args, env=env, capture_output=True, text=True, timeout=240)
    assert r.returncode == 0, r.stdout[-2000:] + r.stderr[-3000:]
    return json.loads(r.stdout.strip().splitlines()[-1])


@pytest.mark.parametrize("d,dt,bc", [(64, "fp16", 128), (128, "bf16", 64)])
def test_prefetch_off_is_stage4_bit_for_bit(d, dt, bc):
    forced = {"FA_FORCE_BR": "128", "FA_FORCE_BC": str(bc)}
    off = _child({**forced, "FA_S5_PREFETCH": "0"}, 1, 4, 640, d, 1, dt)
    assert off["equal_s4"], "FA_S5_PREFETCH=0 must run stage 4's synchronous loop on its tile"
    tol = 2e-3 + (2e-3 if dt == "fp16" else 2 ** -8) * off["ref_max"]
    assert off["err_o"] <= tol and off["err_lse"] <= 1e-3, off
    on = _child(forced, 1, 4, 640, d, 1, dt)
    assert on["err_o"] <= tol and on["err_lse"] <= 1e-3, on


def test_prefetch_off_on_a_tile_stage4_does_not_build():
    # BR 64 / BC 64 at D = 64: stage 4 keeps BR 128, so its output differs only in the
    # accumulation order; stage 5's synchronous instantiation of this tile meets the oracle.
    off = _child({"FA_FORCE_BR": "64", "FA_FORCE_BC": "64", "FA_S5_PREFETCH": "0"},
                 2, 2, 384, 64, 0, "fp16")
    assert off["err_o"] <= 2e-3 + 2e-3 * off["ref_max"] and off["err_lse"] <= 1e-3, off
