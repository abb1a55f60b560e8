"""Seeded random shapes through the split-KV decode (marker ``gpu``).

32 cases drawn once from a fixed seed cover:
* batch 1-3, 1-8 kv heads and a query-head group G of 1-16 per kv head (MHA, GQA, MQA-like),
  with Nq new tokens such that G * Nq <= 64 (one or two 32-row groups per kv head);
* cache lengths from 1 key to a few thousand: shorter than one 32-key block, ragged against the
  128-key tile, and exact multiples;
* D 64 or 128, fp16 or bf16, bottom-right causal or not, and rows that see no key when causal
  with Nq > Nkv;
* the library's split count or a forced one (1 to 16, capped by the library at one tile per
  split), and for a third of the cases a softmax scale other than 1/sqrt(D).
Every row is checked against the fp64 decode oracle at the stated tolerance (helpers from
test_decode_gpu.py). The test id spells out the draw, so a failure names its shape.
"""

from __future__ import annotations

import math
import random

import pytest
import torch

import fused_attn
from test_decode_gpu import check, make, require_ext

pytestmark = pytest.mark.gpu

DTYPES = {"fp16": torch.float16, "bf16": torch.bfloat16}


def _draw(count: int = 32, seed: int = 20261203):
    rng = random.Random(seed)
    cases = []
    for _ in range(count):
        b = rng.choice([1, 1, 2, 3])
        hkv = rng.choice([1, 2, 4, 8])
        g = rng.choice([1, 2, 4, 8, 16])
        nq = rng.randint(1, max(1, min(8, 64 // g)))
        nkv = rng.choice([rng.randint(1, 40), rng.randint(41, 700), rng.randint(701, 3000),
                          128 * rng.randint(1, 16)])
        d = rng.choice([64, 128])
        dt = rng.choice(sorted(DTYPES))
        causal = rng.random() < 0.5
        splits = rng.choice([0, 0, 1, 2, 3, 7, 16])
        scale = rng.choice([None, None, 0.5 / math.sqrt(d)])
        cases.append((b, g * hkv, hkv, nq, nkv, d, dt, causal, splits, scale))
    return cases


def _case_id(c):
    b, h, hkv, nq, nkv, d, dt, causal, splits, scale = c
    return (f"B{b}H{h}kv{hkv}Nq{nq}Nkv{nkv}D{d}{dt}{'-causal' if causal else ''}"
            f"-S{splits}{'-scaled' if scale else ''}")


@pytest.mark.parametrize("case", _draw(), ids=_case_id)
def test_random_decode_matches_oracle(case):
    require_ext()
    b, h, hkv, nq, nkv, d, dt, causal, splits, scale = case
    dtype = DTYPES[dt]
    q, k, v = make(b, h, hkv, nq, nkv, d, dtype, seed=7 * nkv + nq + h)
    print(f"random decode case {_case_id(case)}", flush=True)
    o, lse = fused_attn.decode(q, k, v, is_causal=causal, scale=scale, num_splits=splits)
    torch.cuda.synchronize()
    assert o.shape == q.shape and o.dtype == dtype and lse.shape == (b, h, nq)
    check(o, lse, q, k, v, causal, dtype, scale=scale)
