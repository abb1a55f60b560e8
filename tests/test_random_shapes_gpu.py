"""Seeded random shapes through stage 5 (marker ``gpu``).

48 cases drawn once from a fixed seed cover:
* batch 1-3 and 1-24 query heads, several of them multiples of 8, whose causal grids are issued
  tile-major;
* kv heads a divisor of the query heads (GQA/MQA);
* N a multiple of 32 up to 640 (partial query and key tiles), D 64 or 128;
* fp16 or bf16, causal or not;
* for some, a forced split count of 2, 3 or 5, with the workspace the op sizes through
  ``fa_workspace_bytes``.
A third draw of 24 cases runs the other two stages the library builds: stage 3 (the fp32
rung, checked at fp32's 1e-5 bar) and stage 4 (16-bit, synchronous staging), with GQA, partial
tiles, D and causal drawn as above.
A fourth draw of 12 cases takes sequences of 640 to 4096 tokens, checked on every head
against plain PyTorch fp32 attention on the GPU (the fp64 oracle would take minutes there).
A second draw of 24 cases takes a softmax scale other than 1/sqrt(D): a quarter of it (flat
rows, where the 16-bit rounding of the probabilities averages out least) or twice it (peaked
rows, where the running max moves most). Each case runs on the tile the library picks by itself. Every head is checked against the fp64
oracle at the stated tolerance (tests/_checks.py). The test id spells out the draw, so a failure
names its shape.
"""

from __future__ import annotations

import random

import pytest
import torch

import fused_attn
from _checks import LSE_ATOL, O_TOL, check_against_reference, fp32_reference_head

pytestmark = pytest.mark.gpu

DTYPES = {"fp16": torch.float16, "bf16": torch.bfloat16}


def _draw(count: int = 48, seed: int = 20261202):
    rng = random.Random(seed)
    cases = []
    for _ in range(count):
        b = rng.choice([1, 1, 2, 3])
        h = rng.choice([1, 2, 3, 4, 6, 8, 12, 16, 24])
        hkv = rng.choice([x for x in range(1, h + 1) if h % x == 0])
        n = 32 * rng.randint(1, 20)
        d = rng.choice([64, 128])
        dt = rng.choice(sorted(DTYPES))
        causal = rng.random() < 0.5
        splits = rng.choice([0, 0, 0, 2, 3, 5])
        cases.append((b, h, hkv, n, d, dt, causal, splits))
    return cases


def _draw_scaled(count: int = 24, seed: int = 20261204):
    rng = random.Random(seed)
    cases = []
    for _ in range(count):
        b = rng.choice([1, 2])
        h = rng.choice([1, 2, 4, 8])
        hkv = rng.choice([x for x in range(1, h + 1) if h % x == 0])
        n = 32 * rng.choice([1, 1, 2, 3, rng.randint(4, 16)])
        d = rng.choice([64, 128])
        dt = rng.choice(sorted(DTYPES))
        causal = rng.random() < 0.5
        splits = rng.choice([0, 0, 2, 3])
        mul = rng.choice([0.25, 2.0])
        cases.append((b, h, hkv, n, d, dt, causal, splits, mul))
    return cases


def _case_id(c):
    b, h, hkv, n, d, dt, causal, splits = c
    return f"B{b}H{h}kv{hkv}N{n}D{d}{dt}{'-causal' if causal else ''}{f'-S{splits}' if splits else ''}"


@pytest.mark.parametrize("case", _draw(), ids=_case_id)
def test_random_shape_matches_oracle(case, make_qkv, monkeypatch):
    if not fused_attn.is_available():
        pytest.fail("fused_attn._C is not built: the HIP path must be the one that runs")
    b, h, hkv, n, d, dt, causal, splits = case
    dtype = DTYPES[dt]
    if not fused_attn.impl_supports(5, dtype, d):
        pytest.skip(f"stage 5 is not built for {dt} D={d} on this GPU")
    if splits:
        monkeypatch.setenv("FA_FORCE_SPLITS", str(splits))
    else:
        monkeypatch.delenv("FA_FORCE_SPLITS", raising=False)
    q, k, v = make_qkv(b, h, n, d, dtype=dtype, device="cuda", hkv=hkv, seed=n + 7 * h + d)
    o, lse = fused_attn.forward_stage(q, k, v, 5, is_causal=causal)
    torch.cuda.synchronize()
    check_against_reference(o, q, k, v, causal, dtype, lse=lse)


@pytest.mark.parametrize("case", _draw_scaled(),
                         ids=lambda c: f"{_case_id(c[:8])}-scale{c[8]}x")
def test_random_scaled_shape_matches_oracle(case, make_qkv, monkeypatch):
    if not fused_attn.is_available():
        pytest.fail("fused_attn._C is not built: the HIP path must be the one that runs")
    b, h, hkv, n, d, dt, causal, splits, mul = case
    dtype = DTYPES[dt]
    if not fused_attn.impl_supports(5, dtype, d):
        pytest.skip(f"stage 5 is not built for {dt} D={d} on this GPU")
    if splits:
        monkeypatch.setenv("FA_FORCE_SPLITS", str(splits))
    else:
        monkeypatch.delenv("FA_FORCE_SPLITS", raising=False)
    q, k, v = make_qkv(b, h, n, d, dtype=dtype, device="cuda", hkv=hkv, seed=n + 5 * h + d + 1)
    scale = mul / d ** 0.5
    o, lse = fused_attn.forward_stage(q, k, v, 5, is_causal=causal, scale=scale)
    torch.cuda.synchronize()
    check_against_reference(o, q, k, v, causal, dtype, scale=scale, lse=lse)


def _draw_stages(count: int = 24, seed: int = 20261205):
    rng = random.Random(seed)
    cases = []
    for _ in range(count):
        stage = rng.choice([3, 4])
        b = rng.choice([1, 2])
        h = rng.choice([1, 2, 3, 4, 6, 8])
        hkv = rng.choice([x for x in range(1, h + 1) if h % x == 0])
        n = 32 * rng.randint(1, 12)
        d = rng.choice([64, 128])
        dt = "fp32" if stage == 3 else rng.choice(sorted(DTYPES))
        causal = rng.random() < 0.5
        cases.append((stage, b, h, hkv, n, d, dt, causal))
    return cases


@pytest.mark.parametrize("case", _draw_stages(),
                         ids=lambda c: f"s{c[0]}-{_case_id(c[1:] + (0,))}")
def test_random_shape_other_stages(case, make_qkv):
    if not fused_attn.is_available():
        pytest.fail("fused_attn._C is not built: the HIP path must be the one that runs")
    stage, b, h, hkv, n, d, dt, causal = case
    dtype = torch.float32 if dt == "fp32" else DTYPES[dt]
    if not fused_attn.impl_supports(stage, dtype, d):
        pytest.skip(f"stage {stage} is not built for {dt} D={d} on this GPU")
    q, k, v = make_qkv(b, h, n, d, dtype=dtype, device="cuda", hkv=hkv, seed=n + 3 * h + d + stage)
    o, lse = fused_attn.forward_stage(q, k, v, stage, is_causal=causal)
    torch.cuda.synchronize()
    check_against_reference(o, q, k, v, causal, dtype, lse=lse)


def _draw_large(count: int = 12, seed: int = 20261207):
    rng = random.Random(seed)
    cases = []
    for _ in range(count):
        b = rng.choice([1, 2, 4])
        h = rng.choice([2, 4, 8, 12, 16])
        hkv = rng.choice([x for x in range(1, h + 1) if h % x == 0])
        n = 32 * rng.randint(20, 128)
        d = rng.choice([64, 128])
        dt = rng.choice(sorted(DTYPES))
        causal = rng.random() < 0.5
        cases.append((b, h, hkv, n, d, dt, causal, 0))
    return cases


@pytest.mark.parametrize("case", _draw_large(), ids=lambda c: f"large-{_case_id(c)}")
def test_random_large_shape_every_head(case, make_qkv, monkeypatch):
    """Sequences of 640 to 4096 tokens (the automatic tile and split choices of mid-sized grids),
    every row of every head against plain PyTorch fp32 attention on the GPU at the stated bar."""
    if not fused_attn.is_available():
        pytest.fail("fused_attn._C is not built: the HIP path must be the one that runs")
    b, h, hkv, n, d, dt, causal, _ = case
    dtype = DTYPES[dt]
    if not fused_attn.impl_supports(5, dtype, d):
        pytest.skip(f"stage 5 is not built for {dt} D={d} on this GPU")
    monkeypatch.delenv("FA_FORCE_SPLITS", raising=False)
    q, k, v = make_qkv(b, h, n, d, dtype=dtype, device="cuda", hkv=hkv, seed=n + h + d + 2)
    scale = 1.0 / d ** 0.5
    o, lse = fused_attn.forward_stage(q, k, v, 5, is_causal=causal)
    torch.cuda.synchronize()
    atol, rtol = O_TOL[dtype]
    for bi in range(b):
        for hi in range(h):
            o32, lse32, _s = fp32_reference_head(q, k, v, bi, hi, causal, scale)
            err = (o[bi, hi].float() - o32).abs()
            excess = float((err - (atol + rtol * o32.abs())).max())
            assert excess <= 0.0, f"head ({bi},{hi}): max|O err| {float(err.max()):.3e}"
            lerr = float((lse[bi, hi] - lse32).abs().max())
            assert lerr <= LSE_ATOL, f"head ({bi},{hi}): max|LSE err| {lerr:.3e}"
