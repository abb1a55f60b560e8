#!/usr/bin/env python3
"""Writes the golden vectors under tests/golden/ from the REFERENCE's own fp64 oracle.

The reference ships no data fixtures; its known answers are a 2x2 closed form and its fp64 CPU
oracle ``fa::ref::attention`` / ``attention_tiled`` (ref:src/reference/cpu_reference.cpp:83-165).
This script runs that oracle -- compiled from the reference's unmodified sources into
``oracle/_ref/libfa_ref.so`` by ``make -C oracle ref`` -- on seeded inputs and stores inputs and
outputs as ``.npz`` data. Inputs follow the reference's fixture ``make_qkv``
(ref:tests/conftest.py:99-127): one CPU ``torch.Generator`` seeded per case, fp32 ``randn`` for q, k, v
in that order, then scale and cast. Half-precision cases store the rounded inputs (bf16 as raw
uint16 bits) and the oracle output computed from exactly those rounded values.

Run (in a container that has /root/reference):  make -C oracle ref && python tests/golden/make_golden.py
"""

from __future__ import annotations

import math
import sys
from pathlib import Path

import numpy as np
import torch

ROOT = Path(__file__).resolve().parents[2]
sys.path.insert(0, str(ROOT))
from oracle.oracle import RefOracle  # noqa: E402

OUT = Path(__file__).resolve().parent


def make_qkv(b, h, n, d, hkv=None, seed=0, scale_inputs=1.0, dtype=torch.float32):
    """ref:tests/conftest.py:117-124 -- CPU generator, fp32 randn, q then k then v."""
    gen = torch.Generator(device="cpu").manual_seed(seed)
    hkv = h if hkv is None else hkv
    q = torch.randn(b, h, n, d, generator=gen, dtype=torch.float32)
    k = torch.randn(b, hkv, n, d, generator=gen, dtype=torch.float32)
    v = torch.randn(b, hkv, n, d, generator=gen, dtype=torch.float32)
    return tuple((t * scale_inputs).to(dtype).contiguous() for t in (q, k, v))


def store(t: torch.Tensor) -> np.ndarray:
    if t.dtype == torch.bfloat16:
        return t.view(torch.int16).numpy().view(np.uint16)
    return t.numpy()


def case(name, b, h, n, d, hkv=None, seed=0, dtype=torch.float32, scale=None, tiles=(),
         out_dtype=np.float64):
    ref = RefOracle()
    q, k, v = make_qkv(b, h, n, d, hkv=hkv, seed=seed, dtype=dtype)
    scale = 1.0 / math.sqrt(d) if scale is None else scale
    rec = dict(q=store(q), k=store(k), v=store(v),
               meta=np.array([b, h, k.shape[1], n, d, seed], dtype=np.int64),
               scale=np.array(scale, dtype=np.float64),
               dtype=np.array(str(dtype).replace("torch.", "")))
    for causal in (0, 1):
        o, lse = ref.attention(q, k, v, is_causal=bool(causal), scale=scale)
        rec[f"o_c{causal}"], rec[f"lse_c{causal}"] = o.astype(out_dtype), lse
        for bm, bn, tc in tiles:
            if tc != causal:
                continue
            ot, lt = ref.attention_tiled(q, k, v, bm, bn, is_causal=bool(causal), scale=scale)
            rec[f"o_c{causal}_t{bm}x{bn}"], rec[f"lse_c{causal}_t{bm}x{bn}"] = ot, lt
    np.savez_compressed(OUT / f"{name}.npz", **rec)
    print(f"wrote {name}.npz")


def closed_form():
    """ref:src/reference/test_cpu_reference.cpp:39-67: q = k = I2, v = [[1,2],[3,4]], scale 1."""
    ref = RefOracle()
    q = np.eye(2).reshape(1, 1, 2, 2)
    v = np.array([[1.0, 2.0], [3.0, 4.0]]).reshape(1, 1, 2, 2)
    rec = dict(q=q, k=q.copy(), v=v, scale=np.array(1.0))
    for causal in (0, 1):
        o, lse = ref.attention(q, q, v, is_causal=bool(causal), scale=1.0)
        rec[f"o_c{causal}"], rec[f"lse_c{causal}"] = o, lse
    np.savez_compressed(OUT / "closed_form_2x2.npz", **rec)
    print("wrote closed_form_2x2.npz")


def main() -> int:
    if not RefOracle.available():
        print("oracle/_ref/libfa_ref.so missing: run `make -C oracle ref` first", file=sys.stderr)
        return 2
    closed_form()
    # The reference's CPU-runnable case: B1 H2 N128 D64 fp32, scale 1/sqrt(D); tiled outputs pin
    # the recurrence.
    case("cpu_b1h2n128d64_f32", 1, 2, 128, 64, seed=0, tiles=((32, 16, 0), (32, 16, 1)))
    # GQA head mapping at D=128 with a non-default scale and partial tiles (N=96).
    case("gqa_b1h2kv1n96d128_f32", 1, 2, 96, 128, hkv=1, seed=3, scale=0.05, tiles=((64, 64, 1),))
    # Rounded half-precision inputs: the kernels see exactly these values. O is stored as fp32
    # (ample for the 2e-3 bar these cases are checked at); LSE stays fp64.
    case("f16_b1h2n256d64", 1, 2, 256, 64, seed=1, dtype=torch.float16, out_dtype=np.float32)
    case("bf16_b1h1n256d128", 1, 1, 256, 128, seed=2, dtype=torch.bfloat16,
         out_dtype=np.float32)
    return 0


if __name__ == "__main__":
    sys.exit(main())
