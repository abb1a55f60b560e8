"""Strided inputs through the op and the C-ABI (marker ``gpu``): the ``[B, H, N, D]`` views of
``[B, N, H, D]`` buffers (the head split of a fused QKV projection) run without a copy and give
bitwise the same answer as the dense path on the same data, which the dense parity tests tie to
the fp64 oracle. The output of ``forward_strided`` is dense in q's memory order."""

from __future__ import annotations

import random

import pytest
import torch

import fused_attn
from _checks import check_against_reference
from fused_attn import capi

pytestmark = pytest.mark.gpu

DTYPES = [torch.float16, torch.bfloat16, torch.float32]
_ids = {torch.float32: "fp32", torch.float16: "fp16", torch.bfloat16: "bf16"}


def require_ext():
    if not fused_attn.is_available():
        pytest.fail("fused_attn._C is not built: the HIP path must be the one that runs")


def qkv_views(b, h, hkv, n, d, dtype, seed):
    """q, k, v as [B, H, N, D] views of one fused [B, N, H + 2 Hkv, D] projection buffer."""
    gen = torch.Generator(device="cpu").manual_seed(seed)
    buf = torch.randn(b, n, h + 2 * hkv, d, generator=gen).to("cuda", dtype)
    q = buf[:, :, :h].transpose(1, 2)
    k = buf[:, :, h:h + hkv].transpose(1, 2)
    v = buf[:, :, h + hkv:].transpose(1, 2)
    return q, k, v


@pytest.mark.parametrize("causal", [False, True], ids=["full", "causal"])
@pytest.mark.parametrize("d", [64, 128])
@pytest.mark.parametrize("dtype", DTYPES, ids=lambda t: _ids[t])
def test_strided_views_equal_dense_bitwise(dtype, d, causal):
    require_ext()
    q, k, v = qkv_views(2, 4, 4, 256, d, dtype, seed=3)
    assert not q.is_contiguous() and q.stride(-1) == 1
    o = fused_attn.forward_strided(q, k, v, is_causal=causal)
    o_dense = fused_attn.forward(q.contiguous(), k.contiguous(), v.contiguous(), is_causal=causal)
    torch.cuda.synchronize()
    assert torch.equal(o, o_dense)
    # Output memory follows q's order: [B, N, H, D] dense, so the transpose back is free.
    assert o.transpose(1, 2).is_contiguous()


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16], ids=lambda t: _ids[t])
def test_strided_gqa_against_fp64(dtype):
    require_ext()
    q, k, v = qkv_views(1, 8, 2, 512, 64, dtype, seed=5)
    o = fused_attn.forward_strided(q, k, v, is_causal=True)
    torch.cuda.synchronize()
    check_against_reference(o, q.contiguous(), k.contiguous(), v.contiguous(), True, dtype)


def test_contiguous_inputs_give_contiguous_output():
    require_ext()
    gen = torch.Generator(device="cpu").manual_seed(1)
    q, k, v = (torch.randn(1, 2, 128, 64, generator=gen).to("cuda", torch.float16)
               for _ in range(3))
    o = fused_attn.forward_strided(q, k, v)
    assert o.is_contiguous()
    assert torch.equal(o, fused_attn.forward(q, k, v))


def test_capi_strided_output_into_a_wider_buffer():
    """o is a strided view into a bigger buffer: the kernel writes exactly its elements."""
    require_ext()
    q, k, v = qkv_views(2, 2, 2, 128, 64, torch.float16, seed=7)
    big = torch.full((2, 128, 3, 64), 7.0, dtype=torch.float16, device="cuda")
    o = big[:, :, 1:3].transpose(1, 2)  # [B, H, N, D] view, row stride 3 * 64
    lse = torch.empty(2, 2, 128, dtype=torch.float32, device="cuda")
    rc = capi.forward_strided(5, q, k, v, o, lse, True, 0.125)
    torch.cuda.synchronize()
    assert rc == 0, capi.error_string(rc)
    assert torch.all(big[:, :, 0] == 7.0)
    o_ref, lse_ref = fused_attn.forward_stage(q.contiguous(), k.contiguous(), v.contiguous(), 5,
                                              is_causal=True, scale=0.125)
    assert torch.equal(o, o_ref) and torch.equal(lse, lse_ref)


def test_strided_input_errors():
    require_ext()
    q, k, v = qkv_views(1, 2, 2, 64, 64, torch.float16, seed=9)
    with pytest.raises(RuntimeError, match="contiguous head dim"):
        fused_attn.forward_strided(q.transpose(2, 3), k, v)
    odd = torch.zeros(1, 64, 2, 68, dtype=torch.float16, device="cuda")[..., :64].transpose(1, 2)
    with pytest.raises(RuntimeError, match="multiples of 16 bytes"):
        fused_attn.forward_strided(odd, k, v)
    with pytest.raises(RuntimeError, match="multiple of 32"):
        fused_attn.forward_strided(q[:, :, :48], k[:, :, :48], v[:, :, :48])
    # The reference's own op keeps its contract: dense tensors only.
    with pytest.raises(RuntimeError, match="contiguous"):
        fused_attn.forward(q, k, v)


def test_opcheck_forward_strided():
    require_ext()
    q, k, v = qkv_views(1, 2, 2, 128, 64, torch.float16, seed=11)
    torch.library.opcheck(torch.ops.fused_attn.forward_strided, (q, k, v, True, 0.125),
                          test_utils=("test_schema", "test_faketensor"))


def _layout_views(layout, b, h, hkv, n, d, dtype, seed):
    """q, k, v [B, *, N, D] views of one of three memory layouts (each row 16-byte aligned):
    'qkv' the fused projection buffer above; 'padded' [B, N, heads, D + pad] buffers cut to D;
    'batch' every other batch of [2B, heads, N, D] buffers (a doubled batch stride)."""
    if layout == "qkv":
        return qkv_views(b, h, hkv, n, d, dtype, seed)
    gen = torch.Generator(device="cpu").manual_seed(seed)
    pad = 16 // torch.empty((), dtype=dtype).element_size() * (1 + seed % 3)
    out = []
    for heads in (h, hkv, hkv):
        if layout == "padded":
            buf = torch.randn(b, n, heads, d + pad, generator=gen).to("cuda", dtype)
            out.append(buf[..., :d].transpose(1, 2))
        else:
            buf = torch.randn(2 * b, heads, n, d, generator=gen).to("cuda", dtype)
            out.append(buf[::2])
    return tuple(out)


def _draw_strided(count: int = 24, seed: int = 20261206):
    rng = random.Random(seed)
    cases = []
    for _ in range(count):
        layout = rng.choice(["qkv", "padded", "batch"])
        b = rng.choice([1, 2, 3])
        h = rng.choice([1, 2, 4, 6, 8])
        hkv = rng.choice([x for x in range(1, h + 1) if h % x == 0])
        n = 32 * rng.randint(1, 12)
        d = rng.choice([64, 128])
        dtype = rng.choice(DTYPES)
        causal = rng.random() < 0.5
        cases.append((layout, b, h, hkv, n, d, dtype, causal))
    return cases


@pytest.mark.parametrize("case", _draw_strided(), ids=lambda c: "{}-B{}H{}kv{}N{}D{}{}{}".format(
    c[0], *c[1:6], _ids[c[6]], "-causal" if c[7] else ""))
def test_random_strided_layouts(case):
    """Seeded random layouts, shapes, dtypes and masks: forward_strided on the views equals the
    dense forward on the same data bit for bit, and that forward meets the bar against the fp64
    oracle."""
    require_ext()
    layout, b, h, hkv, n, d, dtype, causal = case
    q, k, v = _layout_views(layout, b, h, hkv, n, d, dtype, seed=n + h + d)
    assert q.stride(-1) == 1
    assert not q.is_contiguous() or (layout == "batch" and b == 1)  # one batch of B is dense
    print(f"strided case {case}", flush=True)
    o = fused_attn.forward_strided(q, k, v, is_causal=causal)
    qd, kd, vd = q.contiguous(), k.contiguous(), v.contiguous()
    o_dense = fused_attn.forward(qd, kd, vd, is_causal=causal)
    torch.cuda.synchronize()
    assert torch.equal(o, o_dense)
    check_against_reference(o_dense, qd, kd, vd, causal, dtype)
