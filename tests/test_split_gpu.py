"""Split key walks of stage 5 (marker ``gpu``).

With a workspace, stage 5 may cut every query tile's key walk into S parts of whole key tiles,
one workgroup each. Each part writes its normalised fp32 O and its LSE to the workspace, and
``fa_s5_combine`` merges them with the log-sum-exp rule (ref:include/fa/softmax_math.cuh:65-68).
The library splits where its cost model says the GPU would otherwise sit idle (one GPU's share of
a head-sharded problem); ``FA_FORCE_SPLITS`` forces S for these tests.

* Forced S in {2, 3, 5} on full and causal problems, fp16 and bf16, D 64 and 128, with N an odd
  multiple of 32 (partial tiles), against the fp64 oracle at the stated tolerance; one shape has
  B * H a multiple of 8, whose causal grid is issued tile-major.
* More parts than key tiles: the empty parts carry LSE = -inf and weigh nothing.
* The shapes the model splits by itself: the C-ABI asks for a workspace, and the op
  (``torch.ops.fused_attn.forward``, which allocates what ``fa_workspace_bytes`` asks for) and the
  C-ABI without a workspace (the whole-walk kernel) both match the oracle.
* A split launch (two kernels) captured into a HIP graph replays bit-identically.
* Walk orders: in-order and rotated walks (one start per 128-row block, or per group of blocks)
  all meet the oracle; on the D = 64 BR x 32 tiles, rotated walks give heights 128, 64 and 32
  the same bits, and the GPT-2 attention shape's automatic tile is that rotated walk.
"""

from __future__ import annotations

import math

import pytest
import torch

import fused_attn
from _checks import check_against_reference
from fused_attn import capi
from oracle.oracle import math_reference

pytestmark = pytest.mark.gpu


def _require():
    if not fused_attn.is_available():
        pytest.fail("fused_attn._C is not built: the HIP path must be the one that runs")


def _inputs(b, h, n, d, dtype, seed):
    g = torch.Generator(device="cpu").manual_seed(seed)
    return tuple(torch.randn(b, h, n, d, generator=g).to("cuda", dtype) for _ in range(3))


def _split_run(q, k, v, causal, scale):
    nbytes = capi.workspace_bytes(5, q, k, causal, scale)
    assert nbytes > 0, "the split path needs a workspace"
    ws = torch.empty(nbytes, dtype=torch.uint8, device="cuda")
    o = torch.empty_like(q)
    lse = torch.empty(q.shape[:3], dtype=torch.float32, device="cuda")
    rc = capi.forward(5, q, k, v, o, lse, causal, scale, workspace=ws)
    assert rc == capi.HIP_SUCCESS, capi.error_string(rc)
    torch.cuda.synchronize()
    return o, lse


@pytest.mark.parametrize("splits", [2, 3, 5])
@pytest.mark.parametrize("causal", [False, True], ids=["full", "causal"])
# (2, 8, 288, 64): B * H a multiple of 8, so the causal runs are issued tile-major
# (layout::grid_item) with the parts of each query tile consecutive on one XCD.
@pytest.mark.parametrize("b,h,n,d", [(1, 2, 352, 64), (2, 3, 224, 128), (1, 1, 1024, 64),
                                     (2, 8, 288, 64)],
                         ids=lambda x: str(x))
@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16], ids=["fp16", "bf16"])
def test_forced_splits_match_oracle(b, h, n, d, dtype, causal, splits, monkeypatch):
    _require()
    monkeypatch.setenv("FA_FORCE_SPLITS", str(splits))
    q, k, v = _inputs(b, h, n, d, dtype, seed=splits + 10 * n)
    o, lse = _split_run(q, k, v, causal, 1.0 / math.sqrt(d))
    check_against_reference(o, q, k, v, causal, dtype, lse=lse)


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16], ids=["fp16", "bf16"])
def test_more_parts_than_key_tiles(dtype, monkeypatch):
    """N = 96 at D = 128 is 2 key tiles of 64 (the first query tile's causal walk is 1): most of
    the 7 parts are empty."""
    _require()
    monkeypatch.setenv("FA_FORCE_SPLITS", "7")
    q, k, v = _inputs(2, 2, 96, 128, dtype, seed=5)
    for causal in (False, True):
        o, lse = _split_run(q, k, v, causal, 1.0 / math.sqrt(128))
        check_against_reference(o, q, k, v, causal, dtype, lse=lse)


@pytest.mark.parametrize("b,h,n,d,dtype,causal", [
    (2, 1, 2048, 128, torch.float16, True),    # C128 causal over 8 GPUs by heads: 3 parts
    (1, 2, 8192, 128, torch.bfloat16, True),   # LONG over 8 GPUs by heads: 2 parts
    (1, 1, 2048, 64, torch.float16, False),    # one head at D = 64: 4 parts
], ids=["C128-causal-heads8", "long-heads8", "one-head-d64"])
def test_model_splits_share_shapes(b, h, n, d, dtype, causal, monkeypatch):
    _require()
    monkeypatch.delenv("FA_FORCE_SPLITS", raising=False)
    q, k, v = _inputs(b, h, n, d, dtype, seed=21)
    scale = 1.0 / math.sqrt(d)
    assert capi.workspace_bytes(5, q, k, causal, scale) > 0, "the cost model should split here"
    o_op = fused_attn.forward(q, k, v, is_causal=causal)  # the op allocates the workspace
    o_whole = torch.empty_like(q)
    lse_whole = torch.empty(b, h, n, dtype=torch.float32, device="cuda")
    assert capi.forward(5, q, k, v, o_whole, lse_whole, causal, scale, workspace=None) == 0
    torch.cuda.synchronize()
    check_against_reference(o_op, q, k, v, causal, dtype)
    check_against_reference(o_whole, q, k, v, causal, dtype, lse=lse_whole)


def test_split_launch_in_graph(monkeypatch):
    """Both kernels of a split launch replay from a graph, bit-identical to the eager launch."""
    _require()
    monkeypatch.setenv("FA_FORCE_SPLITS", "3")
    q, k, v = _inputs(1, 4, 512, 128, torch.bfloat16, seed=8)
    scale = 0.088
    ws = torch.empty(capi.workspace_bytes(5, q, k, True, scale), dtype=torch.uint8, device="cuda")
    o = torch.empty_like(q)
    lse = torch.empty(1, 4, 512, dtype=torch.float32, device="cuda")
    stream = torch.cuda.Stream()
    with torch.cuda.stream(stream):
        assert capi.forward(5, q, k, v, o, lse, True, scale, stream=stream, workspace=ws) == 0
    stream.synchronize()
    o_ref, lse_ref = o.clone(), lse.clone()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=stream):
        capi.forward(5, q, k, v, o, lse, True, scale, stream=stream, workspace=ws)
    for r in range(3):
        o.zero_()
        lse.zero_()
        x = torch.randn(256, 256, device="cuda")
        (x @ x).sum().item()
        torch.cuda.synchronize()
        with torch.cuda.stream(stream):
            graph.replay()
        stream.synchronize()
        assert torch.equal(o, o_ref) and torch.equal(lse, lse_ref), f"replay {r} differs"


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16], ids=["fp16", "bf16"])
def test_split_strided_views(dtype, monkeypatch):
    """fa_forward_strided with a split: q/k/v are head splits of [B, N, H, D] buffers and o a view
    into a wider buffer. The combine writes exactly o's elements, and the result equals the split
    launch on contiguous copies bit for bit (same arithmetic, other addresses)."""
    _require()
    monkeypatch.setenv("FA_FORCE_SPLITS", "3")
    b, h, n, d = 2, 3, 224, 64
    g = torch.Generator(device="cpu").manual_seed(17)
    q, k, v = (torch.randn(b, n, h, d, generator=g).to("cuda", dtype).transpose(1, 2)
               for _ in range(3))
    big = torch.full((b, n, h + 1, d), 7.0, dtype=dtype, device="cuda")
    o = big[:, :, 1:].transpose(1, 2)
    lse = torch.empty(b, h, n, dtype=torch.float32, device="cuda")
    scale = 1.0 / math.sqrt(d)
    assert capi.forward_strided(5, q, k, v, o, lse, True, scale) == 0  # workspace "auto"
    torch.cuda.synchronize()
    assert torch.all(big[:, :, 0] == 7.0)
    o_ref, lse_ref = _split_run(q.contiguous(), k.contiguous(), v.contiguous(), True, scale)
    assert torch.equal(o, o_ref) and torch.equal(lse, lse_ref)
    check_against_reference(o.contiguous(), q.contiguous(), k.contiguous(), v.contiguous(), True,
                            dtype, lse=lse)


def test_op_strided_splits(monkeypatch):
    """torch.ops.fused_attn.forward_strided allocates the split workspace as forward does."""
    _require()
    monkeypatch.setenv("FA_FORCE_SPLITS", "2")
    g = torch.Generator(device="cpu").manual_seed(23)
    q, k, v = (torch.randn(1, 256, 4, 128, generator=g).to("cuda", torch.bfloat16).transpose(1, 2)
               for _ in range(3))
    o = fused_attn.forward_strided(q, k, v, is_causal=True)
    o_ref = fused_attn.forward(q.contiguous(), k.contiguous(), v.contiguous(), is_causal=True)
    assert torch.equal(o, o_ref)
    check_against_reference(o_ref, q.contiguous(), k.contiguous(), v.contiguous(), True,
                            torch.bfloat16)


@pytest.mark.parametrize("hkv", [1, 2])
@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16], ids=["fp16", "bf16"])
def test_gqa_splits(hkv, dtype, monkeypatch):
    """GQA / MQA with split walks: query head h reads kv head h // (H / Hkv) in every part."""
    _require()
    monkeypatch.setenv("FA_FORCE_SPLITS", "3")
    g = torch.Generator(device="cpu").manual_seed(31 + hkv)
    q = torch.randn(1, 4, 352, 128, generator=g).to("cuda", dtype)
    k, v = (torch.randn(1, hkv, 352, 128, generator=g).to("cuda", dtype) for _ in range(2))
    for causal in (False, True):
        o, lse = _split_run(q, k, v, causal, 1.0 / math.sqrt(128))
        check_against_reference(o, q, k, v, causal, dtype, lse=lse)


@pytest.mark.parametrize("b,h,n,d,dtype,causal", [
    (2, 8, 1024, 128, torch.float16, False),
    (2, 4, 768, 64, torch.float16, True),
    (1, 8, 1056, 128, torch.bfloat16, True),
    (2, 2, 640, 64, torch.bfloat16, False),
], ids=lambda x: str(x))
def test_rotated_and_in_order_walks_both_meet_the_oracle(b, h, n, d, dtype, causal, monkeypatch):
    """The key walk's order (in order, or rotated so that workgroups sharing a head fetch different
    tiles at a time: one start per 128-row block, or one per group of blocks) only reorders each
    row's accumulation: every order meets the fp64 oracle, forced with the test-only
    FA_FORCE_ROTATE and FA_FORCE_ROT_GROUPS. One group is the in-order walk again, bit for bit."""
    gen = torch.Generator().manual_seed(31)
    q, k, v = (torch.randn(b, h, n, d, generator=gen).to("cuda", dtype) for _ in range(3))
    ref, lse64 = math_reference(q, k, v, is_causal=causal)
    outs = {}
    for rotate, groups in (("0", None), ("1", None), ("1", "1"), ("1", "2"), ("1", "4")):
        monkeypatch.setenv("FA_FORCE_ROTATE", rotate)
        if groups is None:
            monkeypatch.delenv("FA_FORCE_ROT_GROUPS", raising=False)
        else:
            monkeypatch.setenv("FA_FORCE_ROT_GROUPS", groups)
        o, lse = fused_attn.forward_stage(q, k, v, 5, is_causal=causal)
        torch.cuda.synchronize()
        what = f"FA_FORCE_ROTATE={rotate} FA_FORCE_ROT_GROUPS={groups}"
        err = float(abs(o.double().cpu().numpy() - ref).max())
        lerr = float(abs(lse.double().cpu().numpy() - lse64).max())
        tol = 2e-3 + (2e-3 if dtype == torch.float16 else 2 ** -8) * float(abs(ref).max())
        assert err <= tol, f"{what}: O error {err:.3e}"
        assert lerr <= 1e-3, f"{what}: LSE error {lerr:.3e}"
        outs[(rotate, groups)] = (o, lse)
    in_order, one_group = outs[("0", None)], outs[("1", "1")]
    assert torch.equal(in_order[0], one_group[0]) and torch.equal(in_order[1], one_group[1])
    monkeypatch.delenv("FA_FORCE_ROTATE")
    monkeypatch.delenv("FA_FORCE_ROT_GROUPS", raising=False)


@pytest.mark.parametrize("b,h,n,d,dtype,causal", [
    (2, 4, 768, 64, torch.float16, True),
    (1, 8, 1056, 64, torch.bfloat16, False),
    (8, 12, 1024, 64, torch.float16, True),
], ids=lambda x: str(x))
def test_rotated_bc32_walks_match_across_heights(b, h, n, d, dtype, causal, monkeypatch):
    """The D = 64 tile of one 32-key split per wave (BC 32, the automatic tile of D = 64 grids
    with two or more BR-128 workgroups per CU, rotated up to 4 MB of K/V per XCD): with the walks
    rotated, heights 128, 64 and 32 give every 32-row wave the same key tiles in the same order,
    so their outputs are equal bit for bit, and they meet the fp64 oracle. The last shape is the
    GPT-2 attention shape, which takes this tile and rotation by itself."""
    _require()
    gen = torch.Generator().manual_seed(37)
    q, k, v = (torch.randn(b, h, n, d, generator=gen).to("cuda", dtype) for _ in range(3))
    monkeypatch.setenv("FA_FORCE_ROTATE", "1")
    monkeypatch.delenv("FA_FORCE_ROT_GROUPS", raising=False)
    fused_attn.set_debug_overrides(0, 0)
    p = capi.params(b, h, h, n, d, d ** -0.5, causal)
    try:
        outs = []
        for br in (128, 64, 32):
            fused_attn.set_debug_overrides(br, 32)
            assert capi.s5_plan(capi.DTYPE_CODES[dtype], p)[:2] == (br, 32)
            outs.append(fused_attn.forward_stage(q, k, v, 5, is_causal=causal))
        torch.cuda.synchronize()
    finally:
        fused_attn.set_debug_overrides(0, 0)
    for br, (o, lse) in zip((64, 32), outs[1:]):
        assert torch.equal(o, outs[0][0]) and torch.equal(lse, outs[0][1]), f"BR {br} differs"
    check_against_reference(outs[0][0], q, k, v, causal, dtype, lse=outs[0][1])
    if (b, h, n) == (8, 12, 1024):
        # Without FA_FORCE_ROTATE: the automatic tile, and every forced height at its width,
        # rotate by themselves (the 4 MB bound follows the width).
        monkeypatch.delenv("FA_FORCE_ROTATE")
        try:
            for br in (0, 64, 32):
                fused_attn.set_debug_overrides(br, 0)
                assert capi.s5_plan(capi.DTYPE_CODES[dtype], p)[:2] == (br or 128, 32)
                o, lse = fused_attn.forward_stage(q, k, v, 5, is_causal=causal)
                torch.cuda.synchronize()
                assert torch.equal(o, outs[0][0]) and torch.equal(lse, outs[0][1]), \
                    f"BR {br or 'auto'} is not the rotated BC 32 walk"
        finally:
            fused_attn.set_debug_overrides(0, 0)
