"""HIP graph capture of the forward and decode paths (marker ``gpu``).

Callers under HIP graph capture can use ``fa_forward`` directly: the library allocates nothing
and records no memset. These tests capture launches into a
``torch.cuda.CUDAGraph``, replay the graph several times with unrelated eager work and
synchronisations in between, and compare every replay bitwise with the eager launches (the
kernels are deterministic). The outputs are cleared before each replay, so a replay that did not
run would fail the comparison.
"""

from __future__ import annotations

import math

import pytest
import torch

import fused_attn
from fused_attn import capi

pytestmark = pytest.mark.gpu


def _require():
    if not fused_attn.is_available():
        pytest.fail("fused_attn._C is not built: the HIP path must be the one that runs")


def _inputs(b, h, n, d, dtype, seed, hkv=None):
    g = torch.Generator(device="cpu").manual_seed(seed)
    hkv = hkv or h
    q = torch.randn(b, h, n, d, generator=g).to("cuda", dtype)
    k = torch.randn(b, hkv, n, d, generator=g).to("cuda", dtype)
    v = torch.randn(b, hkv, n, d, generator=g).to("cuda", dtype)
    return q, k, v


def _replay_checked(graph, stream, outs, refs, replays=3):
    for r in range(replays):
        for t in outs:
            t.zero_()
        # Unrelated eager work between replays, as a caller's program would have.
        x = torch.randn(256, 256, device="cuda")
        (x @ x).sum().item()
        torch.cuda.synchronize()
        with torch.cuda.stream(stream):
            graph.replay()
        stream.synchronize()
        for i, (t, ref) in enumerate(zip(outs, refs)):
            assert torch.equal(t, ref), f"replay {r}: output {i} differs from the eager launch"


@pytest.mark.parametrize("causal", [False, True], ids=["full", "causal"])
@pytest.mark.parametrize("dtype,d", [(torch.float16, 64), (torch.bfloat16, 128)],
                         ids=["fp16-D64", "bf16-D128"])
def test_capi_forward_in_graph(dtype, d, causal):
    _require()
    b, h, n = 1, 4, 512
    sets = [_inputs(b, h, n, d, dtype, seed) for seed in (1, 2, 3)]
    outs = [(torch.empty_like(q), torch.empty(b, h, n, device="cuda", dtype=torch.float32))
            for q, _, _ in sets]
    scale = 1.0 / math.sqrt(d)
    stream = torch.cuda.Stream()
    with torch.cuda.stream(stream):
        for (q, k, v), (o, lse) in zip(sets, outs):
            assert capi.forward(5, q, k, v, o, lse, causal, scale, stream=stream) == 0
    stream.synchronize()
    refs = [t.clone() for pair in outs for t in pair]
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=stream):
        for (q, k, v), (o, lse) in zip(sets, outs):
            capi.forward(5, q, k, v, o, lse, causal, scale, stream=stream)
    _replay_checked(graph, stream, [t for pair in outs for t in pair], refs)


def test_op_forward_in_graph():
    _require()
    q, k, v = _inputs(2, 4, 256, 64, torch.float16, 7)
    o_ref, lse_ref = fused_attn.forward_stage(q, k, v, 5, is_causal=True)
    torch.cuda.synchronize()
    stream = torch.cuda.Stream()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=stream):
        o, lse = fused_attn.forward_stage(q, k, v, 5, is_causal=True)
    _replay_checked(graph, stream, [o, lse], [o_ref, lse_ref])


def test_decode_in_graph():
    """Split-KV decode with several splits: the split kernel, its workspace (from the graph's
    memory pool) and the combine kernel all replay."""
    _require()
    g = torch.Generator(device="cpu").manual_seed(11)
    q = torch.randn(2, 8, 1, 128, generator=g).to("cuda", torch.bfloat16)
    k = torch.randn(2, 2, 2048, 128, generator=g).to("cuda", torch.bfloat16)
    v = torch.randn(2, 2, 2048, 128, generator=g).to("cuda", torch.bfloat16)
    o_ref, lse_ref = fused_attn.decode(q, k, v, is_causal=True, num_splits=4)
    torch.cuda.synchronize()
    stream = torch.cuda.Stream()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=stream):
        o, lse = fused_attn.decode(q, k, v, is_causal=True, num_splits=4)
    _replay_checked(graph, stream, [o, lse], [o_ref, lse_ref])
