"""fa_decode_noalloc, the allocation-free decode entry point, against fa_decode.

fa_decode_noalloc runs the same split and combine kernels as fa_decode, with the splits' partials
in the library's per-GPU scratch array instead of a caller workspace, so its output must equal
fa_decode's bit for bit (fa_decode itself is tied to the fp64 decode oracle in
tests/test_decode_gpu.py). Two calls in a row, the second on a smaller problem, check that the
array's leftover contents from the first call never leak into the second. Sizes past the array
are refused before any launch. Everything goes through the C-ABI (ctypes).
"""

from __future__ import annotations

import pytest
import torch

from fused_attn import capi

pytestmark = pytest.mark.gpu


def _inputs(b, h, hkv, nq, nkv, d, dtype, seed):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(b, h, nq, d, generator=g).to("cuda", dtype)
    k = torch.randn(b, hkv, nkv, d, generator=g).to("cuda", dtype)
    v = torch.randn(b, hkv, nkv, d, generator=g).to("cuda", dtype)
    return q, k, v


def _outputs(q):
    b, h, nq, _ = q.shape
    o = torch.full_like(q, float("nan"))
    lse = torch.full((b, h, nq), float("nan"), dtype=torch.float32, device=q.device)
    return o, lse


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16], ids=["fp16", "bf16"])
def test_noalloc_matches_decode_on_consecutive_calls(dtype):
    # (B, H, Hkv, Nq, Nkv, D, causal): a GQA problem the library splits many ways (R = 16 rows per
    # kv head), then a smaller MHA problem at the other head dim that still splits, so the second
    # call reads a scratch array still holding the first call's partials.
    shapes = [(2, 32, 8, 4, 8192 + 77, 128, True), (1, 4, 4, 1, 3000, 64, False)]
    for i, (b, h, hkv, nq, nkv, d, causal) in enumerate(shapes):
        q, k, v = _inputs(b, h, hkv, nq, nkv, d, dtype, seed=40 + i)
        scale = d ** -0.5
        p = capi.decode_params(q, k, causal, scale)
        splits = capi.load().fa_decode_num_splits(p)
        assert splits > 1, "the shape must exercise the scratch array (more than one split)"
        o_ref, lse_ref = _outputs(q)
        rc = capi.decode(q, k, v, o_ref, lse_ref, causal, scale)
        assert rc == capi.HIP_SUCCESS, capi.error_string(rc)
        o, lse = _outputs(q)
        rc = capi.decode_noalloc(q, k, v, o, lse, causal, scale)
        assert rc == capi.HIP_SUCCESS, capi.error_string(rc)
        torch.cuda.synchronize()
        assert torch.isfinite(o).all() and torch.isfinite(lse).all()
        assert torch.equal(o, o_ref), f"call {i} ({splits} splits): O differs from fa_decode"
        assert torch.equal(lse, lse_ref), f"call {i} ({splits} splits): LSE differs from fa_decode"


def test_noalloc_refuses_partials_larger_than_the_scratch():
    # 64 forced splits x 64 rows per kv head x 16 kv heads x (128 + 1) fp32 = 33.8 MB > 16 MiB.
    b, h, hkv, nq, nkv, d = 2, 128, 8, 4, 64 * 128, 128
    q, k, v = _inputs(b, h, hkv, nq, nkv, d, torch.float16, seed=50)
    p = capi.decode_params(q, k, True, d ** -0.5, num_splits=64)
    need = capi.load().fa_decode_workspace_bytes(capi.FA_DTYPE_F16, p)
    assert need > capi.DECODE_SCRATCH_BYTES
    o, lse = _outputs(q)
    rc = capi.decode_noalloc(q, k, v, o, lse, True, d ** -0.5, num_splits=64)
    assert rc == capi.HIP_ERROR_INVALID_VALUE
    torch.cuda.synchronize()
    assert torch.isnan(o).all() and torch.isnan(lse).all(), "a refused call must write nothing"


def test_noalloc_without_split_needs_no_scratch():
    # One split: the split kernel writes o and lse directly; the scratch array is not touched.
    q, k, v = _inputs(1, 2, 2, 1, 200, 64, torch.float16, seed=51)
    p = capi.decode_params(q, k, False, 0.125)
    assert capi.load().fa_decode_num_splits(p) == 1
    o_ref, lse_ref = _outputs(q)
    assert capi.decode(q, k, v, o_ref, lse_ref, False, 0.125) == capi.HIP_SUCCESS
    o, lse = _outputs(q)
    assert capi.decode_noalloc(q, k, v, o, lse, False, 0.125) == capi.HIP_SUCCESS
    torch.cuda.synchronize()
    assert torch.equal(o, o_ref) and torch.equal(lse, lse_ref)


def test_noalloc_replays_from_a_captured_graph():
    """The entry point's purpose: a caller that captures the decode into a HIP graph. The first
    call on the device runs outside the capture (it resolves the scratch array's address); the
    captured call is then replayed twice, with the outputs cleared by eager work in between, and
    each replay must equal fa_decode bit for bit."""
    b, h, hkv, nq, nkv, d = 2, 16, 4, 2, 4096 + 40, 128
    q, k, v = _inputs(b, h, hkv, nq, nkv, d, torch.bfloat16, seed=52)
    scale = d ** -0.5
    assert capi.load().fa_decode_num_splits(capi.decode_params(q, k, True, scale)) > 1
    o_ref, lse_ref = _outputs(q)
    assert capi.decode(q, k, v, o_ref, lse_ref, True, scale) == capi.HIP_SUCCESS
    o, lse = _outputs(q)
    stream = torch.cuda.Stream()
    with torch.cuda.stream(stream):
        assert capi.decode_noalloc(q, k, v, o, lse, True, scale, stream=stream) == capi.HIP_SUCCESS
    stream.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=stream):
        rc = capi.decode_noalloc(q, k, v, o, lse, True, scale, stream=stream)
    assert rc == capi.HIP_SUCCESS, capi.error_string(rc)
    for replay in range(2):
        o.fill_(float("nan"))
        lse.fill_(float("nan"))
        torch.cuda.synchronize()
        with torch.cuda.stream(stream):
            graph.replay()
        stream.synchronize()
        assert torch.equal(o, o_ref) and torch.equal(lse, lse_ref), f"replay {replay}"
