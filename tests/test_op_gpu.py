"""The fused_attn operators as PyTorch custom operators (marker ``gpu``).

Properties a torch.compile user relies on, the ones the reference's operator tests check
(ref:tests/test_op_gpu.py): ``torch.library.opcheck`` passes for ``forward`` and every built
``forward_stage``; the meta kernels produce the right output metadata in FakeTensorMode without a
launch and refuse what the operator refuses; a compiled function around the operator traces as
one graph and reproduces eager execution bit for bit; ``forward_stage`` compiles with a dynamic N;
the Python wrapper is the raw operator. The two extension operators (``forward_strided``,
``decode``) get the same meta-kernel and graph checks.
"""

from __future__ import annotations

import pytest
import torch
from torch._subclasses.fake_tensor import FakeTensorMode

import fused_attn
from fused_attn.ops import LSE_STAGES, opcheck_all

pytestmark = pytest.mark.gpu

ALL_STAGES = (1, 2, 3, 4, 5)
DTYPE_IDS = {torch.float32: "fp32", torch.float16: "fp16", torch.bfloat16: "bf16"}


def built_stages(dtype: torch.dtype, head_dim: int = 64) -> list[int]:
    """The stages built for (dtype, head_dim) on this device; skips the test when there is none."""
    assert fused_attn.is_available(), "fused_attn._C must be built for the GPU tests"
    stages = [st for st in ALL_STAGES if fused_attn.impl_supports(st, dtype, head_dim)]
    if not stages:
        pytest.skip(f"no stage built for {DTYPE_IDS[dtype]} D={head_dim}")
    return stages


def count_graphs(fn, *args):
    """(graphs, breaks) dynamo produces for fn(*args), from a fresh compiler state."""
    torch.compiler.reset()
    report = torch._dynamo.explain(fn)(*args)
    return report.graph_count, report.graph_break_count


@pytest.mark.parametrize("causal", [False, True], ids=["full", "causal"])
@pytest.mark.parametrize("dtype", list(DTYPE_IDS), ids=list(DTYPE_IDS.values()))
def test_opcheck(dtype, causal, make_qkv):
    stages = built_stages(dtype)
    q, k, v = make_qkv(1, 2, 64, 64, dtype=dtype, device="cuda")
    report = opcheck_all(q, k, v, is_causal=causal, stages=stages)
    assert sorted(report) == sorted(["forward", *[f"forward_stage[{st}]" for st in stages]])
    failed = {op: r for op, r in report.items() if set(r.values()) - {"SUCCESS", "SKIPPED"}}
    assert not failed, failed


def test_meta_kernels_in_fake_mode():
    built_stages(torch.float16)
    with FakeTensorMode():
        q = torch.empty(2, 4, 256, 64, dtype=torch.float16, device="cuda")
        kv = torch.empty(2, 2, 256, 64, dtype=torch.float16, device="cuda")  # GQA 2:1
        o = torch.ops.fused_attn.forward(q, kv, kv, False, 0.125)
        assert (o.shape, o.dtype, o.device.type) == (q.shape, q.dtype, "cuda")
        for st in ALL_STAGES:
            o, lse = torch.ops.fused_attn.forward_stage(q, kv, kv, True, 0.125, st)
            assert o.shape == q.shape and o.dtype == q.dtype
            assert lse.dtype == torch.float32
            assert tuple(lse.shape) == ((2, 4, 256) if st in LSE_STAGES else (0,))
        # [B, H, N, D] views of a [B, N, H, D] buffer: O comes back in that memory order.
        qs = torch.empty(2, 256, 4, 64, dtype=torch.float16, device="cuda").transpose(1, 2)
        o = torch.ops.fused_attn.forward_strided(qs, qs, qs, True, 0.125)
        assert o.shape == qs.shape and o.stride() == qs.stride()
        qd = torch.empty(3, 8, 2, 128, dtype=torch.bfloat16, device="cuda")
        cache = torch.empty(3, 2, 1000, 128, dtype=torch.bfloat16, device="cuda")
        o, lse = torch.ops.fused_attn.decode(qd, cache, cache, True, 0.1, 0)
        assert o.shape == qd.shape and tuple(lse.shape) == (3, 8, 2) and lse.dtype == torch.float32
        ragged = torch.empty(2, 4, 100, 64, dtype=torch.float16, device="cuda")
        with pytest.raises(RuntimeError, match="multiple of 32"):
            torch.ops.fused_attn.forward(ragged, ragged, ragged, False, 0.125)


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16], ids=["fp32", "fp16"])
def test_compiled_graph_has_no_break(dtype, make_qkv):
    built_stages(dtype)
    q, k, v = make_qkv(1, 2, 128, 64, dtype=dtype, device="cuda")

    def around_the_op(q, k, v):
        # Work on both sides of the operator: a break would split this into several graphs.
        o = torch.ops.fused_attn.forward(q * 1.0, k, v, True, 0.125)
        return o * 2.0

    assert count_graphs(around_the_op, q, k, v) == (1, 0)
    torch.compiler.reset()
    compiled = torch.compile(around_the_op, fullgraph=True)  # raises on any break
    assert torch.equal(compiled(q, k, v), around_the_op(q, k, v))


def test_compiled_extension_ops_have_no_break():
    built_stages(torch.float16)
    gen = torch.Generator().manual_seed(21)
    qkv = torch.randn(2, 128, 3, 4, 64, generator=gen).to("cuda", torch.float16)
    q_new = torch.randn(2, 8, 1, 64, generator=gen).to("cuda", torch.float16)
    cache = torch.randn(2, 4, 300, 64, generator=gen).to("cuda", torch.float16)

    def block_attention(qkv):  # the head split of a fused projection, read in place
        q, k, v = (qkv[:, :, i].transpose(1, 2) for i in range(3))
        return torch.ops.fused_attn.forward_strided(q, k, v, True, 0.125).transpose(1, 2) + 0.0

    def decode_step(q_new, cache):
        o, lse = torch.ops.fused_attn.decode(q_new, cache, cache, True, 0.125, 0)
        return o * 2.0, lse + 1.0  # exact elementwise work, so compiled == eager bit for bit

    for fn, args in ((block_attention, (qkv,)), (decode_step, (q_new, cache))):
        assert count_graphs(fn, *args) == (1, 0), fn.__name__
        torch.compiler.reset()
        got, want = torch.compile(fn, fullgraph=True)(*args), fn(*args)
        for g, w in zip(got if isinstance(got, tuple) else (got,),
                        want if isinstance(want, tuple) else (want,)):
            assert torch.equal(g, w), fn.__name__


def test_forward_stage_compiles_with_dynamic_n(make_qkv):
    stage = max(built_stages(torch.float32))

    def row_sums(q, k, v):
        o, lse = torch.ops.fused_attn.forward_stage(q, k, v, False, 0.125, stage)
        return o.sum(-1), lse

    torch.compiler.reset()
    compiled = torch.compile(row_sums, fullgraph=True, dynamic=True)
    for n in (128, 256):  # N % 32 == 0 must become a guard on the symbolic N, not a break
        q, k, v = make_qkv(1, 2, n, 64, dtype=torch.float32, device="cuda")
        (got_sum, got_lse), (want_sum, want_lse) = compiled(q, k, v), row_sums(q, k, v)
        torch.testing.assert_close(got_sum, want_sum, atol=1e-4, rtol=1e-5)
        assert got_lse.shape == want_lse.shape == (1, 2, n)


def test_wrapper_is_the_raw_op(make_qkv):
    built_stages(torch.float32)
    q, k, v = make_qkv(1, 2, 64, 64, dtype=torch.float32, device="cuda")
    assert torch.equal(fused_attn.forward(q, k, v, is_causal=True),
                       torch.ops.fused_attn.forward(q, k, v, True, 64 ** -0.5))
    assert [fused_attn.impl_name(st) for st in ALL_STAGES] == \
        ["naive", "tiled", "fused", "wmma", "tuned"]
