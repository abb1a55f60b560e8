"""Fake (meta) kernels and the opcheck helper for the ``fused_attn::*`` ops.

``torch.compile`` / AOTAutograd trace ops on fake tensors that carry only shape, dtype and device.
The fakes below describe the outputs of both ops without touching data, which is what keeps
``torch.compile(fullgraph=True)`` free of graph breaks. Behaviour follows the reference's fakes
(ref:python/fused_attn/ops.py:28-70): the same ``torch._check`` mirrors of the C++ input checks,
``o = empty_like(q)`` and an fp32 ``lse`` of ``[B, H, N]`` for stages 3-5 (``(0,)`` otherwise).
The fakes are registered after ``fused_attn._C`` is loaded (the schemas live in C++).
"""

from __future__ import annotations

from collections.abc import Sequence

import torch
from torch import Tensor

SUPPORTED_DTYPES = (torch.float32, torch.float16, torch.bfloat16)
SUPPORTED_HEAD_DIMS = (64, 128)
# Stages whose kernels write the logsumexp.
LSE_STAGES = (3, 4, 5)

_registered = False


def _check_inputs(q: Tensor, k: Tensor, v: Tensor) -> None:
    """``torch._check`` mirror of the TORCH_CHECKs in csrc/ext.cpp (each becomes a guard or a
    runtime assert under symbolic shapes)."""
    torch._check(q.dim() == 4 and k.dim() == 4 and v.dim() == 4, lambda: "q/k/v must be [B,H,N,D]")
    torch._check(q.dtype == k.dtype and q.dtype == v.dtype, lambda: "q/k/v must share one dtype")
    torch._check(q.dtype in SUPPORTED_DTYPES, lambda: f"unsupported dtype {q.dtype}")
    b, h, n, d = q.shape
    torch._check(d == 64 or d == 128, lambda: f"D must be 64 or 128, got {d}")
    torch._check(n % 32 == 0, lambda: f"N must be a multiple of 32, got {n}")
    torch._check(k.shape[0] == b and v.shape[0] == b, lambda: "batch mismatch")
    torch._check(k.shape[2] == n and v.shape[2] == n, lambda: "Nq == Nkv is required")
    torch._check(k.shape[3] == d and v.shape[3] == d, lambda: "head-dim mismatch")
    torch._check(k.shape[1] == v.shape[1], lambda: "k and v must have the same number of heads")
    torch._check(h % k.shape[1] == 0, lambda: "H must be a multiple of Hkv")


def _fake_forward(q: Tensor, k: Tensor, v: Tensor, is_causal: bool, scale: float) -> Tensor:
    _check_inputs(q, k, v)
    return torch.empty_like(q)


def _fake_forward_stage(q: Tensor, k: Tensor, v: Tensor, is_causal: bool, scale: float,
                        stage: int) -> tuple[Tensor, Tensor]:
    _check_inputs(q, k, v)
    torch._check(1 <= stage <= 5, lambda: f"stage must be in 1..5, got {stage}")
    b, h, n, _ = q.shape
    o = torch.empty_like(q)
    if stage in LSE_STAGES:
        lse = q.new_empty((b, h, n), dtype=torch.float32)
    else:
        lse = q.new_empty((0,), dtype=torch.float32)
    return o, lse


def empty_in_layout_of(q: Tensor) -> Tensor:
    """A dense tensor of q's shape whose memory order follows q's strides (outermost first) --
    the output layout of ``forward_strided`` (csrc/ext.cpp ``empty_in_layout_of``): for the
    [B, H, N, D] view of a [B, N, H, D] buffer it is a [B, N, H, D] buffer seen as [B, H, N, D]."""
    order = sorted(range(4), key=lambda d: -q.stride(d))  # stable: ties keep dimension order
    out = q.new_empty([q.shape[d] for d in order])
    inverse = [order.index(d) for d in range(4)]
    return out.permute(inverse)


def _fake_forward_strided(q: Tensor, k: Tensor, v: Tensor, is_causal: bool, scale: float) -> Tensor:
    torch._check(q.dim() == 4 and k.dim() == 4 and v.dim() == 4, lambda: "q/k/v must be [B,H,N,D]")
    b, h, n, d = q.shape
    torch._check(d == 64 or d == 128, lambda: f"D must be 64 or 128, got {d}")
    torch._check(n % 32 == 0, lambda: f"N must be a multiple of 32, got {n}")
    torch._check(q.dtype == k.dtype and q.dtype == v.dtype, lambda: "q/k/v must share one dtype")
    return empty_in_layout_of(q)


def _fake_decode(q: Tensor, k: Tensor, v: Tensor, is_causal: bool, scale: float,
                 num_splits: int) -> tuple[Tensor, Tensor]:
    torch._check(q.dim() == 4 and k.dim() == 4 and v.dim() == 4,
                 lambda: "decode expects q [B, H, Nq, D] and k, v [B, Hkv, Nkv, D]")
    b, h, nq, d = q.shape
    torch._check(q.dtype == k.dtype and q.dtype == v.dtype, lambda: "q/k/v must share one dtype")
    torch._check(k.shape[1] > 0 and h % k.shape[1] == 0, lambda: "H must be a multiple of Hkv")
    return torch.empty_like(q), q.new_empty((b, h, nq), dtype=torch.float32)


def register_fakes() -> None:
    """Register the fake kernels (idempotent; requires ``fused_attn._C`` to be loaded)."""
    global _registered
    if _registered:
        return
    torch.library.register_fake("fused_attn::forward", _fake_forward)
    torch.library.register_fake("fused_attn::forward_stage", _fake_forward_stage)
    torch.library.register_fake("fused_attn::forward_strided", _fake_forward_strided)
    torch.library.register_fake("fused_attn::decode", _fake_decode)
    _registered = True


# opcheck runs in two groups (ref:python/fused_attn/ops.py:73-96): the autograd-registration check
# needs an input with requires_grad=True, while the others must see plain inputs (with grad-
# requiring inputs the AOT check would trace a backward for an op that has no autograd kernel).
_NO_GRAD_TESTS = ("test_schema", "test_faketensor", "test_aot_dispatch_dynamic")
_GRAD_TESTS = ("test_autograd_registration",)


def _opcheck(op, args: tuple) -> dict[str, str]:
    q, k, v, *rest = args
    res = dict(torch.library.opcheck(op, (q, k, v, *rest), test_utils=_NO_GRAD_TESTS))
    grad_args = (q.detach().requires_grad_(), k.detach().requires_grad_(),
                 v.detach().requires_grad_(), *rest)
    res.update(torch.library.opcheck(op, grad_args, test_utils=_GRAD_TESTS))
    return res


def opcheck_all(q: Tensor, k: Tensor, v: Tensor, is_causal: bool = False,
                scale: float | None = None,
                stages: Sequence[int] = ()) -> dict[str, dict[str, str]]:
    """``torch.library.opcheck`` on ``forward`` and on ``forward_stage`` for each stage
    (schema, fake vs real, AOT dispatch with dynamic shapes, autograd registration)."""
    if scale is None:
        scale = 1.0 / (q.shape[-1] ** 0.5)
    results: dict[str, dict[str, str]] = {}
    results["forward"] = _opcheck(torch.ops.fused_attn.forward, (q, k, v, is_causal, float(scale)))
    for stage in stages:
        results[f"forward_stage[{stage}]"] = _opcheck(
            torch.ops.fused_attn.forward_stage, (q, k, v, is_causal, float(scale), int(stage)))
    return results
