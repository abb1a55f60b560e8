"""Meta kernels of the ``fused_attn`` ops, and an ``opcheck`` driver for them.

A meta ("fake") kernel computes the metadata of an op's outputs -- shape, dtype, device, layout --
from the metadata of its inputs, without reading any data. ``torch.compile``, AOTAutograd and
``FakeTensorMode`` call it in place of the HIP kernel while they trace; without one, tracing stops
at the op (a graph break). The rules below restate what ``csrc/ext.cpp`` allocates and checks:

* ``forward``       -> O shaped and typed like q;
* ``forward_stage`` -> (O, LSE) with LSE fp32 ``[B, H, N]`` for the stages whose kernels produce
  it (3, 4, 5) and an empty ``(0,)`` tensor for stages 1-2, the reference op's contract
  (ref:python/fused_attn/ops.py:28-70, ref:python/fused_attn/ext.cpp:159-188);
* ``forward_strided`` -> O dense in q's memory order;
* ``decode``        -> (O like q, LSE fp32 ``[B, H, Nq]``).

Input rules become ``torch._check`` calls, so under symbolic shapes they turn into guards rather
than failures. The meta kernels are installed once ``fused_attn._C`` has defined the schemas.
"""

from __future__ import annotations

from collections.abc import Sequence

import torch
from torch import Tensor

SUPPORTED_DTYPES = (torch.float32, torch.float16, torch.bfloat16)
SUPPORTED_HEAD_DIMS = (64, 128)
# Stages whose kernels write the row logsumexp; the materialising stages 1-2 return an empty LSE.
LSE_STAGES = (3, 4, 5)

_installed = False


def _rule(ok, message: str) -> None:
    torch._check(ok, lambda: message)


def _attention_contract(q: Tensor, k: Tensor, v: Tensor) -> None:
    """The operand rules of ``forward``, ``forward_stage`` and ``forward_strided`` (layout and
    alignment aside, which fake tensors do not carry); csrc/ext.cpp enforces the same ones, with
    the same wording where a test matches it."""
    _rule(q.dim() == 4 and k.dim() == 4 and v.dim() == 4, "q, k and v must be 4-D [B, H, N, D]")
    _rule(k.dtype == q.dtype and v.dtype == q.dtype, "q, k and v must have the same dtype")
    _rule(q.dtype in SUPPORTED_DTYPES, f"dtype {q.dtype} is not supported")
    batch, heads, n, d = q.shape
    _rule(d == 64 or d == 128, f"D must be 64 or 128 (got {d})")
    _rule(n % 32 == 0, f"N must be a multiple of 32 (got {n})")
    _rule(k.shape[0] == batch and v.shape[0] == batch, "q, k and v must share the batch size")
    _rule(k.shape[2] == n and v.shape[2] == n, "Nq == Nkv is required")
    _rule(k.shape[3] == d and v.shape[3] == d, "q, k and v must share the head dim")
    _rule(k.shape[1] == v.shape[1], "k and v must have the same head count")
    _rule(heads % k.shape[1] == 0, "H must be a multiple of Hkv")


def _meta_forward(q: Tensor, k: Tensor, v: Tensor, is_causal: bool, scale: float) -> Tensor:
    _attention_contract(q, k, v)
    return torch.empty_like(q)


def _meta_forward_stage(q: Tensor, k: Tensor, v: Tensor, is_causal: bool, scale: float,
                        stage: int) -> tuple[Tensor, Tensor]:
    _attention_contract(q, k, v)
    _rule(1 <= stage <= 5, f"stage must be in 1..5 (got {stage})")
    lse_shape = tuple(q.shape[:3]) if stage in LSE_STAGES else (0,)
    return torch.empty_like(q), q.new_empty(lse_shape, dtype=torch.float32)


def empty_in_layout_of(q: Tensor) -> Tensor:
    """A new dense tensor shaped like q whose memory order is q's (dimensions ranked by stride,
    largest first; ties keep their order) -- what ``forward_strided`` allocates for O
    (csrc/ext.cpp ``empty_in_layout_of``). For the [B, H, N, D] view of a [B, N, H, D] buffer it is
    a [B, N, H, D] buffer seen as [B, H, N, D]."""
    by_stride = sorted(range(q.dim()), key=lambda dim: -q.stride(dim))
    storage_order = q.new_empty([q.shape[dim] for dim in by_stride])
    return storage_order.permute([by_stride.index(dim) for dim in range(q.dim())])


def _meta_forward_strided(q: Tensor, k: Tensor, v: Tensor, is_causal: bool,
                          scale: float) -> Tensor:
    _attention_contract(q, k, v)
    return empty_in_layout_of(q)


def _meta_decode(q: Tensor, k: Tensor, v: Tensor, is_causal: bool, scale: float,
                 num_splits: int) -> tuple[Tensor, Tensor]:
    _rule(q.dim() == 4 and k.dim() == 4 and v.dim() == 4,
          "decode takes q [B, H, Nq, D] and k, v [B, Hkv, Nkv, D]")
    _rule(k.dtype == q.dtype and v.dtype == q.dtype, "q, k and v must have the same dtype")
    _rule(k.shape[1] > 0 and q.shape[1] % k.shape[1] == 0, "H must be a multiple of Hkv")
    return torch.empty_like(q), q.new_empty(tuple(q.shape[:3]), dtype=torch.float32)


_META_KERNELS = {
    "fused_attn::forward": _meta_forward,
    "fused_attn::forward_stage": _meta_forward_stage,
    "fused_attn::forward_strided": _meta_forward_strided,
    "fused_attn::decode": _meta_decode,
}


def register_fakes() -> None:
    """Install every meta kernel once (the op schemas must already exist: import ``_C`` first)."""
    global _installed
    if not _installed:
        for name, kernel in _META_KERNELS.items():
            torch.library.register_fake(name, kernel)
        _installed = True


# torch.library.opcheck utilities, and whether each one must see tensor inputs that require grad.
# The autograd-registration check refuses to run without such an input; the AOT-dispatch check
# must not get one, or it would trace a backward for ops that have no autograd formula.
_OPCHECK_UTILS = {
    "test_schema": False,
    "test_faketensor": False,
    "test_aot_dispatch_dynamic": False,
    "test_autograd_registration": True,
}


def _opcheck(op, args: tuple) -> dict[str, str]:
    report: dict[str, str] = {}
    for needs_grad in (False, True):
        utils = tuple(u for u, g in _OPCHECK_UTILS.items() if g is needs_grad)
        call_args = tuple(a.detach().requires_grad_() if needs_grad and isinstance(a, Tensor)
                          else a for a in args)
        report.update(torch.library.opcheck(op, call_args, test_utils=utils))
    return report


def opcheck_all(q: Tensor, k: Tensor, v: Tensor, is_causal: bool = False,
                scale: float | None = None,
                stages: Sequence[int] = ()) -> dict[str, dict[str, str]]:
    """``torch.library.opcheck`` -- schema, meta kernel against the real one, AOT dispatch with
    dynamic shapes, autograd registration -- on ``forward`` and on ``forward_stage`` for every
    stage in ``stages``. Raises on the first failure; returns each op's report."""
    scale = float(q.shape[-1] ** -0.5 if scale is None else scale)
    report = {"forward": _opcheck(torch.ops.fused_attn.forward, (q, k, v, is_causal, scale))}
    for stage in stages:
        report[f"forward_stage[{stage}]"] = _opcheck(
            torch.ops.fused_attn.forward_stage, (q, k, v, is_causal, scale, int(stage)))
    return report
