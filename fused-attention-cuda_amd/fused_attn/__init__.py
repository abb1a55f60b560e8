"""fused_attn -- MI355X-native fused SDPA forward behind the reference's ``torch.ops.fused_attn`` API.

Same public surface as the reference package (ref:python/fused_attn/__init__.py:1-119):
``forward``, ``forward_stage``, ``impl_supports``, ``impl_name``, ``set_debug_overrides``,
``is_available`` and the ``ops`` module with the fake kernels. The ops are registered by the
compiled binding ``_C`` (csrc/ext.cpp), which calls the gfx950 kernels through the C-ABI of
``libfa_hip.so`` (include/fa/attention.h); :mod:`fused_attn.capi` binds that C-ABI with ctypes.

Import always succeeds; calling an op without the compiled extension raises ``ImportError`` with
the build command -- there is no CPU or eager fallback.

Build (from the repo root)::

    python fused-attention-cuda_amd/build.py

Ops (schemas as in the reference, ref:python/fused_attn/ext.cpp:220-230)::

    torch.ops.fused_attn.forward(q, k, v, is_causal, scale) -> Tensor
    torch.ops.fused_attn.forward_stage(q, k, v, is_causal, scale, stage) -> (Tensor, Tensor)

plus two extensions with no counterpart in the reference:
``torch.ops.fused_attn.forward_strided(q, k, v, is_causal, scale) -> Tensor`` over strided views,
and ``torch.ops.fused_attn.decode(q, k, v, is_causal, scale, num_splits) -> (Tensor, Tensor)``,
split-KV decode of Nq new tokens against Nkv cached keys (the reference's stated next step).
"""

from __future__ import annotations

import math

import torch
from torch import Tensor

from . import ops

__all__ = [
    "__version__",
    "decode",
    "forward",
    "forward_stage",
    "forward_strided",
    "impl_name",
    "impl_supports",
    "is_available",
    "ops",
    "set_debug_overrides",
]
__version__ = "0.1.0"

_EXT_ERROR: ImportError | None
try:
    from . import _C  # noqa: F401  (loading the .so runs the TORCH_LIBRARY static initialisers)
except ImportError as exc:  # pragma: no cover - depends on the machine
    _EXT_ERROR = exc
else:
    _EXT_ERROR = None
    ops.register_fakes()

_BUILD_HINT = (
    "fused_attn._C is not built. From the repo root run\n"
    "  python fused-attention-cuda_amd/build.py\n"
    "(needs hipcc from ROCm and a ROCm build of PyTorch; the kernels target gfx950 / MI355X)."
)

_DTYPE_NAMES = {torch.float32: "fp32", torch.float16: "fp16", torch.bfloat16: "bf16"}


def is_available() -> bool:
    """True when the compiled extension imported."""
    return _EXT_ERROR is None


def _require_ext() -> None:
    if _EXT_ERROR is not None:
        raise ImportError(_BUILD_HINT) from _EXT_ERROR


def _resolve_scale(q: Tensor, scale: float | None) -> float:
    # PyTorch's SDPA default; the one place the default is decided.
    return float(1.0 / math.sqrt(q.shape[-1]) if scale is None else scale)


def forward(q: Tensor, k: Tensor, v: Tensor, is_causal: bool = False,
            scale: float | None = None) -> Tensor:
    """Fused attention forward, dispatched to the best implemented stage for (dtype, D, GPU)."""
    _require_ext()
    return torch.ops.fused_attn.forward(q, k, v, bool(is_causal), _resolve_scale(q, scale))


def forward_stage(q: Tensor, k: Tensor, v: Tensor, stage: int, is_causal: bool = False,
                  scale: float | None = None) -> tuple[Tensor, Tensor]:
    """Run one explicit stage (1..5). Returns ``(o, lse)``; ``lse`` is empty for stages 1-2."""
    _require_ext()
    return torch.ops.fused_attn.forward_stage(q, k, v, bool(is_causal),
                                              _resolve_scale(q, scale), int(stage))


def forward_strided(q: Tensor, k: Tensor, v: Tensor, is_causal: bool = False,
                    scale: float | None = None) -> Tensor:
    """``forward`` over strided [B, H, N, D] views (head dim contiguous, batch/head/row strides
    multiples of 16 bytes), e.g. ``qkv.view(B, N, 3, H, D)[:, :, 0].transpose(1, 2)`` with no copy.
    The output is dense in q's memory order (see ``ops.empty_in_layout_of``). An extension of the
    reference op surface, which only takes contiguous tensors."""
    _require_ext()
    return torch.ops.fused_attn.forward_strided(q, k, v, bool(is_causal), _resolve_scale(q, scale))


def decode(q: Tensor, k: Tensor, v: Tensor, is_causal: bool = False, scale: float | None = None,
           num_splits: int = 0) -> tuple[Tensor, Tensor]:
    """Split-KV decode: q [B, H, Nq, D] (the Nq newest tokens) against the cache k, v
    [B, Hkv, Nkv, D] -> (o [B, H, Nq, D], lse [B, H, Nq]). With ``is_causal`` token i sees keys
    j <= Nkv - Nq + i (bottom-right alignment). ``num_splits`` = 0 lets the library choose how
    many pieces of the key range run in parallel; the pieces are combined with LSE weights.
    fp16/bf16, D 64 or 128, (H / Hkv) * Nq <= 64."""
    _require_ext()
    return torch.ops.fused_attn.decode(q, k, v, bool(is_causal), _resolve_scale(q, scale),
                                       int(num_splits))


def impl_supports(stage: int, dtype: torch.dtype, head_dim: int) -> bool:
    """Whether this build can run ``stage`` for (dtype, D) on the *current* device."""
    _require_ext()
    name = _DTYPE_NAMES.get(dtype)
    if name is None:
        return False
    return bool(torch.ops.fused_attn.impl_supports(int(stage), name, int(head_dim)))


def impl_name(stage: int) -> str:
    """ "naive" / "tiled" / "fused" / "wmma" / "tuned" (the reference's stage names)."""
    _require_ext()
    return str(torch.ops.fused_attn.impl_name(int(stage)))


def set_debug_overrides(block_m: int = 0, block_n: int = 0) -> None:
    """TEST-ONLY: force the query-tile height (BR) and key-tile width (BC); 0 = default.

    Global, process-wide, not thread-safe by design -- always reset to ``(0, 0)`` afterwards."""
    _require_ext()
    torch.ops.fused_attn.set_debug_overrides(int(block_m), int(block_n))
