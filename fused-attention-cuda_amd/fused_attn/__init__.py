"""fused_attn: the ``torch.ops.fused_attn`` operators, backed by gfx950 (MI355X) HIP kernels.

The public names and signatures are the reference package's (ref:python/fused_attn/__init__.py:
1-119): ``forward``, ``forward_stage``, ``impl_supports``, ``impl_name``, ``set_debug_overrides``,
``is_available`` and the ``ops`` module. Two operators extend that surface: ``forward_strided``
(strided [B, H, N, D] views, no copies) and ``decode`` (split-KV decode).

Layers: the compiled module ``_C`` (csrc/ext.cpp) defines the operators with the reference's
schemas and calls ``libfa_hip.so`` through its C-ABI (include/fa/attention.h); :mod:`.ops` holds
their meta kernels; :mod:`.capi` binds the C-ABI directly with ctypes.

Importing this package never fails. If ``_C`` did not load, every operator call raises
``ImportError`` naming the build command; nothing falls back to another implementation.
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


class _Binding:
    """The compiled operator library, or why it is missing."""

    BUILD_COMMAND = "python fused-attention-cuda_amd/build.py"

    def __init__(self) -> None:
        self.missing: ImportError | None = None
        try:
            # Loading the shared object runs its TORCH_LIBRARY registration.
            from . import _C  # noqa: F401
        except ImportError as exc:  # pragma: no cover - depends on the build
            self.missing = exc
        else:
            ops.register_fakes()

    def library(self):
        """``torch.ops.fused_attn``, or ImportError with the build instructions."""
        if self.missing is not None:
            raise ImportError(
                "the fused_attn HIP extension (fused_attn/_C.so) is not built; build it from the "
                f"repository root with `{self.BUILD_COMMAND}` (hipcc from ROCm, a ROCm build of "
                "PyTorch; the kernels are compiled for gfx950)") from self.missing
        return torch.ops.fused_attn


_BINDING = _Binding()
_DTYPE_TAGS = {torch.float32: "fp32", torch.float16: "fp16", torch.bfloat16: "bf16"}


def is_available() -> bool:
    """Whether the compiled extension loaded."""
    return _BINDING.missing is None


def _softmax_scale(q: Tensor, scale: float | None) -> float:
    """The scale the operators get: the caller's, else 1/sqrt(D) as in torch's SDPA. The
    operators themselves have no default, so this is the only place one is chosen."""
    return 1.0 / math.sqrt(q.shape[-1]) if scale is None else float(scale)


def forward(q: Tensor, k: Tensor, v: Tensor, is_causal: bool = False,
            scale: float | None = None) -> Tensor:
    """softmax(scale * q k^T) v for q [B, H, N, D] and k, v [B, Hkv, N, D] (top-left causal mask
    when ``is_causal``), on the highest stage built for (dtype, D) on this GPU."""
    return _BINDING.library().forward(q, k, v, bool(is_causal), _softmax_scale(q, scale))


def forward_stage(q: Tensor, k: Tensor, v: Tensor, stage: int, is_causal: bool = False,
                  scale: float | None = None) -> tuple[Tensor, Tensor]:
    """The forward on one named stage (1..5), returning (O, LSE); LSE is fp32 [B, H, N] (the row
    log-sum-exp, natural log) for stages 3-5 and empty for the materialising stages 1-2."""
    return _BINDING.library().forward_stage(q, k, v, bool(is_causal), _softmax_scale(q, scale),
                                            int(stage))


def forward_strided(q: Tensor, k: Tensor, v: Tensor, is_causal: bool = False,
                    scale: float | None = None) -> Tensor:
    """``forward`` on strided [B, H, N, D] views -- the head dim contiguous, every other stride a
    multiple of 16 bytes -- such as ``qkv.view(B, N, 3, H, D)[:, :, 0].transpose(1, 2)``, read in
    place. O comes back dense in q's memory order (``ops.empty_in_layout_of``)."""
    return _BINDING.library().forward_strided(q, k, v, bool(is_causal), _softmax_scale(q, scale))


def decode(q: Tensor, k: Tensor, v: Tensor, is_causal: bool = False, scale: float | None = None,
           num_splits: int = 0) -> tuple[Tensor, Tensor]:
    """Split-KV decode: the Nq newest tokens q [B, H, Nq, D] against the cache k, v
    [B, Hkv, Nkv, D], returning (O [B, H, Nq, D], LSE [B, H, Nq]). ``is_causal`` aligns the mask
    bottom-right (token i sees keys j <= Nkv - Nq + i). The key range runs in ``num_splits``
    parallel pieces merged by their LSE (0: the library chooses). fp16 / bf16, D 64 or 128,
    (H / Hkv) * Nq <= 64."""
    return _BINDING.library().decode(q, k, v, bool(is_causal), _softmax_scale(q, scale),
                                     int(num_splits))


def impl_supports(stage: int, dtype: torch.dtype, head_dim: int) -> bool:
    """Whether ``stage`` is built for (dtype, head_dim) on the current device."""
    library = _BINDING.library()
    tag = _DTYPE_TAGS.get(dtype)
    return tag is not None and bool(library.impl_supports(int(stage), tag, int(head_dim)))


def impl_name(stage: int) -> str:
    """The stage's name in the reference ladder: naive, tiled, fused, wmma or tuned."""
    return str(_BINDING.library().impl_name(int(stage)))


def set_debug_overrides(block_m: int = 0, block_n: int = 0) -> None:
    """For tests only: force the query-tile height (block_m, BR) and key-tile width (block_n, BC)
    of the fused stages; 0 restores the default. The setting is process-wide and not
    thread-safe; reset it to (0, 0) when done."""
    _BINDING.library().set_debug_overrides(int(block_m), int(block_n))
