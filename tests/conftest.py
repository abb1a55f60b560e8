"""Shared pytest configuration (the roles of ref:tests/conftest.py).

* Puts the repo root (for ``oracle``) and ``fused-attention-cuda_amd`` (for ``fused_attn``) on
  ``sys.path`` so a clean checkout needs no install.
* ``gpu`` marker: needs a HIP device; auto-skipped when ``torch.cuda.is_available()`` is False.
* ``--stage N``: restrict stage-parametrised GPU tests to one stage.
* ``make_qkv``: seeded inputs exactly as the reference's fixture (ref:tests/conftest.py:99-127).
"""

from __future__ import annotations

import sys
from collections.abc import Callable
from pathlib import Path

import pytest
import torch

ROOT = Path(__file__).resolve().parents[1]
PKG_DIR = ROOT / "fused-attention-cuda_amd"
for p in (ROOT, PKG_DIR):
    if str(p) not in sys.path:
        sys.path.insert(0, str(p))

STAGES = (1, 2, 3, 4, 5)


def pytest_addoption(parser: pytest.Parser) -> None:
    parser.addoption("--stage", action="store", default="all",
                     help="keep only this stage (1..5) of the stage-parametrised tests")


def pytest_configure(config: pytest.Config) -> None:
    config.addinivalue_line(
        "markers", "gpu: needs a HIP device; skipped where torch.cuda.is_available() is False")


def _stage_of(item: pytest.Item):
    """The ``stage`` parameter of a parametrised test item, or None."""
    callspec = getattr(item, "callspec", None)
    return None if callspec is None else callspec.params.get("stage")


def pytest_collection_modifyitems(config: pytest.Config, items: list[pytest.Item]) -> None:
    """Two adjustments: GPU tests are marked skipped on a machine without a HIP device, and
    ``--stage N`` deselects the stage-parametrised items of the other stages."""
    if not torch.cuda.is_available():
        no_device = pytest.mark.skip(reason="no HIP device (torch.cuda.is_available() is False)")
        for item in items:
            if item.get_closest_marker("gpu") is not None:
                item.add_marker(no_device)
    option = config.getoption("--stage")
    if option in (None, "all"):
        return
    stage = int(option)
    dropped = [it for it in items if _stage_of(it) not in (None, stage)]
    if dropped:
        config.hook.pytest_deselected(items=dropped)
        items[:] = [it for it in items if _stage_of(it) in (None, stage)]


# (B, H, N, D) shapes for the GPU parity tests: the reference's GPU_SHAPES
# (ref:tests/conftest.py:74-80), all small enough for the fp64 oracle to finish in seconds.
GPU_SHAPES = [(1, 1, 64, 64), (2, 4, 256, 64), (1, 2, 512, 128), (2, 2, 1024, 64),
              (1, 2, 2048, 64)]


def shape_id(shape: tuple[int, int, int, int]) -> str:
    b, h, n, d = shape
    return f"B{b}_H{h}_N{n}_D{d}"


@pytest.fixture(params=GPU_SHAPES, ids=shape_id)
def gpu_shape(request: pytest.FixtureRequest) -> tuple[int, int, int, int]:
    return request.param


def make_qkv_impl(b: int, h: int, n: int, d: int, dtype: torch.dtype = torch.float32,
                  device: str | torch.device = "cpu", hkv: int | None = None, seed: int = 0,
                  scale_inputs: float = 1.0):
    """CPU generator seeded once, fp32 randn for q, k, v in that order, then scale, cast, move."""
    gen = torch.Generator(device="cpu").manual_seed(seed)
    hkv = h if hkv is None else hkv
    q = torch.randn(b, h, n, d, generator=gen, dtype=torch.float32)
    k = torch.randn(b, hkv, n, d, generator=gen, dtype=torch.float32)
    v = torch.randn(b, hkv, n, d, generator=gen, dtype=torch.float32)
    return tuple((t * scale_inputs).to(device=device, dtype=dtype).contiguous() for t in (q, k, v))


@pytest.fixture
def make_qkv() -> Callable[..., tuple[torch.Tensor, torch.Tensor, torch.Tensor]]:
    return make_qkv_impl
