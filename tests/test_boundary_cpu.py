"""CPU tests of the drop-in boundary: libfa_hip.so and the torch binding, without a GPU.

* The C-ABI library loads and exports exactly the functions include/fa/attention.h declares.
* Host logic that runs before any device call: parameter validation (hipErrorInvalidValue),
  the stage registry (impl_supports / names / workspace sizes, ref:src/dispatch.cu:56-175) and the
  debug-override state with its environment layering (ref:src/dispatch.cu:177-189).
* The torch op schemas are the reference's verbatim (ref:python/fused_attn/ext.cpp:220-230) and the
  fake kernels give the reference's output metadata (ref:python/fused_attn/ops.py:44-60).
* The product never reaches the oracle: no product source names it.
No test here launches a kernel.
"""

from __future__ import annotations

import ctypes
import re
import subprocess
from pathlib import Path

import pytest
import torch

from fused_attn import capi

ROOT = Path(__file__).resolve().parents[1]
HEADER = ROOT / "include" / "fa" / "attention.h"
PKG = ROOT / "fused-attention-cuda_amd"

pytestmark = pytest.mark.skipif(not capi.LIB_PATH.exists(),
                                reason="libfa_hip.so not built (run __graft_entry__.build())")


def header_functions() -> list[str]:
    text = HEADER.read_text()
    return re.findall(r"^FA_API\s+[\w\s\*]+?\b(fa_\w+)\(", text, flags=re.M)


def test_header_declares_the_capi_exports():
    assert header_functions() == list(capi.EXPORTS)


def test_library_exports_exactly_the_header_functions():
    lib = capi.load()
    for name in header_functions():
        assert hasattr(lib, name), name
    out = subprocess.run(["nm", "-D", "--defined-only", str(capi.LIB_PATH)], capture_output=True,
                         text=True, check=True).stdout
    text_syms = sorted(line.split()[-1] for line in out.splitlines() if " T " in line)
    assert text_syms == sorted(header_functions())


def test_names_and_sizes():
    lib = capi.load()
    assert [lib.fa_impl_name(i).decode() for i in range(0, 7)] == [
        "unknown", "naive", "tiled", "fused", "wmma", "tuned", "unknown"]
    assert [lib.fa_dtype_name(i).decode() for i in range(-1, 4)] == [
        "unknown", "fp32", "fp16", "bf16", "unknown"]
    assert [lib.fa_dtype_size(i) for i in range(-1, 4)] == [0, 4, 2, 2, 0]


def test_workspace_bytes():
    lib = capi.load()
    p = capi.params(2, 8, 8, 2048, 64, 0.125, False)
    assert lib.fa_workspace_bytes(1, 0, p) == 2 * 2 * 8 * 2048 * 2048 * 4
    assert lib.fa_workspace_bytes(2, 1, p) == 2 * 2 * 8 * 2048 * 2048 * 4
    for impl in (3, 4, 5):
        assert lib.fa_workspace_bytes(impl, 1, p) == 0


def _split_bytes(splits, rows, d):
    opart = (splits * rows * d * 4 + 255) // 256 * 256
    return opart + splits * rows * 4


def test_stage5_split_workspace(monkeypatch):
    """Stage 5 asks for a workspace (fp32 partial O [S, B, H, N, D] + LSE [S, B, H, N]) only where
    its cost model splits the key walks. The model assumes MI355X's 256 CUs on any device (the
    size must not depend on which device is current):
    one GPU's share of LONG over 8 GPUs (B1 H2 N8192 causal) splits in two, of C128 causal over 8
    (B2 H1) in three, a single head of N 2048 at D 64 in four; the whole benchmark shapes, the
    GPT-2 attention shape and C64's share over 8 GPUs (B2 H1, whose four-split tile already halves
    the walks) do not."""
    monkeypatch.delenv("FA_FORCE_SPLITS", raising=False)
    lib = capi.load()
    f16, bf16 = capi.FA_DTYPE_F16, capi.FA_DTYPE_BF16
    assert lib.fa_workspace_bytes(5, bf16, capi.params(1, 2, 2, 8192, 128, 0.088, True)) == \
        _split_bytes(2, 2 * 8192, 128)
    assert lib.fa_workspace_bytes(5, f16, capi.params(2, 1, 1, 2048, 128, 0.088, True)) == \
        _split_bytes(3, 2 * 2048, 128)
    assert lib.fa_workspace_bytes(5, f16, capi.params(1, 1, 1, 2048, 64, 0.125, False)) == \
        _split_bytes(4, 2048, 64)
    for b, h, n, d, dt, causal in [(2, 1, 2048, 64, f16, False), (2, 8, 2048, 64, f16, False),
                                   (2, 8, 2048, 128, f16, False),
                                   (2, 8, 2048, 128, f16, True), (1, 16, 8192, 128, bf16, True),
                                   (1, 16, 512, 128, bf16, True), (1, 16, 1024, 128, bf16, True),
                                   (8, 12, 1024, 64, f16, True)]:
        assert lib.fa_workspace_bytes(5, dt, capi.params(b, h, h, n, d, 0.1, causal)) == 0
    # Stages 3 and 4 never split; fp32 has no stage-5 kernel.
    p = capi.params(2, 1, 1, 2048, 64, 0.125, False)
    assert lib.fa_workspace_bytes(3, f16, p) == 0 and lib.fa_workspace_bytes(4, f16, p) == 0
    assert lib.fa_workspace_bytes(5, capi.FA_DTYPE_F32, p) == 0
    # FA_FORCE_SPLITS (test-only) forces S, capped at 16.
    monkeypatch.setenv("FA_FORCE_SPLITS", "3")
    assert lib.fa_workspace_bytes(5, f16, capi.params(1, 2, 2, 256, 64, 0.125, True)) == \
        _split_bytes(3, 2 * 256, 64)
    monkeypatch.setenv("FA_FORCE_SPLITS", "99")
    assert lib.fa_workspace_bytes(5, bf16, capi.params(1, 1, 1, 128, 128, 0.1, False)) == \
        _split_bytes(16, 128, 128)


def test_stage5_plan(monkeypatch):
    """fa_s5_plan names stage 5's (BR, BC, S) without a device (the CU count then reads as
    MI355X's 256): the benchmark shapes' tiles, the four-split tiles of small grids, forced tiles,
    and the same S as fa_workspace_bytes; invalid params and fp32 are refused."""
    for var in ("FA_FORCE_BR", "FA_FORCE_BC", "FA_FORCE_SPLITS"):
        monkeypatch.delenv(var, raising=False)
    lib = capi.load()
    lib.fa_set_debug_overrides(0, 0)
    f16, bf16 = capi.FA_DTYPE_F16, capi.FA_DTYPE_BF16
    cases = [((2, 8, 2048, 64, False), f16, (128, 128, 1)),   # C64
             ((2, 8, 2048, 128, False), f16, (128, 64, 1)),   # C128
             ((2, 8, 2048, 64, True), f16, (64, 128, 1)),     # C64 causal
             ((8, 12, 1024, 64, True), f16, (128, 32, 1)),    # GPT-2 attention
             ((8, 12, 1024, 64, False), f16, (128, 32, 1)),   # D = 64, N <= 2048, 3 per CU
             ((3, 8, 2048, 64, True), f16, (64, 64, 1)),      # D = 64 causal, 1.5 per CU: narrow
             ((4, 8, 4096, 64, False), f16, (256, 64, 1)),    # D = 64 dense, whole rounds
             ((2, 16, 4096, 64, True), f16, (256, 64, 1)),    # D = 64 causal N 4096, 2 rounds
             ((1, 16, 4096, 64, True), f16, (128, 128, 1)),   # one round: wide
             ((1, 16, 8192, 128, True), bf16, (128, 32, 1)),  # LONG
             ((1, 16, 512, 128, True), bf16, (32, 128, 1)),   # four splits, BR 32
             ((1, 16, 1024, 128, True), bf16, (64, 128, 1)),  # four splits, BR 64
             ((1, 8, 2048, 64, False), f16, (64, 256, 1)),    # four splits at D = 64
             ((2, 1, 2048, 64, True), f16, (32, 256, 1)),     # four splits instead of S = 2
             ((1, 2, 8192, 128, True), bf16, (64, 64, 2))]    # S = 2: four splits would not fit
    for (b, h, n, d, causal), dt, plan in cases:
        p = capi.params(b, h, h, n, d, 0.1, causal)
        assert capi.s5_plan(dt, p) == plan, (b, h, n, d, causal)
        s = plan[2]
        want = 0 if s == 1 else _split_bytes(s, b * h * n, d)
        assert lib.fa_workspace_bytes(5, dt, p) == want
    gpt = capi.params(8, 12, 12, 1024, 64, 0.1, True)
    lib.fa_set_debug_overrides(0, 64)    # the tall tile's height goes with its width only
    assert capi.s5_plan(f16, gpt)[:2] == (64, 64)
    lib.fa_set_debug_overrides(64, 0)    # a forced height keeps the tall width
    assert capi.s5_plan(f16, gpt)[:2] == (64, 32)
    p = capi.params(1, 16, 16, 512, 128, 0.1, True)
    lib.fa_set_debug_overrides(128, 0)   # no BR 128 tile of the four-split width: BC 64
    assert capi.s5_plan(bf16, p)[:2] == (128, 64)
    lib.fa_set_debug_overrides(64, 0)    # BR 64 keeps the automatic width
    assert capi.s5_plan(bf16, p)[:2] == (64, 128)
    lib.fa_set_debug_overrides(0, 32)    # a forced width takes the height rule
    assert capi.s5_plan(bf16, p)[:2] == (32, 32)
    monkeypatch.setenv("FA_FORCE_BR", "64")
    monkeypatch.setenv("FA_FORCE_BC", "64")
    assert capi.s5_plan(bf16, p)[:2] == (64, 64)
    lib.fa_set_debug_overrides(0, 0)
    monkeypatch.delenv("FA_FORCE_BR")
    monkeypatch.delenv("FA_FORCE_BC")
    out = ctypes.c_int(-1)
    assert lib.fa_s5_plan(f16, ctypes.byref(p), None, ctypes.byref(out), None) == capi.HIP_SUCCESS
    assert out.value == 128
    bad = capi.params(1, 16, 16, 500, 128, 0.1, True)
    assert lib.fa_s5_plan(f16, ctypes.byref(bad), None, None, None) == capi.HIP_ERROR_INVALID_VALUE
    assert lib.fa_s5_plan(f16, None, None, None, None) == capi.HIP_ERROR_INVALID_VALUE
    assert lib.fa_s5_plan(capi.FA_DTYPE_F32, ctypes.byref(p), None, None, None) == \
        capi.HIP_ERROR_NOT_SUPPORTED


def test_impl_supports_registry():
    lib = capi.load()
    f32, f16, bf16 = capi.FA_DTYPE_F32, capi.FA_DTYPE_F16, capi.FA_DTYPE_BF16
    for d in (64, 128):
        assert not lib.fa_impl_supports(1, f32, d, 950) and not lib.fa_impl_supports(2, f16, d, 950)
        assert lib.fa_impl_supports(3, f32, d, 950) and lib.fa_impl_supports(3, f16, d, 950)
        assert not lib.fa_impl_supports(3, bf16, d, 950)  # contract: fused takes fp32/fp16
        for s in (4, 5):
            assert lib.fa_impl_supports(s, f16, d, 950) and lib.fa_impl_supports(s, bf16, d, 950)
            assert not lib.fa_impl_supports(s, f32, d, 950)
    assert not lib.fa_impl_supports(5, f16, 96, 950)
    assert not lib.fa_impl_supports(5, f16, 64, 942)  # code objects are gfx950-only
    assert not lib.fa_impl_supports(6, f16, 64, 950) and not lib.fa_impl_supports(0, f16, 64, 950)


class _Dev:
    """Fake 16-byte-aligned 'device' addresses: validation must reject before dereferencing."""

    q, k, v, o, lse = 0x10000, 0x20000, 0x30000, 0x40000, 0x50000


@pytest.mark.parametrize("field,value", [("B", 0), ("H", -1), ("Hkv", 0), ("N", 0), ("D", 0),
                                         ("D", 96), ("N", 100), ("Hkv", 4)])
def test_invalid_params_rejected_before_any_device_call(field, value):
    p = capi.params(1, 6, 6, 128, 64, 0.125, False)
    setattr(p, field, value)
    d = _Dev
    rc = capi.forward_raw(5, capi.FA_DTYPE_F16, d.q, d.k, d.v, d.o, d.lse, 0, p, 0)
    assert rc == capi.HIP_ERROR_INVALID_VALUE


def test_null_pointers_and_dtype_rejected():
    p = capi.params(1, 2, 2, 128, 64, 0.125, False)
    d = _Dev
    assert capi.forward_raw(5, 1, 0, d.k, d.v, d.o, d.lse, 0, p, 0) == capi.HIP_ERROR_INVALID_VALUE
    assert capi.forward_raw(5, 1, d.q, d.k, d.v, d.o, 0, 0, p, 0) == capi.HIP_ERROR_INVALID_VALUE
    assert capi.forward_raw(5, 7, d.q, d.k, d.v, d.o, d.lse, 0, p, 0) == \
        capi.HIP_ERROR_INVALID_VALUE
    assert capi.load().fa_forward(5, 1, d.q, d.k, d.v, d.o, d.lse, 0, None, 0) == \
        capi.HIP_ERROR_INVALID_VALUE


@pytest.mark.skipif(torch.cuda.is_available(), reason="checks the no-device path")
def test_valid_call_without_device_reports_the_hip_error():
    p = capi.params(1, 2, 2, 128, 64, 0.125, False)
    d = _Dev
    rc = capi.forward_raw(5, 1, d.q, d.k, d.v, d.o, d.lse, 0, p, 0)
    assert rc not in (capi.HIP_SUCCESS, capi.HIP_ERROR_INVALID_VALUE)
    assert "device" in capi.error_string(rc).lower()


def test_debug_overrides_and_env_layering(monkeypatch):
    lib = capi.load()
    bm, bn = ctypes.c_int(-1), ctypes.c_int(-1)
    monkeypatch.delenv("FA_FORCE_BR", raising=False)
    monkeypatch.delenv("FA_FORCE_BC", raising=False)
    try:
        lib.fa_set_debug_overrides(64, 32)
        lib.fa_get_debug_overrides(True, ctypes.byref(bm), ctypes.byref(bn))
        assert (bm.value, bn.value) == (64, 32)
        monkeypatch.setenv("FA_FORCE_BC", "128")
        lib.fa_get_debug_overrides(True, ctypes.byref(bm), ctypes.byref(bn))
        assert (bm.value, bn.value) == (64, 128)  # environment wins
        lib.fa_get_debug_overrides(False, ctypes.byref(bm), ctypes.byref(bn))
        assert (bm.value, bn.value) == (64, 32)
        monkeypatch.setenv("FA_FORCE_BR", "abc")  # malformed: ignored (and reported)
        lib.fa_get_debug_overrides(True, ctypes.byref(bm), ctypes.byref(bn))
        assert (bm.value, bn.value) == (64, 128)
    finally:
        lib.fa_set_debug_overrides(0, 0)


# ------------------------------------------------------------------------------------------------
# torch binding
# ------------------------------------------------------------------------------------------------
def test_op_schemas_are_the_references():
    import fused_attn

    assert fused_attn.is_available()
    schemas = {str(torch.ops.fused_attn.forward.default._schema),
               str(torch.ops.fused_attn.forward_stage.default._schema)}
    assert schemas == {
        "fused_attn::forward(Tensor q, Tensor k, Tensor v, bool is_causal, float scale) -> Tensor",
        "fused_attn::forward_stage(Tensor q, Tensor k, Tensor v, bool is_causal, float scale, "
        "int stage) -> (Tensor, Tensor)",
    }
    assert torch.ops.fused_attn.impl_name(5) == "tuned"
    with pytest.raises(RuntimeError, match="stage must be in 1..5"):
        torch.ops.fused_attn.impl_name(0)
    if not torch.cuda.is_available():
        assert torch.ops.fused_attn.impl_supports(5, "fp16", 64) is False


def test_fake_kernels_give_reference_metadata():
    import fused_attn  # noqa: F401  (registers the fakes)
    from torch._subclasses.fake_tensor import FakeTensorMode

    with FakeTensorMode():
        q = torch.empty(2, 4, 256, 64, dtype=torch.float16)
        o = torch.ops.fused_attn.forward(q, q, q, False, 0.125)
        assert o.shape == q.shape and o.dtype == q.dtype
        for stage in (1, 2, 3, 4, 5):
            o_s, lse = torch.ops.fused_attn.forward_stage(q, q, q, True, 0.125, stage)
            assert o_s.shape == q.shape
            assert tuple(lse.shape) == ((2, 4, 256) if stage >= 3 else (0,))
            assert lse.dtype == torch.float32
        bad = torch.empty(2, 4, 100, 64, dtype=torch.float16)
        with pytest.raises(RuntimeError, match="multiple of 32"):
            torch.ops.fused_attn.forward(bad, bad, bad, False, 0.125)


def test_cpu_tensors_are_refused():
    import fused_attn

    q = torch.randn(1, 2, 64, 64)
    with pytest.raises(RuntimeError, match="CUDA"):
        fused_attn.forward(q, q, q)


def test_product_sources_never_reach_the_oracle():
    """The product (kernel library, binding, Python package) must not import, link or call the
    CPU oracle: parity claims rest on the HIP path being the thing that runs."""
    for path in list((PKG / "csrc").iterdir()) + list((PKG / "fused_attn").glob("*.py")):
        if path.suffix in {".h", ".cpp", ".hip", ".py"}:
            text = path.read_text()
            assert "oracle" not in text.lower().replace("oracle-free", ""), path


def test_noalloc_scratch_holds_every_automatic_split():
    """fa_decode_noalloc serves every problem whose split count the library picks itself
    (num_splits = 0): for B*Hkv from 1 to 300 split groups, up to 64 query rows per kv head and
    D = 64 or 128 on a long cache, the partials of the automatic split count fit the scratch
    array. B*Hkv = 255 with 64 rows of D = 128 is the largest (2 splits, 16,842,240 bytes)."""
    lib = capi.load()
    text = HEADER.read_text()
    m = re.search(r"#define FA_DECODE_SCRATCH_BYTES \((\d+)u << (\d+)\)", text)
    assert m is not None
    assert int(m.group(1)) << int(m.group(2)) == capi.DECODE_SCRATCH_BYTES
    worst = 0
    for groups in range(1, 301):
        for g, nq in ((1, 1), (4, 4), (16, 4), (64, 1)):
            for d in (64, 128):
                p = capi.FaDecodeParams(groups, g, 1, nq, 1 << 20, d, 0.125, True, 0)
                need = lib.fa_decode_workspace_bytes(capi.FA_DTYPE_BF16, ctypes.byref(p))
                assert need <= capi.DECODE_SCRATCH_BYTES, (groups, g, nq, d, need)
                worst = max(worst, need)
    assert worst == 16_842_240
