"""GPU parity through the C-ABI (marker ``gpu``): ``fa_forward`` of libfa_hip.so called with ctypes
on device buffers, with no torch op in between.

* Golden vectors written by the reference's own fp64 oracle (tests/golden/) -- the reference's
  CPU-runnable case (B1 H2 N128 D64 fp32), a GQA/D128/partial-tile case and rounded fp16/bf16 inputs -- on
  every stage that takes the dtype, to the stated tolerance.
* Status codes of the boundary on a real device (ref:src/dispatch.cu:140-161,
  ref:src/stage5_tuned.cu:983-1026): unsupported stage -> hipErrorNotSupported; misaligned
  pointer, non-positive scale, uninstantiated tile, B*H > 65535 -> hipErrorInvalidValue; nothing
  is written on a refused call.
* Writes stay inside o / lse: both live between guard bands that must be untouched afterwards.
* The launch honours the caller's stream.
"""

from __future__ import annotations

from pathlib import Path

import numpy as np
import pytest
import torch

from _checks import LSE_ATOL, O_TOL, assert_close_tol
from fused_attn import capi

pytestmark = pytest.mark.gpu

GOLDEN = Path(__file__).resolve().parent / "golden"
TORCH_DTYPE = {"float32": torch.float32, "float16": torch.float16, "bfloat16": torch.bfloat16}
DTYPE_STAGES = {torch.float32: [3], torch.float16: [3, 4, 5], torch.bfloat16: [4, 5]}


def golden(name):
    z = np.load(GOLDEN / f"{name}.npz", allow_pickle=False)
    dt = TORCH_DTYPE[str(z["dtype"])]

    def dev(a):
        t = torch.from_numpy(a.view(np.int16)).view(torch.bfloat16) if dt == torch.bfloat16 \
            else torch.from_numpy(a)
        return t.to("cuda").contiguous()

    return z, dt, dev(z["q"]), dev(z["k"]), dev(z["v"]), float(z["scale"])


def run(stage, q, k, v, causal, scale, stream=None):
    b, h, n, d = q.shape
    o = torch.empty_like(q)
    lse = torch.empty(b, h, n, dtype=torch.float32, device=q.device)
    rc = capi.forward(stage, q, k, v, o, lse, causal, scale, stream=stream)
    return rc, o, lse


@pytest.mark.parametrize("causal", [0, 1], ids=["full", "causal"])
@pytest.mark.parametrize("name", ["cpu_b1h2n128d64_f32", "gqa_b1h2kv1n96d128_f32",
                                  "f16_b1h2n256d64", "bf16_b1h1n256d128"])
def test_golden_vectors_through_capi(name, causal):
    z, dt, q, k, v, scale = golden(name)
    assert capi.current_arch() == 950
    for stage in DTYPE_STAGES[dt]:
        rc, o, lse = run(stage, q, k, v, bool(causal), scale)
        assert rc == capi.HIP_SUCCESS, capi.error_string(rc)
        torch.cuda.synchronize()
        atol, rtol = O_TOL[dt]
        assert_close_tol(o, z[f"o_c{causal}"].astype(np.float64), atol, rtol, what=f"O s{stage}")
        assert_close_tol(lse, z[f"lse_c{causal}"], LSE_ATOL, 0.0, what=f"LSE s{stage}")


def test_fp32_input_on_a_half_stage_is_not_supported():
    q = torch.randn(1, 2, 64, 64, device="cuda")
    rc, _, _ = run(5, q, q, q, False, 0.125)
    assert rc == capi.HIP_ERROR_NOT_SUPPORTED
    rc, _, _ = run(1, q, q, q, False, 0.125)
    assert rc == capi.HIP_ERROR_NOT_SUPPORTED


@pytest.mark.parametrize("stage", [3, 4, 5])
def test_refused_calls_write_nothing(stage):
    dt = torch.float32 if stage == 3 else torch.float16
    b, h, n, d = 1, 2, 128, 64
    q = torch.randn(b, h, n, d, device="cuda").to(dt)
    o = torch.full_like(q, 7.0)
    lse = torch.full((b, h, n), 7.0, device="cuda")
    lib = capi.load()

    def call(p, qp=q.data_ptr()):
        return capi.forward_raw(stage, capi.DTYPE_CODES[dt], qp, q.data_ptr(), q.data_ptr(),
                                o.data_ptr(), lse.data_ptr(), 0, p, 0)

    assert call(capi.params(b, h, h, n, d, 0.0, False)) == capi.HIP_ERROR_INVALID_VALUE
    assert call(capi.params(b, h, h, n, d, float("nan"), False)) == capi.HIP_ERROR_INVALID_VALUE
    assert call(capi.params(b, h, h, n, d, 0.125, False), q.data_ptr() + 4) == \
        capi.HIP_ERROR_INVALID_VALUE
    assert call(capi.params(65536, 1, 1, n, d, 0.125, False)) == capi.HIP_ERROR_INVALID_VALUE
    lib.fa_set_debug_overrides(0, 48)
    try:
        assert call(capi.params(b, h, h, n, d, 0.125, False)) == capi.HIP_ERROR_INVALID_VALUE
    finally:
        lib.fa_set_debug_overrides(0, 0)
    torch.cuda.synchronize()
    assert bool((o == 7.0).all()) and bool((lse == 7.0).all())


@pytest.mark.parametrize("causal", [False, True], ids=["full", "causal"])
@pytest.mark.parametrize("stage,dt,d", [(3, torch.float32, 128), (4, torch.bfloat16, 64),
                                        (5, torch.float16, 64), (5, torch.bfloat16, 128)])
def test_writes_stay_inside_o_and_lse(stage, dt, d, causal):
    """o and lse are carved out of larger buffers; the guard bands around them must keep their
    sentinel. N = 96 leaves a partial key tile, and with BR = 128 (stages 3 and 4 always; stage 5
    when forced, its default height for this small grid being 32) a partial query tile."""
    b, h, n = 2, 3, 96
    guard = 4096
    gen = torch.Generator().manual_seed(3)
    q, k, v = (torch.randn(b, h, n, d, generator=gen).to("cuda", dt) for _ in range(3))
    from oracle.oracle import math_reference

    ref, lse64 = math_reference(q, k, v, is_causal=causal)
    numel = q.numel()
    lib = capi.load()
    for br in ((0, 128) if stage == 5 else (0,)):
        obuf = torch.full((guard + numel + guard,), 3.0, dtype=dt, device="cuda")
        lbuf = torch.full((guard + b * h * n + guard,), 3.0, dtype=torch.float32, device="cuda")
        o = obuf[guard:guard + numel].view(b, h, n, d)
        lse = lbuf[guard:guard + b * h * n].view(b, h, n)
        lib.fa_set_debug_overrides(br, 0)
        try:
            rc = capi.forward(stage, q, k, v, o, lse, causal, d ** -0.5)
        finally:
            lib.fa_set_debug_overrides(0, 0)
        assert rc == capi.HIP_SUCCESS, capi.error_string(rc)
        torch.cuda.synchronize()
        for buf, n_in in ((obuf, numel), (lbuf, b * h * n)):
            assert bool((buf[:guard] == 3.0).all()) and bool((buf[guard + n_in:] == 3.0).all())
        assert_close_tol(o, ref, *O_TOL[dt])
        assert_close_tol(lse, lse64, LSE_ATOL, 0.0, what="LSE")


def test_launch_honours_the_callers_stream():
    gen = torch.Generator().manual_seed(4)
    q, k, v = (torch.randn(2, 4, 512, 64, generator=gen).to("cuda", torch.float16)
               for _ in range(3))
    rc, o_ref, _ = run(5, q, k, v, True, 0.125)
    assert rc == capi.HIP_SUCCESS
    torch.cuda.synchronize()
    s = torch.cuda.Stream()
    with torch.cuda.stream(s):
        o = torch.empty_like(q)
        lse = torch.empty(2, 4, 512, device="cuda")
    s.wait_stream(torch.cuda.current_stream())
    rc = capi.forward(5, q, k, v, o, lse, True, 0.125, stream=s)
    assert rc == capi.HIP_SUCCESS
    s.synchronize()
    assert torch.equal(o, o_ref)


def test_forced_height_alone_is_valid_on_any_grid():
    """A forced stage-5 height without a forced width takes a built width for that height: on
    B1 H1 N4096 D64 the automatic width is 128 and (256, 128) is not built, so BR = 256 alone runs
    with the widest built width for that height (64). Before, the pair was refused."""
    gen = torch.Generator().manual_seed(8)
    q, k, v = (torch.randn(1, 1, 4096, 64, generator=gen).to("cuda", torch.float16)
               for _ in range(3))
    from oracle.oracle import math_reference_rows

    lib = capi.load()
    lib.fa_set_debug_overrides(256, 0)
    try:
        rc, o, lse = run(5, q, k, v, False, 0.125)
    finally:
        lib.fa_set_debug_overrides(0, 0)
    assert rc == capi.HIP_SUCCESS, capi.error_string(rc)
    torch.cuda.synchronize()
    rows = np.r_[0:64, 2000:2064, 4032:4096]
    o64, l64 = math_reference_rows(q, k, v, 0, 0, rows, is_causal=False, scale=0.125)
    assert_close_tol(o[0, 0, rows], o64, *O_TOL[torch.float16])
    assert_close_tol(lse[0, 0, rows], l64, LSE_ATOL, 0.0, what="LSE")
