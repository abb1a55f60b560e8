"""Tolerance policy and the comparison helper shared by the GPU parity tests.

Two bars, both enforced:

* The build's stated tolerance against the fp64 oracle (north star): O within
  ``|o - ref| <= atol + rtol * |ref|`` with fp32 (1e-5, 1e-5) and fp16/bf16 (2e-3, 2e-3); LSE within
  1e-3 absolute. For bf16 the relative term adds bf16's unit roundoff 2^-8 (~3.9e-3): O is stored
  in the input dtype, and rounding the exact answer to bf16 alone can move it by up to 2^-8 * |O|,
  more than 2e-3 -- no bf16-output kernel can do better. fp16's unit roundoff (2^-11) fits inside
  the 2e-3 bar, so fp16 gets no such term.
* The reference's own gate (ref:tests/test_kernels_gpu.py:34-68): finite output, the
  FlashAttention ratio rule ``err_mine <= 2 * err_torch + 1e-6`` against torch's unfused attention in
  the same dtype, and the absolute caps fp32 1e-4 / fp16 1e-2 / bf16 5e-2.
"""

from __future__ import annotations

import numpy as np
import torch

from oracle.oracle import error_ratio, math_reference, to_f64, unfused_reference

BF16_UNIT_ROUNDOFF = 2.0 ** -8
O_TOL = {torch.float32: (1e-5, 1e-5), torch.float16: (2e-3, 2e-3),
         torch.bfloat16: (2e-3, 2e-3 + BF16_UNIT_ROUNDOFF)}
LSE_ATOL = 1e-3
ABS_CAP = {torch.float32: 1e-4, torch.float16: 1e-2, torch.bfloat16: 5e-2}
# The reference's LSE tolerance (atol, rtol), ref:tests/test_kernels_gpu.py:36.
LSE_TOL_REF = {torch.float32: (1e-4, 1e-5), torch.float16: (2e-2, 1e-3),
               torch.bfloat16: (5e-2, 5e-3)}


def assert_close_tol(out, ref64: np.ndarray, atol: float, rtol: float, what: str = "O") -> float:
    o = to_f64(out)
    err = np.abs(o - ref64)
    bound = atol + rtol * np.abs(ref64)
    worst = float(np.max(err - bound)) if err.size else -1.0
    assert np.isfinite(o).all(), f"{what}: non-finite values"
    assert worst <= 0.0, (f"{what}: max |err| {float(err.max()):.3e} exceeds atol {atol} + rtol "
                          f"{rtol}*|ref| (worst excess {worst:.3e})")
    return float(err.max()) if err.size else 0.0


def check_against_reference(o, q, k, v, causal, dtype, attn_mask=None, scale=None, lse=None):
    """Ratio rule + caps (reference) and the north-star tolerance; returns the ratio result."""
    ref64, lse64 = math_reference(q, k, v, is_causal=causal, scale=scale, attn_mask=attn_mask)
    pt = unfused_reference(q, k, v, is_causal=causal, scale=scale, attn_mask=attn_mask,
                           device=str(q.device))
    r = error_ratio(o, ref64, pt)
    assert r.out_finite, "kernel produced NaN/inf"
    assert r.ok, f"ratio rule failed: {r}"
    assert r.err_mine <= ABS_CAP[dtype], f"absolute cap {ABS_CAP[dtype]} exceeded: {r}"
    atol, rtol = O_TOL[dtype]
    assert_close_tol(o, ref64, atol, rtol)
    if lse is not None:
        assert_close_tol(lse, lse64, LSE_ATOL, 0.0, what="LSE")
    return r


def fp32_reference_head(q, k, v, bi, hi, causal, scale):
    """Plain PyTorch fp32 attention for one head, every row, on the tensors' device: the fp32
    reference of the op. The kv head is h // (H / Hkv). Returns (O [N, D], LSE [N], scores [N, N])
    in fp32; the scores are returned for the LSE bounds some tests check."""
    hk = hi // (q.shape[1] // k.shape[1])
    q32, k32, v32 = q[bi, hi].float(), k[bi, hk].float(), v[bi, hk].float()
    s = torch.matmul(q32, k32.t().contiguous()) * scale
    if causal:
        n = s.shape[0]
        s = s.masked_fill(~torch.ones(n, n, dtype=torch.bool, device=s.device).tril(),
                          float("-inf"))
    return torch.matmul(torch.softmax(s, dim=-1), v32), torch.logsumexp(s, dim=-1), s


def assert_every_head_close(o, lse, q, k, v, causal, scale, what=""):
    """O and LSE of every (b, h) head against the fp32 reference, to the stated tolerance."""
    atol, rtol = O_TOL[o.dtype]
    b, h = q.shape[:2]
    for bi in range(b):
        for hi in range(h):
            o32, lse32, s = fp32_reference_head(q, k, v, bi, hi, causal, scale)
            del s
            err = (o[bi, hi].float() - o32).abs()
            excess = float((err - (atol + rtol * o32.abs())).max())
            assert excess <= 0.0, f"{what} head ({bi},{hi}): max|O err| {float(err.max()):.3e}"
            lerr = float((lse[bi, hi] - lse32).abs().max())
            assert lerr <= LSE_ATOL, f"{what} head ({bi},{hi}): max|LSE err| {lerr:.3e}"
