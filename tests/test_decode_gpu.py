"""Split-KV decode on the GPU (marker ``gpu``), through the torch op and through the C-ABI,
against the fp64 decode oracle (``oracle.decode_reference``, pinned in test_decode_cpu.py) at the
O within 2e-3 abs + 2e-3 rel (plus bf16's output rounding), LSE within 1e-3.

Cases cover MHA and GQA decode (Nq = 1), several new tokens with bottom-right causal masking,
ragged cache lengths (Nkv not a multiple of 32 or of the 128-key tile, shorter than one tile),
the full 32-row group, one split against many, and rows that see no key (Nq > Nkv, causal)."""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch

import fused_attn
from _checks import LSE_ATOL, O_TOL, assert_close_tol
from fused_attn import capi
from oracle.oracle import decode_reference

pytestmark = pytest.mark.gpu
_ids = {torch.float16: "fp16", torch.bfloat16: "bf16"}


def require_ext():
    if not fused_attn.is_available():
        pytest.fail("fused_attn._C is not built: the HIP path must be the one that runs")


def make(b, h, hkv, nq, nkv, d, dtype, seed):
    gen = torch.Generator(device="cpu").manual_seed(seed)
    q = torch.randn(b, h, nq, d, generator=gen).to("cuda", dtype)
    k = torch.randn(b, hkv, nkv, d, generator=gen).to("cuda", dtype)
    v = torch.randn(b, hkv, nkv, d, generator=gen).to("cuda", dtype)
    return q, k, v


def check(o, lse, q, k, v, causal, dtype, scale=None):
    ref_o, ref_lse = decode_reference(q, k, v, is_causal=causal, scale=scale)
    atol, rtol = O_TOL[dtype]
    assert_close_tol(o, ref_o, atol, rtol)
    lse64 = lse.double().cpu().numpy()
    fin = np.isfinite(ref_lse)
    assert np.array_equal(np.isposinf(lse64), ~fin), "rows without keys must report lse = +inf"
    assert_close_tol(lse64[fin], ref_lse[fin], LSE_ATOL, 0.0, what="LSE")


CASES = [
    # b, h, hkv, nq, nkv, d, causal, splits
    (2, 8, 8, 1, 1000, 128, False, 0),   # MHA decode, ragged cache
    (1, 32, 8, 1, 4096, 128, True, 0),   # GQA 4:1
    (2, 8, 2, 4, 777, 64, True, 0),      # 4 new tokens, 16-row groups, ragged
    (1, 8, 1, 4, 300, 64, True, 3),      # full 32-row group (MQA-like), 3 splits
    (1, 2, 2, 1, 5, 64, False, 0),       # cache shorter than one 32-key block
    (3, 4, 4, 2, 129, 128, True, 0),     # one key past a tile
    (1, 4, 4, 8, 2048, 64, False, 1),    # a single split
    (2, 16, 2, 6, 900, 128, True, 0),    # R = 48: two row groups, the second half full, ragged
    (1, 64, 8, 8, 3000, 128, True, 0),   # R = 64: GQA 8:1 with 8 new tokens (speculative)
    (1, 32, 1, 2, 513, 64, False, 2),    # R = 64 at D = 64 (MQA-like), 2 splits
]


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16], ids=lambda t: _ids[t])
@pytest.mark.parametrize("case", CASES, ids=lambda c: "b{}h{}kv{}nq{}nkv{}d{}{}s{}".format(
    *c[:6], "c" if c[6] else "", c[7]))
def test_decode_op_matches_oracle(case, dtype):
    require_ext()
    b, h, hkv, nq, nkv, d, causal, splits = case
    q, k, v = make(b, h, hkv, nq, nkv, d, dtype, seed=nkv + nq)
    print(f"decode case {case} {dtype}", flush=True)
    o, lse = fused_attn.decode(q, k, v, is_causal=causal, num_splits=splits)
    torch.cuda.synchronize()
    assert o.shape == q.shape and o.dtype == dtype and lse.shape == (b, h, nq)
    check(o, lse, q, k, v, causal, dtype)


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16], ids=lambda t: _ids[t])
def test_one_split_and_many_splits_agree(dtype):
    require_ext()
    q, k, v = make(1, 8, 2, 2, 5000, 128, dtype, seed=3)
    o1, l1 = fused_attn.decode(q, k, v, is_causal=True, num_splits=1)
    o8, l8 = fused_attn.decode(q, k, v, is_causal=True, num_splits=8)
    o0, l0 = fused_attn.decode(q, k, v, is_causal=True)  # library choice
    torch.cuda.synchronize()
    atol, rtol = O_TOL[dtype]
    for o, lse in ((o8, l8), (o0, l0)):
        assert_close_tol(o, o1.double().cpu().numpy(), atol, rtol)
        assert_close_tol(lse, l1.double().cpu().numpy(), LSE_ATOL, 0.0, what="LSE")
    check(o8, l8, q, k, v, True, dtype)


@pytest.mark.parametrize("nkv,nq,causal", [(2, 1, False), (6, 2, False), (16, 4, True),
                                            (100, 1, False), (140, 16, True), (200, 1, False)])
def test_bf16_short_cache_flat_rows(nkv, nq, causal):
    """bf16 rows over a few keys with a small scale (flat probabilities): the probabilities' bf16
    rounding does not average out over a few keys, so below 128 visible keys the kernel adds their
    low parts; at and above it (140 keys minus 15 for the first causal token, 200) it does not
    need them. Both sides must meet the bar."""
    require_ext()
    q, k, v = make(2, 8, 4, nq, nkv, 128, torch.bfloat16, seed=11 * nkv + nq)
    scale = 0.25 / math.sqrt(128)
    o, lse = fused_attn.decode(q, k, v, is_causal=causal, scale=scale)
    torch.cuda.synchronize()
    check(o, lse, q, k, v, causal, torch.bfloat16, scale=scale)


def test_rows_without_keys():
    """Nq > Nkv, causal: tokens i < Nq - Nkv see no key -> O = 0, lse = +inf."""
    require_ext()
    q, k, v = make(1, 2, 2, 8, 4, 64, torch.float16, seed=5)
    o, lse = fused_attn.decode(q, k, v, is_causal=True)
    torch.cuda.synchronize()
    assert torch.all(o[:, :, :4] == 0) and torch.all(torch.isinf(lse[:, :, :4]))
    check(o, lse, q, k, v, True, torch.float16)


def test_capi_decode_with_caller_workspace():
    require_ext()
    q, k, v = make(2, 16, 4, 1, 3000, 128, torch.bfloat16, seed=7)
    p = capi.decode_params(q, k, True, 1 / 128 ** 0.5, 0)
    lib = capi.load()
    splits = lib.fa_decode_num_splits(p)
    nbytes = lib.fa_decode_workspace_bytes(capi.FA_DTYPE_BF16, p)
    assert splits > 1 and nbytes >= 2 * 4 * splits * 4 * 129 * 4
    ws = torch.empty(nbytes, dtype=torch.uint8, device="cuda")
    o = torch.empty_like(q)
    lse = torch.empty(2, 16, 1, dtype=torch.float32, device="cuda")
    rc = capi.decode(q, k, v, o, lse, True, 1 / 128 ** 0.5, workspace=ws)
    torch.cuda.synchronize()
    assert rc == 0, capi.error_string(rc)
    check(o, lse, q, k, v, True, torch.bfloat16)


def test_capi_decode_errors():
    require_ext()
    q, k, v = make(1, 8, 8, 1, 256, 64, torch.float16, seed=9)
    o = torch.empty_like(q)
    lse = torch.empty(1, 8, 1, dtype=torch.float32, device="cuda")
    # missing workspace while more than one split is needed
    p = capi.decode_params(q, k, False, 0.125, 2)
    rc = capi.load().fa_decode(capi.FA_DTYPE_F16, q.data_ptr(), k.data_ptr(), v.data_ptr(),
                               o.data_ptr(), lse.data_ptr(), None, p, 0)
    assert rc == capi.HIP_ERROR_INVALID_VALUE
    # fp32 is not covered by decode
    q32, k32, v32 = (t.float() for t in (q, k, v))
    rc = capi.decode(q32, k32, v32, q32.clone(), lse, False, 0.125)
    assert rc == capi.HIP_ERROR_NOT_SUPPORTED
    # more than 64 query rows per kv head
    qb, kb, vb = make(1, 8, 1, 9, 256, 64, torch.float16, seed=10)
    rc = capi.decode(qb, kb, vb, torch.empty_like(qb), torch.empty(1, 8, 9, device="cuda"), False,
                     0.125)
    assert rc == capi.HIP_ERROR_NOT_SUPPORTED


def test_op_error_messages_and_opcheck():
    require_ext()
    q, k, v = make(1, 8, 1, 9, 256, 64, torch.float16, seed=11)
    with pytest.raises(RuntimeError, match="not implemented"):
        fused_attn.decode(q, k, v)
    q, k, v = make(1, 6, 4, 1, 64, 64, torch.float16, seed=12)
    with pytest.raises(RuntimeError, match="multiple of Hkv"):
        fused_attn.decode(q, k, v)
    q, k, v = make(1, 4, 2, 2, 300, 64, torch.bfloat16, seed=13)
    torch.library.opcheck(torch.ops.fused_attn.decode, (q, k, v, True, 0.125, 0),
                          test_utils=("test_schema", "test_faketensor"))
