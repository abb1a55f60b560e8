"""Pinning of the split-KV decode oracle (``oracle.decode_reference``, ``oracle.combine_splits``)
without a GPU. Decode has no reference implementation (it is the reference's stated next step,
ref:README.md:1357-1358), so each function is pinned by what the mathematics fixes:

* bottom-right causal with Nq == Nkv is the top-left causal of the pinned forward oracle;
* against torch SDPA MATH in fp64 (a library routine), with the mask built by torch's own
  ``tril`` for the causal case and no mask otherwise;
* brute-force Python loops on tiny shapes;
* the split/combine identity: running the oracle on key chunks and combining with the LSE rule
  reproduces the unsplit answer (and a mistaken weight, e.g. dropping the max shift or using
  e^L_s without normalising, fails it);
* rows that see no key: O = 0, LSE = +inf, and empty splits carry no weight.
"""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle.oracle import combine_splits, decode_keep_mask, decode_reference, math_reference

TOL = 1e-12


def rand(shape, seed):
    return np.random.default_rng(seed).standard_normal(shape)


def sdpa64(q, k, v, mask, scale):
    with torch.nn.attention.sdpa_kernel(torch.nn.attention.SDPBackend.MATH):
        o = F.scaled_dot_product_attention(torch.from_numpy(q), torch.from_numpy(k),
                                           torch.from_numpy(v), attn_mask=mask, scale=scale)
    return o.numpy()


def test_square_causal_equals_top_left_forward():
    q, k, v = rand((1, 2, 64, 32), 1), rand((1, 2, 64, 32), 2), rand((1, 2, 64, 32), 3)
    o, lse = decode_reference(q, k, v, is_causal=True)
    o2, lse2 = math_reference(q, k, v, is_causal=True)
    assert np.abs(o - o2).max() < TOL and np.abs(lse - lse2).max() < TOL


@pytest.mark.parametrize("nq,nkv,causal", [(1, 37, False), (1, 37, True), (4, 70, True),
                                           (8, 8, True), (3, 200, False)])
def test_against_torch_sdpa_fp64(nq, nkv, causal):
    q, k, v = rand((2, 4, nq, 16), 4), rand((2, 4, nkv, 16), 5), rand((2, 4, nkv, 16), 6)
    scale = 0.3
    mask = (torch.ones(nq, nkv, dtype=torch.bool).tril(diagonal=nkv - nq) if causal else None)
    ref = sdpa64(q, k, v, mask, scale)
    o, _ = decode_reference(q, k, v, is_causal=causal, scale=scale)
    assert np.abs(o - ref).max() < TOL


def test_gqa_head_mapping_against_sdpa():
    q, k, v = rand((1, 8, 2, 16), 7), rand((1, 2, 50, 16), 8), rand((1, 2, 50, 16), 9)
    mask = torch.ones(2, 50, dtype=torch.bool).tril(diagonal=48)
    ref = sdpa64(q, np.repeat(k, 4, axis=1), np.repeat(v, 4, axis=1), mask, 0.25)
    o, _ = decode_reference(q, k, v, is_causal=True, scale=0.25)
    assert np.abs(o - ref).max() < TOL


def test_brute_force_loops_tiny():
    nq, nkv, d = 3, 5, 4
    q, k, v = rand((1, 1, nq, d), 10), rand((1, 1, nkv, d), 11), rand((1, 1, nkv, d), 12)
    scale = 0.7
    o, lse = decode_reference(q, k, v, is_causal=True, scale=scale)
    for i in range(nq):
        keys = [j for j in range(nkv) if j <= nkv - nq + i]
        sc = [scale * sum(q[0, 0, i, x] * k[0, 0, j, x] for x in range(d)) for j in keys]
        m = max(sc)
        w = [math.exp(s - m) for s in sc]
        tot = sum(w)
        for x in range(d):
            want = sum(w[t] * v[0, 0, j, x] for t, j in enumerate(keys)) / tot
            assert abs(o[0, 0, i, x] - want) < TOL
        assert abs(lse[0, 0, i] - (m + math.log(tot))) < TOL


def split_partials(q, k, v, causal, scale, bounds):
    """Oracle on each key chunk [a, b): mask = global bottom-right mask restricted to the chunk."""
    nq, nkv = q.shape[2], k.shape[2]
    full = decode_keep_mask(nq, nkv, causal)
    os_, ls = [], []
    for a, b in bounds:
        keep = np.ones((nq, b - a), dtype=bool) if full is None else full[:, a:b]
        o, lse = math_reference(q, k[:, :, a:b], v[:, :, a:b], scale=scale, attn_mask=keep)
        lse = np.where(np.isposinf(lse), -np.inf, lse)  # empty split: weight 0
        os_.append(o)
        ls.append(lse)
    return np.stack(os_), np.stack(ls)


@pytest.mark.parametrize("causal", [False, True])
def test_split_combine_identity(causal):
    q, k, v = rand((2, 2, 4, 16), 13), rand((2, 2, 300, 16), 14), rand((2, 2, 300, 16), 15)
    o_ref, lse_ref = decode_reference(q, k, v, is_causal=causal, scale=0.2)
    bounds = [(0, 128), (128, 256), (256, 300)]
    op, lp = split_partials(q, k, v, causal, 0.2, bounds)
    o, lse = combine_splits(op, lp)
    assert np.abs(o - o_ref).max() < TOL and np.abs(lse - lse_ref).max() < TOL


def test_combine_rejects_plausible_mistakes():
    """The identity must catch a wrong weight: unnormalised e^L_s, or O_s averaged uniformly."""
    q, k, v = rand((1, 1, 2, 8), 16), rand((1, 1, 256, 8), 17), rand((1, 1, 256, 8), 18)
    o_ref, _ = decode_reference(q, k, v, scale=1.0)
    op, lp = split_partials(q, k, v, False, 1.0, [(0, 64), (64, 256)])
    wrong_unnormalised = (np.exp(lp)[..., None] * op).sum(axis=0)
    wrong_uniform = op.mean(axis=0)
    assert np.abs(wrong_unnormalised - o_ref).max() > 1e-3
    assert np.abs(wrong_uniform - o_ref).max() > 1e-3


def test_rows_without_keys_and_empty_splits():
    # Nq > Nkv, causal: token i sees keys j <= Nkv - Nq + i, none for i < Nq - Nkv.
    q, k, v = rand((1, 1, 6, 8), 19), rand((1, 1, 3, 8), 20), rand((1, 1, 3, 8), 21)
    o, lse = decode_reference(q, k, v, is_causal=True)
    assert np.all(o[0, 0, :3] == 0) and np.all(np.isposinf(lse[0, 0, :3]))
    assert np.all(np.isfinite(lse[0, 0, 3:]))
    # A split that a row cannot see carries lse -inf and leaves the combine unchanged.
    op, lp = split_partials(q, k, v, True, 1 / math.sqrt(8), [(0, 1), (1, 3)])
    o2, lse2 = combine_splits(op, lp)
    assert np.all(o2[0, 0, :3] == 0) and np.all(np.isposinf(lse2[0, 0, :3]))
    assert np.abs(o2[0, 0, 3:] - o[0, 0, 3:]).max() < TOL
