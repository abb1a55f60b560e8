"""Pins the CPU oracle (oracle/oracle.py and oracle/attn_oracle.c) before anything trusts it.

Independent checks, each chosen so a plausible mistake (a dropped rescale, a wrong sign or index,
a transposed operand, the wrong causal alignment, a mis-scaled LSE) fails at least one:

1. Golden vectors written by the REFERENCE's own compiled oracle (tests/golden/, produced by
   tests/golden/make_golden.py from ref:src/reference/cpu_reference.cpp via oracle/_ref).
2. The 2x2 closed form of ref:src/reference/test_cpu_reference.cpp:39-67 (hand-derived values).
3. torch SDPA under the MATH backend in fp64 (a library routine), incl. GQA via enable_gqa.
4. Invariants from the reference's CPU tests (ref:tests/test_reference_cpu.py): tiled == direct
   for any tiling, LSE == logsumexp, scale folding, causal == explicit tril, row 0 == v[0],
   sum_j exp(s_ij - lse_i) == 1, the fully-masked-row guards, and a deliberately broken recurrence
   (a mistake planted in a private oracle copy here on the CPU) that the tile test must catch.
5. The live reference oracle (oracle/_ref/libfa_ref.so) on fresh random shapes, when it is built.
"""

from __future__ import annotations

import math
from pathlib import Path

import numpy as np
import pytest
import torch

from oracle.oracle import (
    LOG2E,
    COracle,
    RefOracle,
    default_scale,
    error_ratio,
    math_reference,
    math_reference_rows,
    tiled_online_softmax_reference,
    unfused_reference,
)

GOLDEN = Path(__file__).resolve().parent / "golden"
TOL64 = 1e-10  # two exact fp64 algorithms that differ only in summation order


def qkv64(b, h, n, d, seed=0, hkv=None):
    gen = torch.Generator().manual_seed(seed)
    hkv = h if hkv is None else hkv
    q = torch.randn(b, h, n, d, generator=gen, dtype=torch.float64).numpy()
    k = torch.randn(b, hkv, n, d, generator=gen, dtype=torch.float64).numpy()
    v = torch.randn(b, hkv, n, d, generator=gen, dtype=torch.float64).numpy()
    return q, k, v


def max_abs(a, b) -> float:
    return float(np.max(np.abs(np.asarray(a, dtype=np.float64) - np.asarray(b, dtype=np.float64))))


@pytest.fixture(scope="module")
def c_oracle() -> COracle:
    return COracle()


def load_golden(name: str):
    z = np.load(GOLDEN / f"{name}.npz", allow_pickle=False)
    dtype = str(z["dtype"]) if "dtype" in z.files else "float64"

    def dec(a):
        if dtype == "bfloat16":
            return torch.from_numpy(a.view(np.int16)).view(torch.bfloat16).to(torch.float64).numpy()
        return a.astype(np.float64)

    return z, dec(z["q"]), dec(z["k"]), dec(z["v"]), float(z["scale"])


GOLDEN_CASES = ["cpu_b1h2n128d64_f32", "gqa_b1h2kv1n96d128_f32", "f16_b1h2n256d64",
                "bf16_b1h1n256d128"]


# ------------------------------------------------------------------------------------------------
# 1. golden vectors from the reference's own oracle
# ------------------------------------------------------------------------------------------------
@pytest.mark.parametrize("causal", [0, 1], ids=["full", "causal"])
@pytest.mark.parametrize("name", GOLDEN_CASES)
def test_oracles_match_reference_golden(name, causal, c_oracle):
    z, q, k, v, scale = load_golden(name)
    o_ref, lse_ref = z[f"o_c{causal}"], z[f"lse_c{causal}"]
    # O of the half-precision cases is stored as fp32 (rounded once): compare at that precision.
    tol_o = TOL64 if o_ref.dtype == np.float64 else 1e-6
    o_np, lse_np = math_reference(q, k, v, is_causal=bool(causal), scale=scale)
    o_c, lse_c = c_oracle.attention(q, k, v, is_causal=bool(causal), scale=scale)
    o_t, lse_t = tiled_online_softmax_reference(q, k, v, is_causal=bool(causal), scale=scale,
                                                block_m=32, block_n=16)
    for o, lse in ((o_np, lse_np), (o_c, lse_c), (o_t, lse_t)):
        assert max_abs(o, o_ref) < tol_o
        assert max_abs(lse, lse_ref) < TOL64
    # Bitwise-identical algorithm to the reference's direct form: the C restatement follows the
    # same loop order, so it must agree to the last few ulps.
    assert max_abs(o_c, o_ref) < (1e-13 if o_ref.dtype == np.float64 else 1e-6)


@pytest.mark.parametrize("name", ["cpu_b1h2n128d64_f32", "gqa_b1h2kv1n96d128_f32"])
def test_tiled_models_match_reference_tiled_golden(name, c_oracle):
    z, q, k, v, scale = load_golden(name)
    keys = [f for f in z.files if f.startswith("o_c") and "_t" in f]
    assert keys, "golden file carries tiled outputs"
    for key in keys:
        causal = int(key[3])
        bm, bn = (int(x) for x in key.split("_t")[1].split("x"))
        o_ref, lse_ref = z[key], z["lse" + key[1:]]
        o_c, lse_c = c_oracle.attention_tiled(q, k, v, bm, bn, is_causal=bool(causal), scale=scale)
        o_n, lse_n = tiled_online_softmax_reference(q, k, v, is_causal=bool(causal), scale=scale,
                                                    block_m=bm, block_n=bn)
        assert max_abs(o_c, o_ref) < 1e-13 and max_abs(lse_c, lse_ref) < 1e-12
        assert max_abs(o_n, o_ref) < TOL64 and max_abs(lse_n, lse_ref) < TOL64


# ------------------------------------------------------------------------------------------------
# 2. closed form
# ------------------------------------------------------------------------------------------------
def test_closed_form_2x2(c_oracle):
    """q = k = I2, v = [[1,2],[3,4]], scale 1: S = I2, so row 0 = softmax([1,0]) and
    row 1 = softmax([0,1]); causal row 0 sees key 0 only (o0 = v0, lse0 = 1)."""
    e = math.e
    q = np.eye(2).reshape(1, 1, 2, 2)
    v = np.array([[1.0, 2.0], [3.0, 4.0]]).reshape(1, 1, 2, 2)
    full = np.array([[(e + 3) / (1 + e), (2 * e + 4) / (1 + e)],
                     [(1 + 3 * e) / (1 + e), (2 + 4 * e) / (1 + e)]])
    for fn in (lambda c: math_reference(q, q, v, is_causal=c, scale=1.0),
               lambda c: c_oracle.attention(q, q, v, is_causal=c, scale=1.0),
               lambda c: tiled_online_softmax_reference(q, q, v, is_causal=c, scale=1.0,
                                                        block_m=1, block_n=1)):
        o, lse = fn(False)
        assert max_abs(o[0, 0], full) < 1e-14
        assert max_abs(lse[0, 0], [math.log(1 + e)] * 2) < 1e-14
        o, lse = fn(True)
        assert max_abs(o[0, 0, 0], [1.0, 2.0]) < 1e-15 and abs(lse[0, 0, 0] - 1.0) < 1e-15
        assert max_abs(o[0, 0, 1], full[1]) < 1e-14
    z = np.load(GOLDEN / "closed_form_2x2.npz", allow_pickle=False)
    assert max_abs(z["o_c0"][0, 0], full) < 1e-14 and abs(z["lse_c1"][0, 0, 0] - 1.0) < 1e-15


# ------------------------------------------------------------------------------------------------
# 3. torch SDPA MATH fp64
# ------------------------------------------------------------------------------------------------
def sdpa64(q, k, v, causal, scale=None, attn_mask=None):
    import torch.nn.functional as F
    from torch.nn.attention import SDPBackend, sdpa_kernel

    tq, tk, tv = (torch.from_numpy(x) for x in (q, k, v))
    with sdpa_kernel([SDPBackend.MATH]):
        return F.scaled_dot_product_attention(
            tq, tk, tv, attn_mask=None if attn_mask is None else torch.from_numpy(attn_mask),
            is_causal=causal, scale=default_scale(q.shape[-1]) if scale is None else scale,
            enable_gqa=k.shape[1] != q.shape[1]).numpy()


@pytest.mark.parametrize("causal", [False, True], ids=["full", "causal"])
@pytest.mark.parametrize("n,d", [(64, 64), (128, 128), (256, 64)])
def test_oracles_match_sdpa_math_fp64(n, d, causal, c_oracle):
    q, k, v = qkv64(2, 2, n, d, seed=1)
    ref = sdpa64(q, k, v, causal)
    assert max_abs(math_reference(q, k, v, is_causal=causal)[0], ref) < TOL64
    assert max_abs(c_oracle.attention(q, k, v, is_causal=causal)[0], ref) < TOL64
    assert max_abs(tiled_online_softmax_reference(q, k, v, is_causal=causal, block_m=32,
                                                  block_n=32)[0], ref) < TOL64


def test_gqa_heads_match_sdpa_enable_gqa(c_oracle):
    q, k, v = qkv64(1, 4, 64, 64, hkv=2)
    ref = sdpa64(q, k, v, True)
    assert max_abs(math_reference(q, k, v, is_causal=True)[0], ref) < TOL64
    assert max_abs(c_oracle.attention(q, k, v, is_causal=True)[0], ref) < TOL64
    assert max_abs(tiled_online_softmax_reference(q, k, v, is_causal=True, block_m=16,
                                                  block_n=16)[0], ref) < TOL64


# ------------------------------------------------------------------------------------------------
# 4. invariants
# ------------------------------------------------------------------------------------------------
@pytest.mark.parametrize("causal", [False, True], ids=["full", "causal"])
@pytest.mark.parametrize("bm,bn", [(128, 128), (32, 64), (16, 16), (64, 8), (1, 7), (96, 512)])
def test_tiled_equals_direct_any_tiling(bm, bn, causal, c_oracle):
    q, k, v = qkv64(1, 2, 128, 64, seed=2)
    o_ref, lse_ref = math_reference(q, k, v, is_causal=causal)
    o, lse = tiled_online_softmax_reference(q, k, v, is_causal=causal, block_m=bm, block_n=bn)
    assert max_abs(o, o_ref) < TOL64 and max_abs(lse, lse_ref) < TOL64
    o, lse = c_oracle.attention_tiled(q, k, v, bm, bn, is_causal=causal)
    assert max_abs(o, o_ref) < TOL64 and max_abs(lse, lse_ref) < TOL64


def test_causal_block_skipping_is_exact():
    q, k, v = qkv64(1, 2, 128, 64)
    a = tiled_online_softmax_reference(q, k, v, is_causal=True, block_m=32, block_n=16)
    b = tiled_online_softmax_reference(q, k, v, is_causal=True, block_m=32, block_n=16,
                                       skip_masked_blocks=False)
    assert np.array_equal(a[0], b[0]) and np.array_equal(a[1], b[1])


@pytest.mark.parametrize("causal", [False, True], ids=["full", "causal"])
@pytest.mark.parametrize("scale", [None, 0.37])
def test_lse_equals_logsumexp(causal, scale, c_oracle):
    n, d = 128, 64
    q, k, v = qkv64(1, 2, n, d, seed=3)
    s = torch.from_numpy(q @ np.swapaxes(k, -1, -2)) * (default_scale(d) if scale is None else scale)
    if causal:
        s = s.masked_fill(~torch.ones(n, n, dtype=torch.bool).tril(), float("-inf"))
    lse_t = torch.logsumexp(s, dim=-1).numpy()
    assert max_abs(math_reference(q, k, v, is_causal=causal, scale=scale)[1], lse_t) < TOL64
    assert max_abs(c_oracle.attention(q, k, v, is_causal=causal, scale=scale)[1], lse_t) < TOL64
    # LSE is a real logsumexp: the probabilities it implies sum to one.
    assert max_abs(torch.exp(s - torch.from_numpy(lse_t)[..., None]).sum(-1).numpy(), 1.0) < 1e-12


def test_scale_folding_and_scale_matters(c_oracle):
    q, k, v = qkv64(1, 2, 128, 128, seed=4)
    o1, l1 = c_oracle.attention(q, k, v, scale=0.05)
    o2, l2 = c_oracle.attention(2 * q, k, v, scale=0.025)
    assert max_abs(o1, o2) < 1e-13 and max_abs(l1, l2) < 1e-12
    assert max_abs(o1, c_oracle.attention(q, k, v)[0]) > 1e-3
    x = np.linspace(-30.0, 5.0, 101)
    assert max_abs(np.exp2(x * 0.05 * LOG2E), np.exp(x * 0.05)) < 1e-14


def test_causal_equals_explicit_tril_mask(c_oracle):
    n = 128
    q, k, v = qkv64(1, 2, n, 64, seed=5)
    tril = np.tril(np.ones((n, n), dtype=bool))
    o_c, lse_c = math_reference(q, k, v, is_causal=True)
    o_m, lse_m = math_reference(q, k, v, attn_mask=tril)
    assert np.array_equal(o_c, o_m) and np.array_equal(lse_c, lse_m)
    assert max_abs(o_c, sdpa64(q, k, v, False, attn_mask=tril)) < TOL64
    assert max_abs(c_oracle.attention(q, k, v, is_causal=True)[0], o_c) < TOL64
    assert max_abs(o_c[:, :, 0, :], v[:, :, 0, :]) < TOL64  # row 0 sees key 0 only


def test_rows_subset_matches_full(c_oracle):
    q, k, v = qkv64(2, 4, 96, 64, seed=6, hkv=2)
    o, lse = math_reference(q, k, v, is_causal=True)
    rows = np.array([0, 1, 31, 32, 95])
    o_r, lse_r = math_reference_rows(q, k, v, 1, 3, rows, is_causal=True)
    assert max_abs(o_r, o[1, 3, rows]) < TOL64 and max_abs(lse_r, lse[1, 3, rows]) < TOL64
    o_c, lse_c = c_oracle.attention_rows(q, k, v, 1, 3, 5, 7, is_causal=True)
    assert max_abs(o_c, o[1, 3, 5:12]) < TOL64 and max_abs(lse_c, lse[1, 3, 5:12]) < TOL64


def test_fully_masked_row_guards_never_nan():
    n, bn = 64, 16
    q, k, v = qkv64(1, 2, n, 64, seed=7)
    keep = np.ones((n, n), dtype=bool)
    keep[5, :] = False     # fully masked row: l == 0 at the end
    keep[7, :bn] = False   # first key tile masked: m == -inf after tile 0
    keep[9, bn:] = False   # everything after tile 0 masked
    o_m, lse_m = math_reference(q, k, v, attn_mask=keep)
    o_t, lse_t = tiled_online_softmax_reference(q, k, v, attn_mask=keep, block_m=16, block_n=bn)
    for o, lse in ((o_m, lse_m), (o_t, lse_t)):
        assert not np.isnan(o).any() and not np.isnan(lse).any()
        assert np.array_equal(o[:, :, 5, :], np.zeros_like(o[:, :, 5, :]))
        assert np.isposinf(lse[:, :, 5]).all()
        assert np.isfinite(o[:, :, [7, 9], :]).all() and np.isfinite(lse[:, :, [7, 9]]).all()
    assert max_abs(o_t, o_m) < TOL64
    ref = sdpa64(q, k, v, False, attn_mask=keep)
    assert max_abs(o_t[:, :, [7, 9], :], ref[:, :, [7, 9], :]) < TOL64


def test_error_ratio_rule():
    rng = np.random.default_rng(6)
    ref = rng.standard_normal((2, 2, 32, 64))
    noise = rng.standard_normal(ref.shape)
    torch_same = ref + 1e-3 * noise
    good = error_ratio(ref + 1e-3 * noise[::-1], ref, torch_same)
    assert good.ok and good.out_finite and good.torch_finite
    assert good.bound == pytest.approx(2 * good.err_torch + 1e-6)
    assert not error_ratio(ref + 1e-2 * noise, ref, torch_same).ok
    bad = ref.copy()
    bad[0, 0, 0, 0] = np.nan
    assert not error_ratio(bad, ref, torch_same).out_finite
    tn = torch_same.copy()
    tn[0, 0, 0, 0] = np.inf
    r = error_ratio(ref, ref, tn)
    assert not r.torch_finite and not r.ok
    # torch's own unfused fp32 attention passes its own rule with a tiny error.
    q, k, v = qkv64(1, 2, 128, 64, seed=7)
    pt = unfused_reference(*(torch.from_numpy(x).float() for x in (q, k, v)), is_causal=True)
    assert pt.dtype == torch.float32
    self_check = error_ratio(pt, math_reference(q, k, v, is_causal=True)[0], pt)
    assert self_check.ok and self_check.err_torch < 1e-5


def test_multithreaded_c_oracle_is_bitwise_single_threaded(c_oracle):
    q, k, v = qkv64(2, 3, 64, 64, seed=8, hkv=1)
    a = c_oracle.attention(q, k, v, is_causal=True)
    b = c_oracle.attention(q, k, v, is_causal=True, threads=4)
    assert np.array_equal(a[0], b[0]) and np.array_equal(a[1], b[1])


def _tiled_with_bug(q, k, v, bug: str, block_m: int, block_n: int):
    """Private copy of the recurrence with ONE step removed (a planted mistake, CPU only).
    no_acc_rescale: acc = acc + p v ; no_l_rescale: l = l + sum p."""
    b, h, n, d = q.shape
    c = default_scale(d) * LOG2E
    o = np.empty_like(q)
    for i0 in range(0, n, block_m):
        qt = q[:, :, i0:i0 + block_m]
        m = np.full(qt.shape[:3] + (1,), -np.inf)
        l_row = np.zeros_like(m)
        acc = np.zeros_like(qt)
        for j0 in range(0, n, block_n):
            s = qt @ np.swapaxes(k[:, :, j0:j0 + block_n], -1, -2)
            m_new = np.maximum(m, s.max(-1, keepdims=True))
            alpha = np.exp2((m - m_new) * c)
            p = np.exp2((s - m_new) * c)
            l_row = (l_row if bug == "no_l_rescale" else alpha * l_row) + p.sum(-1, keepdims=True)
            acc = (acc if bug == "no_acc_rescale" else alpha * acc) + p @ v[:, :, j0:j0 + block_n]
            m = m_new
        o[:, :, i0:i0 + block_m] = acc / l_row
    return o


@pytest.mark.parametrize("bug", ["no_acc_rescale", "no_l_rescale"])
def test_rescale_bug_is_caught_by_tile_invariance(bug):
    """Teeth (ref:tests/test_reference_cpu.py:258-302): invisible with one key tile per row,
    wrong by a wide margin with four."""
    n = 128
    q, k, v = qkv64(1, 2, n, 64, seed=9)
    o_ref, _ = math_reference(q, k, v)
    assert max_abs(_tiled_with_bug(q, k, v, bug, 32, n), o_ref) < TOL64
    assert max_abs(_tiled_with_bug(q, k, v, bug, 32, n // 4), o_ref) > 1e-3
    assert max_abs(tiled_online_softmax_reference(q, k, v, block_m=32, block_n=n // 4)[0],
                   o_ref) < TOL64


# ------------------------------------------------------------------------------------------------
# 5. live reference oracle
# ------------------------------------------------------------------------------------------------
@pytest.mark.skipif(not RefOracle.available(), reason="oracle/_ref not built (no /root/reference)")
@pytest.mark.parametrize("causal", [False, True], ids=["full", "causal"])
@pytest.mark.parametrize("b,h,hkv,n,d", [(1, 3, 1, 96, 64), (2, 2, 2, 160, 128)])
def test_c_oracle_matches_live_reference(b, h, hkv, n, d, causal, c_oracle):
    q, k, v = qkv64(b, h, n, d, seed=10 + n, hkv=hkv)
    ref = RefOracle()
    o_r, lse_r = ref.attention(q, k, v, is_causal=causal, scale=0.11)
    o_c, lse_c = c_oracle.attention(q, k, v, is_causal=causal, scale=0.11)
    assert max_abs(o_c, o_r) < 1e-13 and max_abs(lse_c, lse_r) < 1e-12
    o_h, lse_h = ref.attention_heads(q, k, v, 1, b * h - 1, is_causal=causal, scale=0.11,
                                     threads=3)
    assert np.array_equal(o_h, o_r.reshape(b * h, n, d)[1:])
    assert np.array_equal(lse_h, lse_r.reshape(b * h, n)[1:])


def test_reference_ctest_passes():
    """The reference's own oracle test binary (ref:src/reference/test_cpu_reference.cpp, its ctest
    target ref:CMakeLists.txt:33-37), built from the reference's sources by ``make -C oracle ref``:
    it must pass here too, so the oracle the golden vectors came from is the tested one."""
    import subprocess

    root = Path(__file__).resolve().parents[1]
    exe = root / "oracle" / "_ref" / "test_cpu_reference"
    if Path("/root/reference/src/reference/test_cpu_reference.cpp").exists():
        cmd = ["make", "-s", "-C", str(root / "oracle"), "ref-check"]  # builds, then runs it
    elif exe.exists():
        cmd = [str(exe)]  # a tree without the reference sources: the binary built earlier
    else:
        pytest.skip("the reference sources are absent and oracle/_ref was not built")
    res = subprocess.run(cmd, capture_output=True, text=True, timeout=300)
    assert res.returncode == 0, res.stdout[-2000:] + res.stderr[-2000:]
    assert "PASS" in res.stdout, res.stdout[-2000:]
