"""GPU parity tests for every implemented stage (marker ``gpu``), mirroring
ref:tests/test_kernels_gpu.py case by case.

Each stage runs through ``torch.ops.fused_attn.forward_stage`` (the binding calls the C-ABI
``fa_forward`` of libfa_hip.so) and is judged against the fp64 CPU oracle on the same seeded inputs
with the reference's ratio rule + caps and the build's tighter stated tolerance (tests/_checks.py).
Stages this build does not implement (1, 2) must raise "not implemented".
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

import fused_attn
from fused_attn import capi
from _checks import ABS_CAP, LSE_ATOL, LSE_TOL_REF, O_TOL, assert_close_tol, \
    assert_every_head_close, check_against_reference
from oracle.oracle import error_ratio, math_reference, unfused_reference

pytestmark = pytest.mark.gpu

STAGES = [1, 2, 3, 4, 5]
LSE_STAGES = [3, 4, 5]
STAGE_DTYPES = {
    3: [torch.float32, torch.float16],
    4: [torch.float16, torch.bfloat16],
    5: [torch.float16, torch.bfloat16],
}
STAGE_DTYPE_PAIRS = [(s, dt) for s in (3, 4, 5) for dt in STAGE_DTYPES[s]]
# Instantiated (BR, BC) tiles per stage (csrc/attn_mfma16.h and csrc/attn_kernel.h tables;
# 0 = default). Stages 3 and 4 fix BR at 128 and ignore a forced BR, as the reference's S3/S4 do.
STAGE_BC = {3: {32, 64}, 4: {32, 64, 128}}
S5_TILES = {(32, 32), (32, 64), (32, 128), (32, 256), (64, 32), (64, 64), (64, 128), (64, 256),
            (128, 32), (128, 64), (128, 128), (256, 64)}
S5_DEFAULT = (128, 128)  # at D = 64, the head dim of the tile tests

_ids = {torch.float32: "fp32", torch.float16: "fp16", torch.bfloat16: "bf16"}


def _pair_id(p):
    return str(p) if isinstance(p, int) else _ids[p]


def require(stage: int, dtype: torch.dtype, head_dim: int) -> None:
    """Fails when the extension is missing (the HIP path must be what runs); skips a
    (stage, dtype, D) this build does not implement."""
    assert fused_attn.is_available(), "fused_attn._C is not built"
    built = fused_attn.impl_supports(stage, dtype, head_dim)
    if not built:
        pytest.skip(f"stage {stage} is not built for {_ids[dtype]} D={head_dim}")


def tile_supported(stage: int, bm: int, bn: int) -> bool:
    if stage == 5:
        return (bm or S5_DEFAULT[0], bn or S5_DEFAULT[1]) in S5_TILES
    return bn == 0 or bn in STAGE_BC[stage]


@pytest.fixture
def reset_overrides():
    yield
    if fused_attn.is_available():
        fused_attn.set_debug_overrides(0, 0)


# ------------------------------------------------------------------------------------------------
@pytest.mark.parametrize("causal", [False, True], ids=["full", "causal"])
@pytest.mark.parametrize("stage,dtype", STAGE_DTYPE_PAIRS, ids=_pair_id)
def test_matches_fp64_reference(stage, dtype, causal, gpu_shape, make_qkv):
    b, h, n, d = gpu_shape
    require(stage, dtype, d)
    q, k, v = make_qkv(b, h, n, d, dtype=dtype, device="cuda")
    o, lse = fused_attn.forward_stage(q, k, v, stage, is_causal=causal)
    assert o.shape == q.shape and o.dtype == dtype and o.is_contiguous()
    assert tuple(lse.shape) == (b, h, n) and lse.dtype == torch.float32
    check_against_reference(o, q, k, v, causal, dtype, lse=lse)


# Stage 5 runs every key tile through its steady step when all tiles are full (non-causal, N a
# multiple of BC); the last two steps then load clamped tiles into buffers nobody reads again.
# These short problems run BC = 64 at both head dims, so the lengths give 1 to 10 full tiles (odd
# and even counts, so the unrolled-by-two loop ends on either parity) plus one ragged length.
@pytest.mark.parametrize("n,d", [(128, 64), (192, 64), (320, 64), (640, 64), (64, 128),
                                 (192, 128), (320, 128), (160, 128)],
                         ids=lambda x: str(x))
@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16], ids=_pair_id)
def test_stage5_full_tile_counts(n, d, dtype, make_qkv):
    require(5, dtype, d)
    q, k, v = make_qkv(1, 3, n, d, dtype=dtype, device="cuda")
    o, lse = fused_attn.forward_stage(q, k, v, 5, is_causal=False)
    check_against_reference(o, q, k, v, False, dtype, lse=lse)


# Stage 5 picks its workgroup height from the grid when no BR is forced: the tallest of 128 / 64 /
# 32 rows that still gives every compute unit a workgroup. Each 32-row wave runs the same key split
# and key order at every height, so the default must equal every forced height that keeps the
# default width bit for bit (fa_s5_plan names the width a forced height gets: a height with no tile
# of the default width, such as BR 128 beside a four-split default, takes another width and is
# checked against the oracle instead). The shapes are small grids (the default is BR 32 or 64
# there) with N an odd multiple of 32, so the forced BR = 64 / 128 runs also cover partial query
# tiles.
@pytest.mark.parametrize("causal", [False, True], ids=["full", "causal"])
@pytest.mark.parametrize("b,h,n,d", [(1, 3, 96, 64), (2, 4, 224, 64), (1, 16, 512, 128),
                                     (2, 3, 352, 128)], ids=lambda x: str(x))
@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16], ids=_pair_id)
def test_stage5_default_height_matches_forced_heights(b, h, n, d, dtype, causal, make_qkv,
                                                      reset_overrides):
    require(5, dtype, d)
    q, k, v = make_qkv(b, h, n, d, dtype=dtype, device="cuda", seed=5)
    code = capi.DTYPE_CODES[dtype]
    p = capi.params(b, h, h, n, d, d ** -0.5, causal)
    fused_attn.set_debug_overrides(0, 0)
    _, bc0, _ = capi.s5_plan(code, p)
    o0, lse0 = fused_attn.forward_stage(q, k, v, 5, is_causal=causal)
    check_against_reference(o0, q, k, v, causal, dtype, lse=lse0)
    same_width = 0
    for br in (128, 64, 32):
        fused_attn.set_debug_overrides(br, 0)
        assert capi.s5_plan(code, p)[0] == br
        bc = capi.s5_plan(code, p)[1]
        o, lse = fused_attn.forward_stage(q, k, v, 5, is_causal=causal)
        torch.cuda.synchronize()
        if bc == bc0:
            same_width += 1
            assert torch.equal(o, o0) and torch.equal(lse, lse0), \
                f"BR = {br} (BC {bc}) differs from the default"
        else:
            check_against_reference(o, q, k, v, causal, dtype, lse=lse)
    fused_attn.set_debug_overrides(0, 0)
    assert same_width >= 2, "fewer than two heights keep the default width"


# The tile stage 5 picks by itself on grids that fill a 256-CU device (csrc/dispatch.cpp,
# auto_bc_s5 / auto_br_s5): narrow tiles where several workgroups share a CU, except for causal
# long walks at D = 128 with fewer than three BR-128 workgroups per CU (grids issued tile-major,
# B * H a multiple of 8). The height never changes results, so the comparison with the forced tile
# pins the width; the forced tile names the height the rules pick too.
@pytest.mark.parametrize("b,h,n,d,dtype,causal,tile", [
    (8, 32, 1024, 64, torch.float16, False, (256, 64)),     # D = 64 dense, 4 rounds of BR 256
    (8, 12, 1024, 64, torch.float16, False, (128, 32)),     # 1.5 rounds of BR 256: tall
    (8, 12, 1024, 64, torch.float16, True, (128, 32)),      # GPT-2 attention, rotated (3 MB)
    (3, 8, 2048, 64, torch.float16, True, (64, 64)),        # D = 64 causal, 1.5 BR-128 per CU
    (2, 16, 4096, 64, torch.float16, True, (256, 64)),      # D = 64 causal N 4096, 2 rounds
    (4, 32, 512, 128, torch.float16, False, (128, 32)),     # D = 128, 2 per CU
    (4, 32, 512, 128, torch.bfloat16, True, (64, 32)),      # short causal walks
    (2, 8, 4096, 128, torch.float16, True, (128, 64)),      # causal long walks, 2 per CU
    (8, 12, 1024, 128, torch.float16, True, (128, 32)),     # causal, 3 per CU, tile-major
    (1, 16, 8192, 128, torch.bfloat16, True, (128, 32)),    # LONG: causal, 4 per CU
    (2, 8, 2048, 64, torch.float16, True, (64, 128)),       # C64 causal: halved height
    (2, 8, 2048, 128, torch.float16, True, (64, 64)),       # C128 causal: halved height
    (2, 4, 4096, 64, torch.float16, False, (128, 128)),     # D = 64 long walks, 1 per CU: wide
    (8, 8, 2048, 64, torch.float16, False, (256, 64)),      # 2 rounds of BR 256
    (8, 8, 2048, 64, torch.bfloat16, False, (256, 64)),     # same grid, bf16
], ids=["d64-wide256", "d64-tall-dense", "d64-gpt2-causal", "d64-narrow", "d64-wide256-causal",
        "d128-dense", "d128-short-causal", "d128-causal-2cu", "d128-causal-3cu", "long",
        "c64-causal", "c128-causal", "d64-long-walk", "d64-fp16-wide256", "d64-bf16-wide256"])
def test_stage5_automatic_tile_on_full_grids(b, h, n, d, dtype, causal, tile, make_qkv,
                                             reset_overrides):
    require(5, dtype, d)
    if torch.cuda.get_device_properties(0).multi_processor_count != 256:
        pytest.skip("the expected tiles are those of a 256-CU device")
    q, k, v = make_qkv(b, h, n, d, dtype=dtype, device="cuda", seed=9)
    fused_attn.set_debug_overrides(0, 0)
    o0, lse0 = fused_attn.forward_stage(q, k, v, 5, is_causal=causal)
    fused_attn.set_debug_overrides(*tile)
    o, lse = fused_attn.forward_stage(q, k, v, 5, is_causal=causal)
    fused_attn.set_debug_overrides(0, 0)
    torch.cuda.synchronize()
    assert torch.equal(o, o0) and torch.equal(lse, lse0), f"the default is not {tile}"
    head = (slice(0, 1), slice(0, 1))
    check_against_reference(o0[head].contiguous(), q[head].contiguous(), k[head].contiguous(),
                            v[head].contiguous(), causal, dtype, lse=lse0[head].contiguous())
    # Every head of the grid against the fp32 reference: a tile rule that mixed up heads,
    # query tiles or key splits anywhere would show here.
    assert_every_head_close(o0, lse0, q, k, v, causal, d ** -0.5, what=f"tile {tile}")


# The D = 64 rule tiles on ragged grids: N = 1056 and 4128 leave a partial last query tile (32 of
# 256 or 128 rows) and a partial last key tile, with and without GQA. The 256-row tile (dense, whole rounds
# of 256-row workgroups) and the tall 128 x 32 tile (rotated where the K/V per XCD fit 4 MB) are
# the automatic tiles here; every head is checked against the fp32 reference.
@pytest.mark.parametrize("b,h,hkv,n,dtype,causal,tile", [
    (16, 16, 16, 1056, torch.float16, False, (256, 64)),   # 5 rounds of BR 256
    (16, 16, 4, 1056, torch.bfloat16, False, (256, 64)),   # GQA, 4 query heads per kv head
    (8, 12, 12, 1056, torch.float16, True, (128, 32)),     # tall, causal, rotated (3.1 MB)
    (8, 12, 4, 1056, torch.bfloat16, False, (128, 32)),    # tall, dense GQA (1.9 rounds of 256)
    (2, 16, 16, 4128, torch.float16, True, (256, 64)),     # causal 256-row tile, 32-row last tile
    (2, 16, 4, 4128, torch.bfloat16, True, (256, 64)),     # the same with GQA, bf16
], ids=["wide256", "wide256-gqa", "tall-causal", "tall-gqa", "wide256-causal",
        "wide256-causal-gqa"])
def test_stage5_d64_rule_tiles_on_ragged_grids(b, h, hkv, n, dtype, causal, tile, make_qkv,
                                               reset_overrides):
    require(5, dtype, 64)
    if torch.cuda.get_device_properties(0).multi_processor_count != 256:
        pytest.skip("the expected tiles are those of a 256-CU device")
    fused_attn.set_debug_overrides(0, 0)
    p = capi.params(b, h, hkv, n, 64, 0.125, causal)
    assert capi.s5_plan(capi.DTYPE_CODES[dtype], p)[:2] == tile
    q, k, v = make_qkv(b, h, n, 64, dtype=dtype, device="cuda", hkv=hkv, seed=23)
    o, lse = fused_attn.forward_stage(q, k, v, 5, is_causal=causal)
    torch.cuda.synchronize()
    assert_every_head_close(o, lse, q, k, v, causal, 0.125, what=f"tile {tile}")


# Grids of at most one workgroup per CU whose two-split tile would leave a SIMD with one wave take
# the tile of twice the width and twice the waves at the same height: four key splits of 32 keys
# (D = 128) or 64 keys (D = 64) per row group. Compared with the forced tile bit for bit, every head
# against the fp32 reference, and with the two-split tile of the same height within twice the bar.
@pytest.mark.parametrize("b,h,n,d,dtype,causal,tile,two", [
    (1, 16, 512, 128, torch.bfloat16, True, (32, 128), (32, 64)),    # LONG_N512
    (1, 16, 1024, 128, torch.bfloat16, True, (64, 128), (64, 64)),   # LONG_N1024
    (1, 16, 1024, 128, torch.bfloat16, False, (64, 128), (64, 64)),  # LONG_ring8
    (1, 8, 2048, 64, torch.float16, False, (64, 256), (64, 128)),    # D = 64
    (2, 1, 2048, 64, torch.float16, True, (32, 256), (32, 128)),     # C64 / 8 GPUs, causal
    (1, 3, 544, 128, torch.float16, True, (32, 128), (32, 64)),      # ragged last key tile
], ids=["long-n512", "long-n1024", "ring8", "d64", "d64-causal-heads", "ragged"])
def test_stage5_four_split_tile_on_small_grids(b, h, n, d, dtype, causal, tile, two, make_qkv,
                                              reset_overrides):
    require(5, dtype, d)
    if torch.cuda.get_device_properties(0).multi_processor_count != 256:
        pytest.skip("the expected tiles are those of a 256-CU device")
    p = capi.params(b, h, h, n, d, d ** -0.5, causal)
    fused_attn.set_debug_overrides(0, 0)
    assert capi.s5_plan(capi.DTYPE_CODES[dtype], p)[:2] == tile
    q, k, v = make_qkv(b, h, n, d, dtype=dtype, device="cuda", seed=13)
    o0, lse0 = fused_attn.forward_stage(q, k, v, 5, is_causal=causal)
    fused_attn.set_debug_overrides(*tile)
    o, lse = fused_attn.forward_stage(q, k, v, 5, is_causal=causal)
    fused_attn.set_debug_overrides(*two)
    o2, _ = fused_attn.forward_stage(q, k, v, 5, is_causal=causal)
    fused_attn.set_debug_overrides(0, 0)
    torch.cuda.synchronize()
    assert torch.equal(o, o0) and torch.equal(lse, lse0), f"the default is not {tile}"
    assert_every_head_close(o0, lse0, q, k, v, causal, d ** -0.5, what=f"tile {tile}")
    atol, rtol = O_TOL[dtype]
    base = o2.double()
    excess = float(((o0.double() - base).abs() - 2 * (atol + rtol * base.abs())).max())
    assert excess <= 0.0, f"four splits differ from two by more than twice the bar ({excess})"


@pytest.mark.parametrize("stage", [1, 2])
def test_unbuilt_stages_raise_not_implemented(stage, make_qkv):
    if not fused_attn.is_available():
        pytest.fail("fused_attn._C is not built")
    assert not fused_attn.impl_supports(stage, torch.float32, 64)
    q, k, v = make_qkv(1, 2, 64, 64, device="cuda")
    with pytest.raises(RuntimeError, match="not implemented"):
        fused_attn.forward_stage(q, k, v, stage)


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16],
                         ids=lambda d: _ids[d])
@pytest.mark.parametrize("d", [64, 128])
def test_forward_dispatches_to_best_stage(dtype, d, make_qkv):
    if not fused_attn.is_available():
        pytest.fail("fused_attn._C is not built")
    supported = [s for s in STAGES if fused_attn.impl_supports(s, dtype, d)]
    assert supported, "every dtype has a stage on gfx950"
    best = max(supported)
    assert best == (3 if dtype == torch.float32 else 5)
    q, k, v = make_qkv(1, 2, 256, d, dtype=dtype, device="cuda")
    o = fused_attn.forward(q, k, v, is_causal=True)
    o_best, _ = fused_attn.forward_stage(q, k, v, best, is_causal=True)
    assert torch.equal(o, o_best), f"forward() did not dispatch to stage {best}"
    check_against_reference(o, q, k, v, True, dtype)


# ------------------------------------------------------------------------------------------------
@pytest.mark.parametrize("n", [128, 256])
@pytest.mark.parametrize("causal", [False, True], ids=["full", "causal"])
@pytest.mark.parametrize("stage,dtype", STAGE_DTYPE_PAIRS, ids=_pair_id)
def test_tile_invariance(stage, dtype, causal, n, make_qkv, reset_overrides):
    """The rescale path only runs when a row spans several key tiles: the same problem with the
    default tiles and with BC in {N/2, N/4} (and BR = N/4) must pass and agree
    (ref:tests/test_kernels_gpu.py:114-134; N is doubled so every tile is an instantiated one)."""
    d = 64
    require(stage, dtype, d)
    q, k, v = make_qkv(2, 2, n, d, dtype=dtype, device="cuda", seed=11)
    outs = {}
    for bm, bn in [(0, 0), (0, n // 2), (0, n // 4), (n // 4, n // 4)]:
        if not tile_supported(stage, bm, bn):
            continue
        fused_attn.set_debug_overrides(bm, bn)
        o, lse = fused_attn.forward_stage(q, k, v, stage, is_causal=causal)
        torch.cuda.synchronize()
        check_against_reference(o, q, k, v, causal, dtype, lse=lse)
        outs[(bm, bn)] = o.double()
    fused_attn.set_debug_overrides(0, 0)
    assert len(outs) >= 3
    base = outs[(0, 0)]
    atol, rtol = O_TOL[dtype]
    for key, o in outs.items():
        excess = float(((o - base).abs() - 2 * (atol + rtol * base.abs())).max())
        assert excess <= 0.0, f"tiles {key} differ from the default tiling by more than 2x the bar"


@pytest.mark.parametrize("stage,dtype", STAGE_DTYPE_PAIRS, ids=_pair_id)
def test_uninstantiated_tile_is_an_error_not_a_fault(stage, dtype, make_qkv, reset_overrides):
    require(stage, dtype, 64)
    q, k, v = make_qkv(1, 2, 256, 64, dtype=dtype, device="cuda")
    fused_attn.set_debug_overrides(0, 48)
    with pytest.raises(RuntimeError, match="failed"):
        fused_attn.forward_stage(q, k, v, stage)


# ------------------------------------------------------------------------------------------------
@pytest.mark.parametrize("stage,dtype", STAGE_DTYPE_PAIRS, ids=_pair_id)
def test_determinism_50_runs_bitwise_equal(stage, dtype, make_qkv):
    """No atomics, no uninitialised LDS, no order that depends on scheduling: 50 launches of the
    same causal problem (B2 H4 N256 D64, the reference's determinism case) are identical."""
    require(stage, dtype, 64)
    q, k, v = make_qkv(2, 4, 256, 64, dtype=dtype, device="cuda", seed=12)
    runs = [fused_attn.forward_stage(q, k, v, stage, is_causal=True) for _ in range(50)]
    o0, lse0 = runs[0]
    differing = [i for i, (o, lse) in enumerate(runs) if not (torch.equal(o, o0) and
                                                              torch.equal(lse, lse0))]
    assert not differing, f"launches {differing} differ from launch 0"


# ------------------------------------------------------------------------------------------------
@pytest.mark.parametrize("factor", [1e2, 1e-3], ids=["x1e2", "x1e-3"])
@pytest.mark.parametrize("stage,dtype",
                         [p for p in STAGE_DTYPE_PAIRS if p[1] != torch.float32], ids=_pair_id)
def test_half_precision_dynamic_range(stage, dtype, factor, make_qkv):
    """Inputs scaled by 1e2 make raw scores of ~1e5, beyond fp16's range and beyond exp() in fp32
    without the running-max subtraction; scaled by 1e-3 they make near-uniform rows (the cases
    of ref:tests/test_kernels_gpu.py:150-172)."""
    require(stage, dtype, 64)
    q, k, v = make_qkv(1, 2, 256, 64, dtype=dtype, device="cuda", seed=13, scale_inputs=factor)
    o, lse = fused_attn.forward_stage(q, k, v, stage)
    assert bool(torch.isfinite(o).all() and torch.isfinite(lse).all()), \
        "overflow: scores, max, sum and accumulator must stay in fp32"
    ref64, _ = math_reference(q, k, v)
    verdict = error_ratio(o, ref64, unfused_reference(q, k, v))
    if verdict.torch_finite:  # torch's own fp16 attention overflows at x1e2 on some rows
        assert verdict.ok, f"ratio rule: {verdict}"
    peak = max(float(abs(ref64).max()), 1e-30)
    assert verdict.err_mine / peak <= ABS_CAP[dtype], f"relative error past the cap: {verdict}"
    if factor < 1.0:
        # The stated tolerance is checked at the small end. At x1e2 the scores' own fp32 sums
        # carry ~1e-2 of absolute error (in every kernel, the reference's included), so only the
        # relative cap applies there.
        assert_close_tol(o, ref64, *O_TOL[dtype])


# ------------------------------------------------------------------------------------------------
@pytest.mark.parametrize("stage", [3, 4, 5])
def test_n_not_multiple_of_32_raises(stage, make_qkv):
    dtype = torch.float32 if stage == 3 else torch.float16
    require(stage, dtype, 64)
    q, k, v = make_qkv(1, 1, 100, 64, dtype=dtype, device="cuda")
    with pytest.raises(RuntimeError, match="multiple of 32"):
        fused_attn.forward_stage(q, k, v, stage)
    with pytest.raises(RuntimeError, match="multiple of 32"):
        fused_attn.forward(q, k, v)


def _misaligned(t):
    """t's values in a buffer that starts 4 bytes past a 16-byte boundary (fp32)."""
    store = torch.empty(t.numel() + 8, dtype=t.dtype, device=t.device)
    view = store[1:1 + t.numel()].view(t.shape)
    view.copy_(t)
    return view


# (case, how to make (q, k, v, stage) bad from good fp32 operands, message the op must give).
# The messages are the reference op's (ref:tests/test_kernels_gpu.py:177-214).
_BAD_CALLS = [
    ("cpu operands", lambda q, k, v: (q.cpu(), k.cpu(), v.cpu(), None), "CUDA"),
    ("non-contiguous q", lambda q, k, v: (q.transpose(2, 3).contiguous().transpose(2, 3), k, v,
                                          None), "contiguous"),
    ("mixed dtypes", lambda q, k, v: (q, k.half(), v, None), "dtype"),
    ("D = 32", lambda q, k, v: (q[..., :32].contiguous(), k[..., :32].contiguous(),
                                v[..., :32].contiguous(), None), "D must be 64 or 128"),
    ("stage 0", lambda q, k, v: (q, k, v, 0), r"stage must be in 1\.\.5"),
    ("stage 6", lambda q, k, v: (q, k, v, 6), r"stage must be in 1\.\.5"),
    ("Nkv != Nq", lambda q, k, v: (q, k[:, :, :32].contiguous(), v[:, :, :32].contiguous(), None),
     "Nq == Nkv"),
    ("H not a multiple of Hkv", lambda q, k, v: (q[:, :1].contiguous(), k, v, None),
     "multiple of Hkv"),
    ("q not 16-byte aligned", lambda q, k, v: (_misaligned(q), k, v, None), "16-byte aligned"),
]


@pytest.mark.parametrize("case,make_bad,message", _BAD_CALLS, ids=[c[0] for c in _BAD_CALLS])
def test_input_validation_messages(case, make_bad, message, make_qkv):
    assert fused_attn.is_available(), "fused_attn._C is not built"
    q, k, v, stage = make_bad(*make_qkv(1, 2, 64, 64, dtype=torch.float32, device="cuda"))
    with pytest.raises(RuntimeError, match=message):
        if stage is None:
            fused_attn.forward(q, k, v)
        else:
            fused_attn.forward_stage(q, k, v, stage)


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16],
                         ids=lambda d: _ids[d])
@pytest.mark.parametrize("stage", STAGES)
def test_stage_dtype_pairs_run_or_raise_not_implemented(stage, dtype, make_qkv):
    """Every (stage, dtype) pair either runs (impl_supports says it is built: the call returns
    finite outputs of the right shape) or raises "not implemented" (the reference's message for
    an unbuilt pair, ref:python/fused_attn/ext.cpp:166-167)."""
    assert fused_attn.is_available(), "fused_attn._C is not built"
    q, k, v = make_qkv(1, 2, 64, 64, dtype=dtype, device="cuda")
    if fused_attn.impl_supports(stage, dtype, 64):
        o, lse = fused_attn.forward_stage(q, k, v, stage)
        torch.cuda.synchronize()
        assert o.shape == q.shape and o.dtype == q.dtype and lse.shape == (1, 2, 64)
        assert torch.isfinite(o).all() and torch.isfinite(lse).all()
        return
    with pytest.raises(RuntimeError, match="not implemented"):
        fused_attn.forward_stage(q, k, v, stage)


# ------------------------------------------------------------------------------------------------
@pytest.mark.parametrize("stage,dtype", STAGE_DTYPE_PAIRS, ids=_pair_id)
def test_causal_equals_explicit_tril_mask(stage, dtype, make_qkv):
    """is_causal must be the top-left mask: the oracle is run with an explicit lower-triangular
    boolean mask (key j visible from query i iff j <= i), so j < i, bottom-right alignment or a
    diagonal-block slip all fail; query row 0 sees key 0 only, so its output is v[0]."""
    require(stage, dtype, 64)
    n = 512
    q, k, v = make_qkv(1, 2, n, 64, dtype=dtype, device="cuda", seed=14)
    visible = np.tri(n, n, dtype=bool)
    o, _ = fused_attn.forward_stage(q, k, v, stage, is_causal=True)
    check_against_reference(o, q, k, v, False, dtype, attn_mask=visible)
    first_row_err = (o[:, :, 0].double() - v[:, :, 0].double()).abs().max().item()
    assert first_row_err <= ABS_CAP[dtype], f"row 0 is not v[0]: {first_row_err:.3e}"


@pytest.mark.parametrize("scale", [0.05, 0.25])
@pytest.mark.parametrize("stage,dtype", STAGE_DTYPE_PAIRS, ids=_pair_id)
def test_non_default_scale(stage, dtype, scale, make_qkv):
    d = 128
    require(stage, dtype, d)
    q, k, v = make_qkv(1, 2, 256, d, dtype=dtype, device="cuda", seed=15)
    o, lse = fused_attn.forward_stage(q, k, v, stage, is_causal=False, scale=scale)
    check_against_reference(o, q, k, v, False, dtype, scale=scale, lse=lse)


# ------------------------------------------------------------------------------------------------
@pytest.mark.parametrize("causal", [False, True], ids=["full", "causal"])
@pytest.mark.parametrize("stage,dtype", STAGE_DTYPE_PAIRS, ids=_pair_id)
def test_lse_matches_fp64(stage, dtype, causal, gpu_shape, make_qkv):
    """The row log-sum-exp (natural log of sum_j exp(scale q.k_j)) against the fp64 oracle, to the
    stated 1e-3 and to the reference's own per-dtype tolerance."""
    b, h, n, d = gpu_shape
    require(stage, dtype, d)
    q, k, v = make_qkv(b, h, n, d, dtype=dtype, device="cuda", seed=16)
    _, lse = fused_attn.forward_stage(q, k, v, stage, is_causal=causal)
    _, lse64 = math_reference(q, k, v, is_causal=causal)
    assert (tuple(lse.shape), lse.dtype) == ((b, h, n), torch.float32)
    assert bool(torch.isfinite(lse).all())
    assert_close_tol(lse, lse64, LSE_ATOL, 0.0, what="LSE")
    ref_atol, ref_rtol = LSE_TOL_REF[dtype]
    assert_close_tol(lse, lse64, ref_atol, ref_rtol, what="LSE (reference tolerance)")


# ------------------------------------------------------------------------------------------------
@pytest.mark.parametrize("hkv", [1, 2])
@pytest.mark.parametrize("stage,dtype", STAGE_DTYPE_PAIRS, ids=_pair_id)
def test_gqa_heads(stage, dtype, hkv, make_qkv):
    """GQA/MQA: query head h reads kv head h // (H // Hkv). An xfail in the reference
    (ref:tests/test_kernels_gpu.py:261-268); implemented by every stage here."""
    d = 64
    require(stage, dtype, d)
    q, k, v = make_qkv(1, 4, 256, d, dtype=dtype, device="cuda", hkv=hkv, seed=17)
    o, lse = fused_attn.forward_stage(q, k, v, stage, is_causal=True)
    check_against_reference(o, q, k, v, True, dtype, lse=lse)
