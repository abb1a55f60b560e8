"""The GPT-2-small block harness (ref:bench/gpt_block.py:53-158) runs its attention through the fused op
(marker ``gpu``): the strided call inside the block equals the dense call bitwise, the block's
attention matches an fp32 torch computation of the same attention, and the timing helper runs."""

from __future__ import annotations

import math

import pytest
import torch

import fused_attn
from fused_attn import gpt_block

pytestmark = pytest.mark.gpu


def require_ext():
    if not fused_attn.is_available():
        pytest.fail("fused_attn._C is not built: the HIP path must be the one that runs")


def test_strided_and_dense_fused_blocks_agree_bitwise():
    require_ext()
    idx = gpt_block.token_ids(2, 512, seed=1)
    with torch.no_grad():
        y_strided = gpt_block.build("fused", seed=3)(idx)
        y_dense = gpt_block.build("fused_dense", seed=3)(idx)
    torch.cuda.synchronize()
    assert torch.equal(y_strided, y_dense)


@pytest.mark.parametrize("batch", [2, 8], ids=["b2", "b8-config5"])
def test_block_attention_matches_fp32_attention(batch):
    """The attention output inside the block (fp16 kernel) against fp32 torch attention on the
    same q, k, v, to the fp16 bar of the dense parity tests; batch 8 is the benchmark's timed
    GPT-2-small block (T 1024, 12 heads of 64)."""
    require_ext()
    model = gpt_block.build("fused", seed=4)
    attn = model.block.attn
    idx = gpt_block.token_ids(batch, 1024, seed=2)
    with torch.no_grad():
        x = model.block.ln_1(model.wte(idx) + model.wpe(torch.arange(1024, device="cuda")))
        qkv = attn.c_attn(x)
        b, t, c = x.shape
        h, d = attn.n_head, c // attn.n_head
        q, k, v = (qkv[..., i * c:(i + 1) * c].view(b, t, h, d).transpose(1, 2) for i in range(3))
        o = attn.attn(q, k, v)
        qf, kf, vf = (z.float() for z in (q, k, v))
        s = torch.matmul(qf, kf.transpose(-1, -2).contiguous()) / math.sqrt(d)
        s = s.masked_fill(~torch.ones(t, t, dtype=torch.bool, device="cuda").tril(), float("-inf"))
        ref = torch.matmul(torch.softmax(s, dim=-1), vf)
    err = (o.float() - ref).abs()
    assert float((err - (2e-3 + 2e-3 * ref.abs())).max()) <= 0.0, float(err.max())


def test_fused_and_sdpa_blocks_are_close():
    require_ext()
    idx = gpt_block.token_ids(1, 256, seed=5)
    with torch.no_grad():
        y_f = gpt_block.build("fused", seed=6)(idx).float()
        y_s = gpt_block.build("sdpa", seed=6)(idx).float()
    assert float((y_f - y_s).abs().max()) < 5e-2


def test_measure_reports_tokens_per_second():
    require_ext()
    model = gpt_block.build("fused", seed=7)
    res = gpt_block.measure(model, gpt_block.token_ids(2, 256, seed=7), warmup=2, iters=5)
    assert res["tokens_per_s"] > 0 and 0 < res["attn_share"] < 1
