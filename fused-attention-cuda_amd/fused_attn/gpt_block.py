"""GPT-2-small decoder block with a swappable attention call, and its tokens/s measurement.

This is the end-to-end consumer of the op, restating the reference's nanoGPT block check
(ref:bench/gpt_block.py:53-158), the reference's GPT-2-small block benchmark:
- token + position embedding (wte 50257 x 768, wpe 1024 x 768);
- LayerNorm -> causal self-attention (12 heads of 64) -> residual;
- LayerNorm -> MLP (768 -> 3072 -> 768, GELU) -> residual;
- fp16, random init, inference.

The reference feeds ``randn`` activations straight into the block (ref:bench/gpt_block.py:191).
Config 5 asks for random token ids in [0, 50257) through an embedding, which is what
``GPTBlock`` adds in front.

Attention callables (``attention_fn``), each given q, k, v as [B, H, T, D] views of the c_attn
output and returning [B, H, T, D]:
- ``"fused"``: ``fused_attn.forward_strided`` on the views, no copy in or out. The output is
  dense in [B, T, H, D] order, so the caller's transpose back is free.
- ``"fused_dense"``: ``fused_attn.forward`` after ``.contiguous()`` on q, k, v. This is the
  reference's binding cost (ref:bench/gpt_block.py:130-135), timed on purpose.
- ``"sdpa"``: ``torch.nn.functional.scaled_dot_product_attention`` (the ROCm backend torch
  picks).

``measure`` follows the reference's warm protocol: warm-up, then one event pair per iteration
around the block and one around the attention window, one synchronize, medians.
"""

from __future__ import annotations

import math
from collections.abc import Callable

import torch
import torch.nn as nn
import torch.nn.functional as F

VOCAB = 50257
N_POS = 1024

AttnFn = Callable[[torch.Tensor, torch.Tensor, torch.Tensor], torch.Tensor]


def attention_fn(kind: str, scale: float) -> AttnFn:
    """The causal attention callable ``kind`` in {"fused", "fused_dense", "sdpa"}."""
    if kind == "fused":
        import fused_attn

        return lambda q, k, v: fused_attn.forward_strided(q, k, v, is_causal=True, scale=scale)
    if kind == "fused_dense":
        import fused_attn

        return lambda q, k, v: torch.ops.fused_attn.forward(q.contiguous(), k.contiguous(),
                                                            v.contiguous(), True, scale)
    if kind == "sdpa":
        return lambda q, k, v: F.scaled_dot_product_attention(q, k, v, is_causal=True,
                                                              scale=scale)
    raise ValueError(f"unknown attention kind {kind!r}")


class CausalSelfAttention(nn.Module):
    """Fused QKV projection, head split as views, the attention call, output projection. An event
    pair around the attention window (layout work included) is kept per call when timing."""

    def __init__(self, n_embd: int, n_head: int, attn: AttnFn):
        super().__init__()
        self.c_attn = nn.Linear(n_embd, 3 * n_embd)
        self.c_proj = nn.Linear(n_embd, n_embd)
        self.n_head = n_head
        self.attn = attn
        self.timing = False
        self.windows: list[tuple[torch.cuda.Event, torch.cuda.Event]] = []

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        b, t, c = x.shape
        h, d = self.n_head, c // self.n_head
        qkv = self.c_attn(x)
        if self.timing:
            t0, t1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            t0.record()
        # [B, T, 3C] -> three [B, H, T, D] views (strides T*3C, D, 3C, 1): no data movement.
        q, k, v = (qkv[..., i * c:(i + 1) * c].view(b, t, h, d).transpose(1, 2) for i in range(3))
        y = self.attn(q, k, v).transpose(1, 2).reshape(b, t, c)
        if self.timing:
            t1.record()
            self.windows.append((t0, t1))
        return self.c_proj(y)


class Block(nn.Module):
    def __init__(self, n_embd: int, n_head: int, attn: AttnFn):
        super().__init__()
        self.ln_1 = nn.LayerNorm(n_embd)
        self.attn = CausalSelfAttention(n_embd, n_head, attn)
        self.ln_2 = nn.LayerNorm(n_embd)
        self.mlp = nn.Sequential(nn.Linear(n_embd, 4 * n_embd), nn.GELU(),
                                 nn.Linear(4 * n_embd, n_embd))

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        x = x + self.attn(self.ln_1(x))
        return x + self.mlp(self.ln_2(x))


class GPTBlock(nn.Module):
    """Embedding (token + position) followed by one decoder block."""

    def __init__(self, n_embd: int = 768, n_head: int = 12, attn: AttnFn | None = None):
        super().__init__()
        scale = 1.0 / math.sqrt(n_embd // n_head)
        self.wte = nn.Embedding(VOCAB, n_embd)
        self.wpe = nn.Embedding(N_POS, n_embd)
        self.block = Block(n_embd, n_head, attn or attention_fn("fused", scale))

    def forward(self, idx: torch.Tensor) -> torch.Tensor:
        t = idx.shape[1]
        pos = torch.arange(t, device=idx.device)
        return self.block(self.wte(idx) + self.wpe(pos))


def build(kind: str, n_embd: int = 768, n_head: int = 12, dtype=torch.float16, seed: int = 0,
          device: str = "cuda") -> GPTBlock:
    """A random-init GPTBlock with attention ``kind`` (the same weights for every kind at one
    seed)."""
    torch.manual_seed(seed)
    model = GPTBlock(n_embd, n_head, attention_fn(kind, 1.0 / math.sqrt(n_embd // n_head)))
    return model.to(device, dtype).eval()


def token_ids(batch: int = 8, seq: int = 1024, seed: int = 0, device: str = "cuda"):
    """Random token ids in [0, 50257) (the GPT-2 vocabulary)."""
    gen = torch.Generator(device="cpu").manual_seed(seed)
    return torch.randint(0, VOCAB, (batch, seq), generator=gen).to(device)


def measure(model: GPTBlock, idx: torch.Tensor, warmup: int = 10, iters: int = 50) -> dict:
    """Warm timing: median block ms (embedding included), median attention-window ms, tokens/s."""
    attn = model.block.attn
    with torch.no_grad():
        for _ in range(warmup):
            model(idx)
        torch.cuda.synchronize()
        attn.windows.clear()
        attn.timing = True
        starts = [torch.cuda.Event(enable_timing=True) for _ in range(iters)]
        ends = [torch.cuda.Event(enable_timing=True) for _ in range(iters)]
        for i in range(iters):
            starts[i].record()
            model(idx)
            ends[i].record()
        torch.cuda.synchronize()
        attn.timing = False
    block_ms = sorted(a.elapsed_time(b) for a, b in zip(starts, ends))
    attn_ms = sorted(a.elapsed_time(b) for a, b in attn.windows)
    blk, att = block_ms[len(block_ms) // 2], attn_ms[len(attn_ms) // 2]
    b, t = idx.shape
    return {"tokens_per_s": b * t / (blk * 1e-3), "block_ms": blk, "attn_ms": att,
            "attn_share": att / blk, "iters": iters, "warmup": warmup}
