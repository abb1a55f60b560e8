"""fp64 CPU oracle for the fused SDPA forward -- TEST INFRASTRUCTURE.

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline`` leg may import this
module, and only as the checker (or the timed CPU baseline). The product (``fused_attn``,
``libfa_hip.so``) never imports it; the op fails loudly when its HIP extension is missing instead
of falling back to anything here.

Restatements (numpy, float64), each following the reference's own model:

* :func:`math_reference` -- explicit softmax attention returning ``(o, lse)``
  (ref:python/fused_attn/reference.py:116-145, ref:src/reference/cpu_reference.cpp:47-92).
* :func:`math_reference_rows` -- the same for a subset of query rows of one head, for spot checks at
  full benchmark sizes (the reference harness checks selected rows the same way,
  ref:bench/bench_main.cu:589-655).
* :func:`tiled_online_softmax_reference` -- the online-softmax recurrence of the fused kernels
  (ref:python/fused_attn/reference.py:181-285, ref:src/reference/cpu_reference.cpp:94-165).
* :func:`unfused_reference` -- naive attention in the *input* dtype (torch, CPU), the "what torch
  itself gets wrong" term of the ratio rule (ref:python/fused_attn/reference.py:288-311).
* :func:`error_ratio` -- the FlashAttention ratio rule (ref:python/fused_attn/reference.py:331-352).
* :class:`COracle` -- ctypes binding of ``oracle/liboracle.so`` (the C restatement,
  ``attn_oracle.c``); :class:`RefOracle` -- ctypes binding of ``oracle/_ref/libfa_ref.so``, the
  reference's own ``cpu_reference.cpp`` built by ``oracle/Makefile``.

Pinning (tests/test_oracle_cpu.py): golden vectors written by the reference's own compiled oracle,
the 2x2 closed form, torch SDPA MATH fp64, tiled == direct, scale folding, LSE == logsumexp, the
fully-masked-row guards, and a deliberately broken recurrence that the tile test must catch.

Conventions: ``[B, H, N, D]`` layouts, ``k``/``v`` may carry ``Hkv`` heads (query head ``h`` reads kv
head ``h // (H // Hkv)``), top-left causal (``j <= i``), default scale ``1/sqrt(D)``,
``lse = +inf`` for a row with no visible key.
"""

from __future__ import annotations

import ctypes
import math
from pathlib import Path
from typing import NamedTuple

import numpy as np

ORACLE_DIR = Path(__file__).resolve().parent
LOG2E = 1.4426950408889634

__all__ = [
    "LOG2E",
    "COracle",
    "RatioResult",
    "RefOracle",
    "combine_splits",
    "decode_keep_mask",
    "decode_reference",
    "default_scale",
    "error_ratio",
    "keep_mask",
    "math_reference",
    "math_reference_rows",
    "tiled_online_softmax_reference",
    "to_f64",
    "unfused_reference",
]


def default_scale(head_dim: int) -> float:
    """PyTorch's SDPA default scale ``1/sqrt(D)`` (ref:python/fused_attn/reference.py:55-57)."""
    return 1.0 / math.sqrt(head_dim)


def to_f64(x) -> np.ndarray:
    """numpy float64 copy of an ndarray or a (CPU or device) torch tensor of any float dtype."""
    if isinstance(x, np.ndarray):
        return x.astype(np.float64, copy=False)
    import torch  # local: the numpy path must not need torch

    assert isinstance(x, torch.Tensor)
    return x.detach().to("cpu", torch.float64).numpy()


def _expand_kv(q: np.ndarray, k: np.ndarray, v: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
    """Broadcast Hkv kv heads to H query heads: head h reads kv head h // (H // Hkv)
    (ref:python/fused_attn/reference.py:60-74, ref:src/reference/cpu_reference.cpp:26-28)."""
    h, hkv = q.shape[1], k.shape[1]
    if hkv == h:
        return k, v
    if h % hkv != 0:
        raise ValueError(f"H={h} must be a multiple of Hkv={hkv}")
    rep = h // hkv
    return np.repeat(k, rep, axis=1), np.repeat(v, rep, axis=1)


def keep_mask(n_q: int, n_kv: int, is_causal: bool, attn_mask=None) -> np.ndarray | None:
    """Boolean "attend" mask (True = keep), top-left causal: query i sees keys j <= i
    (ref:python/fused_attn/reference.py:77-100). ``attn_mask`` exists only to drive the guards."""
    keep = None
    if is_causal:
        keep = np.tril(np.ones((n_q, n_kv), dtype=bool))
    if attn_mask is not None:
        am = np.asarray(to_f64(attn_mask) if not isinstance(attn_mask, np.ndarray) else attn_mask)
        if am.dtype != bool:
            am = am.astype(bool)
        keep = am if keep is None else (keep & am)
    return keep


def _prep(q, k, v, scale):
    q64, k64, v64 = to_f64(q), to_f64(k), to_f64(v)
    if q64.ndim != 4 or k64.ndim != 4 or v64.ndim != 4:
        raise ValueError("q, k, v must be [B, H, N, D]")
    k64, v64 = _expand_kv(q64, k64, v64)
    return q64, k64, v64, float(default_scale(q64.shape[-1]) if scale is None else scale)


def math_reference(q, k, v, is_causal: bool = False, scale: float | None = None, attn_mask=None):
    """Explicit fp64 softmax attention -> ``(o, lse)`` float64 numpy arrays.

    Materialised scaled scores, one global row max, exp, sum, ``o = (p @ v) / l``,
    ``lse = m + ln l``; guards: a fully masked row gives o = 0 and lse = +inf
    (ref:python/fused_attn/reference.py:116-145)."""
    q64, k64, v64, scale = _prep(q, k, v, scale)
    s = np.matmul(q64, np.swapaxes(k64, -1, -2)) * scale
    keep = keep_mask(q64.shape[2], k64.shape[2], is_causal, attn_mask)
    if keep is not None:
        s = np.where(keep, s, -np.inf)
    m = s.max(axis=-1, keepdims=True)
    m_safe = np.where(np.isneginf(m), 0.0, m)
    p = np.exp(s - m_safe)
    l_row = p.sum(axis=-1, keepdims=True)
    with np.errstate(divide="ignore"):
        inv_l = np.where(l_row == 0, 0.0, 1.0 / np.where(l_row == 0, 1.0, l_row))
        lse = np.where(l_row == 0, np.inf, m_safe + np.log(np.where(l_row == 0, 1.0, l_row)))
    o = np.matmul(p, v64) * inv_l
    return o, lse[..., 0]


def decode_keep_mask(n_q: int, n_kv: int, is_causal: bool) -> np.ndarray | None:
    """Keep mask of split-KV decode: the n_q new tokens are the last positions of the sequence,
    so with ``is_causal`` token i sees keys j <= n_kv - n_q + i (bottom-right alignment, what a KV
    cache means); without it every token sees every key. For n_q == n_kv this is the top-left
    mask of :func:`keep_mask`. There is no reference implementation (decode is the reference's
    stated next step, ref:README.md:1357-1358); the tests pin this against torch SDPA MATH with
    torch's own ``tril`` mask and brute-force loops."""
    if not is_causal:
        return None
    return np.tril(np.ones((n_q, n_kv), dtype=bool), k=n_kv - n_q)


def decode_reference(q, k, v, is_causal: bool = False, scale: float | None = None):
    """fp64 split-KV decode answer: q [B, H, Nq, D] against k, v [B, Hkv, Nkv, D] with the
    bottom-right mask -> ``(o, lse)``; rows with no visible key give o = 0, lse = +inf."""
    nq, nkv = q.shape[2], k.shape[2]
    return math_reference(q, k, v, is_causal=False, scale=scale,
                          attn_mask=decode_keep_mask(nq, nkv, is_causal))


def combine_splits(o_parts, lse_parts):
    """LSE-weighted combine of per-split partials (ref:docs/RESEARCH.md:151-156):
    O = sum_s e^(L_s - L*) O_s / sum_s e^(L_s - L*), L = L* + ln sum_s e^(L_s - L*), L* = max_s L_s.
    ``o_parts`` [S, ..., D], ``lse_parts`` [S, ...]; an empty split carries L_s = -inf and weight
    0; a row whose splits are all empty gives O = 0 and L = +inf."""
    o_parts = np.asarray(o_parts, dtype=np.float64)
    lse_parts = np.asarray(lse_parts, dtype=np.float64)
    lmax = lse_parts.max(axis=0)
    lmax_safe = np.where(np.isneginf(lmax), 0.0, lmax)
    w = np.exp(lse_parts - lmax_safe)
    wsum = w.sum(axis=0)
    with np.errstate(divide="ignore", invalid="ignore"):
        o = np.where(wsum[..., None] > 0, (w[..., None] * o_parts).sum(axis=0) / wsum[..., None],
                     0.0)
        lse = np.where(wsum > 0, lmax_safe + np.log(np.where(wsum > 0, wsum, 1.0)), np.inf)
    return o, lse


def math_reference_rows(q, k, v, b: int, h: int, rows, is_causal: bool = False,
                        scale: float | None = None):
    """``math_reference`` for query rows ``rows`` (1-D int array) of head (b, h) only.

    Cost is O(len(rows) * N * D): this is what makes full-size spot checks cheap (the reference's
    own harness checks the first/last Q tile of two heads, ref:bench/bench_main.cu:589-655).
    Returns ``(o[len(rows), D], lse[len(rows)])`` float64."""
    rows = np.asarray(rows, dtype=np.int64)
    hq, hkv = q.shape[1], k.shape[1]
    hk = h // (hq // hkv)
    qr = to_f64(q[b, h][rows] if isinstance(q, np.ndarray) else q[b, h, rows])
    kk = to_f64(k[b, hk])
    vv = to_f64(v[b, hk])
    d = qr.shape[-1]
    scale = float(default_scale(d) if scale is None else scale)
    s = (qr @ kk.T) * scale
    if is_causal:
        s = np.where(np.arange(kk.shape[0])[None, :] <= rows[:, None], s, -np.inf)
    m = s.max(axis=-1, keepdims=True)
    p = np.exp(s - m)
    l_row = p.sum(axis=-1, keepdims=True)
    return (p @ vv) / l_row, (m + np.log(l_row))[:, 0]


def tiled_online_softmax_reference(q, k, v, is_causal: bool = False, scale: float | None = None,
                                   block_m: int = 64, block_n: int = 64, attn_mask=None,
                                   skip_masked_blocks: bool = True):
    """The online-softmax recurrence of the fused kernels, in fp64.

    Per query tile: raw-score running max ``m``, ``c = scale*log2(e)``,
    ``alpha = exp2((m_old - m_new) c)``, ``p = exp2((s - m_new) c)``, ``l = alpha l + sum p``,
    ``acc = alpha acc + p v``; deferred ``o = acc / l``; ``lse = m scale + ln l``; causal key tiles
    wholly above the diagonal skipped before any load (ref:python/fused_attn/reference.py:181-285).
    """
    q64, k64, v64, scale = _prep(q, k, v, scale)
    if block_m <= 0 or block_n <= 0:
        raise ValueError("block_m and block_n must be positive")
    b, h, n_q, d = q64.shape
    n_kv = k64.shape[2]
    c = scale * LOG2E
    keep = keep_mask(n_q, n_kv, is_causal, attn_mask)
    o = np.empty_like(q64)
    lse = np.empty((b, h, n_q), dtype=np.float64)
    for i0 in range(0, n_q, block_m):
        i1 = min(i0 + block_m, n_q)
        qt = q64[:, :, i0:i1, :]
        m = np.full((b, h, i1 - i0, 1), -np.inf)
        l_row = np.zeros((b, h, i1 - i0, 1))
        acc = np.zeros((b, h, i1 - i0, d))
        for j0 in range(0, n_kv, block_n):
            j1 = min(j0 + block_n, n_kv)
            if is_causal and skip_masked_blocks and j0 > i1 - 1:
                continue
            s = np.matmul(qt, np.swapaxes(k64[:, :, j0:j1, :], -1, -2))  # raw, unscaled
            if keep is not None:
                blk = keep[i0:i1, j0:j1]
                if not blk.all():
                    s = np.where(blk, s, -np.inf)
            m_new = np.maximum(m, s.max(axis=-1, keepdims=True))
            m_safe = np.where(np.isneginf(m_new), 0.0, m_new)
            alpha = np.exp2((m - m_safe) * c)
            p = np.exp2((s - m_safe) * c)
            l_row = alpha * l_row + p.sum(axis=-1, keepdims=True)
            acc = alpha * acc + np.matmul(p, v64[:, :, j0:j1, :])
            m = m_new
        with np.errstate(divide="ignore", invalid="ignore"):
            inv_l = np.where(l_row == 0, 0.0, 1.0 / np.where(l_row == 0, 1.0, l_row))
            lse_t = np.where(l_row == 0, np.inf,
                             m * scale + np.log(np.where(l_row == 0, 1.0, l_row)))
        o[:, :, i0:i1, :] = acc * inv_l
        lse[:, :, i0:i1] = lse_t[..., 0]
    return o, lse


def unfused_reference(q, k, v, is_causal: bool = False, scale: float | None = None,
                      attn_mask=None, device: str = "cpu"):
    """Naive torch attention in the *input* dtype (ref:python/fused_attn/reference.py:288-311:
    scale q, matmul, softmax, matmul, all in the input dtype). Computed on ``device`` and returned
    there. Half-precision inputs are always computed on the CPU (batched 16-bit products on the
    device are not something this checker relies on); fp32 may run on the device, as the
    reference's tests do."""
    import torch

    if q.dtype in (torch.float16, torch.bfloat16):
        device = "cpu"
    q, k, v = (t.detach().to(device) for t in (q, k, v))
    hq, hkv = q.shape[1], k.shape[1]
    if hkv != hq:
        k = k.repeat_interleave(hq // hkv, dim=1)
        v = v.repeat_interleave(hq // hkv, dim=1)
    scale = float(default_scale(q.shape[-1]) if scale is None else scale)
    s = torch.matmul(q * scale, k.transpose(-1, -2).contiguous())
    keep = keep_mask(q.shape[2], k.shape[2], is_causal, attn_mask)
    if keep is not None:
        s = s.masked_fill(~torch.from_numpy(keep).to(s.device), float("-inf"))
    return torch.matmul(torch.softmax(s, dim=-1), v)


class RatioResult(NamedTuple):
    """Outcome of the ratio rule (ref:python/fused_attn/reference.py:314-328)."""

    err_mine: float
    err_torch: float
    bound: float
    ok: bool
    out_finite: bool
    torch_finite: bool

    def __str__(self) -> str:  # pragma: no cover - formatting only
        return (f"err_mine={self.err_mine:.3e} err_torch={self.err_torch:.3e} "
                f"bound={self.bound:.3e} ok={self.ok} out_finite={self.out_finite} "
                f"torch_finite={self.torch_finite}")


def error_ratio(out, ref64, torch_same_dtype) -> RatioResult:
    """``err_mine <= 2 * err_torch + 1e-6`` with both errors max-abs against the fp64 oracle
    (ref:python/fused_attn/reference.py:331-352)."""
    out64, r64, t64 = to_f64(out), to_f64(ref64), to_f64(torch_same_dtype)
    with np.errstate(invalid="ignore"):
        err_mine = float(np.max(np.abs(out64 - r64)))
        err_torch = float(np.max(np.abs(t64 - r64)))
    bound = 2.0 * err_torch + 1e-6
    out_finite = bool(np.isfinite(out64).all())
    torch_finite = math.isfinite(err_torch)
    ok = out_finite and torch_finite and err_mine <= bound
    return RatioResult(err_mine, err_torch, bound, ok, out_finite, torch_finite)


# ------------------------------------------------------------------------------------------------
# ctypes bindings of the two compiled oracles
# ------------------------------------------------------------------------------------------------
_dp = ctypes.POINTER(ctypes.c_double)


class _Shape(ctypes.Structure):
    _fields_ = [("B", ctypes.c_int), ("H", ctypes.c_int), ("Hkv", ctypes.c_int),
                ("N", ctypes.c_int), ("D", ctypes.c_int), ("scale", ctypes.c_double),
                ("causal", ctypes.c_int)]


def _c64(x) -> np.ndarray:
    return np.ascontiguousarray(to_f64(x))


def _ptr(a: np.ndarray):
    return a.ctypes.data_as(_dp)


class COracle:
    """``oracle/liboracle.so``: this repo's C restatement (attn_oracle.c)."""

    def __init__(self, path: Path | None = None):
        path = path or ORACLE_DIR / "liboracle.so"
        if not path.exists():
            raise FileNotFoundError(f"{path} is not built (run `make -C oracle`)")
        self.lib = ctypes.CDLL(str(path))
        sp = ctypes.POINTER(_Shape)
        self.lib.fao_attention.argtypes = [_dp, _dp, _dp, sp, _dp, _dp]
        self.lib.fao_attention_rows.argtypes = [_dp, _dp, _dp, sp, ctypes.c_int, ctypes.c_int,
                                                ctypes.c_int, ctypes.c_int, _dp, _dp]
        self.lib.fao_attention_tiled.argtypes = [_dp, _dp, _dp, sp, ctypes.c_int, ctypes.c_int,
                                                 _dp, _dp]
        self.lib.fao_attention_mt.argtypes = [_dp, _dp, _dp, sp, _dp, _dp, ctypes.c_int]
        self.lib.fao_attention_mt.restype = ctypes.c_int

    @staticmethod
    def _shape(q, k, scale, causal) -> _Shape:
        b, h, n, d = q.shape
        scale = default_scale(d) if scale is None else scale
        return _Shape(b, h, k.shape[1], n, d, float(scale), int(bool(causal)))

    def attention(self, q, k, v, is_causal=False, scale=None, threads: int = 1):
        q, k, v = _c64(q), _c64(k), _c64(v)
        s = self._shape(q, k, scale, is_causal)
        o = np.empty_like(q)
        lse = np.empty(q.shape[:3])
        if threads > 1:
            rc = self.lib.fao_attention_mt(_ptr(q), _ptr(k), _ptr(v), ctypes.byref(s), _ptr(o),
                                           _ptr(lse), int(threads))
            if rc != 0:
                raise RuntimeError("fao_attention_mt: thread start failed")
        else:
            self.lib.fao_attention(_ptr(q), _ptr(k), _ptr(v), ctypes.byref(s), _ptr(o), _ptr(lse))
        return o, lse

    def attention_rows(self, q, k, v, b, h, row0, rows, is_causal=False, scale=None):
        q, k, v = _c64(q), _c64(k), _c64(v)
        s = self._shape(q, k, scale, is_causal)
        o = np.empty((rows, q.shape[-1]))
        lse = np.empty(rows)
        self.lib.fao_attention_rows(_ptr(q), _ptr(k), _ptr(v), ctypes.byref(s), b, h, row0, rows,
                                    _ptr(o), _ptr(lse))
        return o, lse

    def attention_tiled(self, q, k, v, block_m, block_n, is_causal=False, scale=None):
        q, k, v = _c64(q), _c64(k), _c64(v)
        s = self._shape(q, k, scale, is_causal)
        o = np.empty_like(q)
        lse = np.empty(q.shape[:3])
        self.lib.fao_attention_tiled(_ptr(q), _ptr(k), _ptr(v), ctypes.byref(s), block_m, block_n,
                                     _ptr(o), _ptr(lse))
        return o, lse


class RefOracle:
    """``oracle/_ref/libfa_ref.so``: the reference's own ``fa::ref`` oracle
    (ref:src/reference/cpu_reference.cpp), compiled from its sources by ``make -C oracle ref``."""

    PATH = ORACLE_DIR / "_ref" / "libfa_ref.so"

    @classmethod
    def available(cls) -> bool:
        return cls.PATH.exists()

    def __init__(self):
        if not self.PATH.exists():
            raise FileNotFoundError(f"{self.PATH} is not built (run `make -C oracle ref`)")
        self.lib = ctypes.CDLL(str(self.PATH))
        i = ctypes.c_int
        head = [_dp, _dp, _dp, i, i, i, i, i, ctypes.c_double, i]
        self.lib.faref_attention.argtypes = head + [_dp, _dp]
        self.lib.faref_attention_rows.argtypes = head + [i, i, i, i, _dp, _dp]
        self.lib.faref_attention_tiled.argtypes = head + [i, i, _dp, _dp]
        self.lib.faref_attention_heads_mt.argtypes = head + [i, i, _dp, _dp, i]

    @staticmethod
    def _dims(q, k, scale, causal):
        b, h, n, d = q.shape
        scale = default_scale(d) if scale is None else scale
        return (b, h, k.shape[1], n, d, float(scale), int(bool(causal)))

    def attention(self, q, k, v, is_causal=False, scale=None):
        q, k, v = _c64(q), _c64(k), _c64(v)
        o = np.empty_like(q)
        lse = np.empty(q.shape[:3])
        self.lib.faref_attention(_ptr(q), _ptr(k), _ptr(v), *self._dims(q, k, scale, is_causal),
                                 _ptr(o), _ptr(lse))
        return o, lse

    def attention_tiled(self, q, k, v, block_m, block_n, is_causal=False, scale=None):
        q, k, v = _c64(q), _c64(k), _c64(v)
        o = np.empty_like(q)
        lse = np.empty(q.shape[:3])
        self.lib.faref_attention_tiled(_ptr(q), _ptr(k), _ptr(v),
                                       *self._dims(q, k, scale, is_causal), block_m, block_n,
                                       _ptr(o), _ptr(lse))
        return o, lse

    def attention_heads(self, q, k, v, head0, nheads, is_causal=False, scale=None, threads=1):
        """Heads [head0, head0+nheads) of the flattened B*H axis, on `threads` threads."""
        q, k, v = _c64(q), _c64(k), _c64(v)
        n, d = q.shape[2], q.shape[3]
        o = np.empty((nheads, n, d))
        lse = np.empty((nheads, n))
        self.lib.faref_attention_heads_mt(_ptr(q), _ptr(k), _ptr(v),
                                          *self._dims(q, k, scale, is_causal), head0, nheads,
                                          _ptr(o), _ptr(lse), int(threads))
        return o, lse
