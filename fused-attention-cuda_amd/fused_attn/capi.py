"""ctypes binding of ``libfa_hip.so`` -- the C-ABI of include/fa/attention.h.

This is the kind of binding any FFI consumer of the kernel library writes: plain pointers, sizes
and a POD params struct, no torch types at the boundary. The torch op (``_C``, csrc/ext.cpp) is a
C++ consumer of the same functions; tests and ``bench.py`` use this module to call the C-ABI
directly on device buffers owned by torch.

``torch`` is imported first on purpose: PyTorch-ROCm ships its own HIP runtime, and loading it
before ``libfa_hip.so`` makes the library bind to that same runtime instance (one HIP runtime per
process, so device pointers and streams from torch are valid here).
"""

from __future__ import annotations

import ctypes
from pathlib import Path

import torch

LIB_PATH = Path(__file__).resolve().parent / "libfa_hip.so"

# Codes of include/fa/attention.h (same integers as ref:include/fa/attention.cuh:17-26).
FA_DTYPE_F32, FA_DTYPE_F16, FA_DTYPE_BF16 = 0, 1, 2
FA_IMPL_NAIVE, FA_IMPL_TILED, FA_IMPL_FUSED, FA_IMPL_WMMA, FA_IMPL_TUNED = 1, 2, 3, 4, 5
HIP_SUCCESS, HIP_ERROR_INVALID_VALUE, HIP_ERROR_NOT_SUPPORTED = 0, 1, 801

DTYPE_CODES = {torch.float32: FA_DTYPE_F32, torch.float16: FA_DTYPE_F16,
               torch.bfloat16: FA_DTYPE_BF16}

# Every function include/fa/attention.h declares, in declaration order.
EXPORTS = ("fa_forward", "fa_forward_strided", "fa_workspace_bytes", "fa_impl_supports",
           "fa_set_debug_overrides", "fa_get_debug_overrides", "fa_s5_plan", "fa_impl_name", "fa_dtype_name",
           "fa_dtype_size", "fa_current_arch", "fa_error_string", "fa_decode_num_splits",
           "fa_decode_workspace_bytes", "fa_decode", "fa_decode_noalloc")

# FA_DECODE_SCRATCH_BYTES of include/fa/attention.h: the scratch behind fa_decode_noalloc.
DECODE_SCRATCH_BYTES = 17 << 20


class FaParams(ctypes.Structure):
    """``fa_params`` (include/fa/attention.h): B, H, Hkv, N, D, scale, causal."""

    _fields_ = [("B", ctypes.c_int), ("H", ctypes.c_int), ("Hkv", ctypes.c_int),
                ("N", ctypes.c_int), ("D", ctypes.c_int), ("scale", ctypes.c_float),
                ("causal", ctypes.c_bool)]


class FaStrides(ctypes.Structure):
    """``fa_strides`` (include/fa/attention.h): per batch, per head, per row, in elements."""

    _fields_ = [("b", ctypes.c_longlong), ("h", ctypes.c_longlong), ("n", ctypes.c_longlong)]


class FaDecodeParams(ctypes.Structure):
    """``fa_decode_params`` (include/fa/attention.h)."""

    _fields_ = [("B", ctypes.c_int), ("H", ctypes.c_int), ("Hkv", ctypes.c_int),
                ("Nq", ctypes.c_int), ("Nkv", ctypes.c_int), ("D", ctypes.c_int),
                ("scale", ctypes.c_float), ("causal", ctypes.c_bool),
                ("num_splits", ctypes.c_int)]


_lib: ctypes.CDLL | None = None


def load(path: Path | None = None) -> ctypes.CDLL:
    """Load ``libfa_hip.so`` once and declare every prototype of the header."""
    global _lib
    if _lib is not None and path is None:
        return _lib
    p = path or LIB_PATH
    if not p.exists():
        raise ImportError(f"{p} is not built; run `python fused-attention-cuda_amd/build.py`")
    lib = ctypes.CDLL(str(p))
    vp, ci = ctypes.c_void_p, ctypes.c_int
    lib.fa_forward.argtypes = [ci, ci, vp, vp, vp, vp, vp, vp, ctypes.POINTER(FaParams), vp]
    lib.fa_forward.restype = ci
    sp = ctypes.POINTER(FaStrides)
    lib.fa_forward_strided.argtypes = [ci, ci, vp, sp, vp, sp, vp, sp, vp, sp, vp, vp,
                                       ctypes.POINTER(FaParams), vp]
    lib.fa_forward_strided.restype = ci
    lib.fa_workspace_bytes.argtypes = [ci, ci, ctypes.POINTER(FaParams)]
    lib.fa_workspace_bytes.restype = ctypes.c_size_t
    lib.fa_impl_supports.argtypes = [ci, ci, ci, ci]
    lib.fa_impl_supports.restype = ctypes.c_bool
    lib.fa_set_debug_overrides.argtypes = [ci, ci]
    lib.fa_set_debug_overrides.restype = None
    lib.fa_get_debug_overrides.argtypes = [ctypes.c_bool, ctypes.POINTER(ci), ctypes.POINTER(ci)]
    lib.fa_get_debug_overrides.restype = None
    ip = ctypes.POINTER(ci)
    lib.fa_s5_plan.argtypes = [ci, ctypes.POINTER(FaParams), ip, ip, ip]
    lib.fa_s5_plan.restype = ci
    lib.fa_impl_name.argtypes = [ci]
    lib.fa_impl_name.restype = ctypes.c_char_p
    lib.fa_dtype_name.argtypes = [ci]
    lib.fa_dtype_name.restype = ctypes.c_char_p
    lib.fa_dtype_size.argtypes = [ci]
    lib.fa_dtype_size.restype = ctypes.c_size_t
    lib.fa_current_arch.argtypes = [ctypes.POINTER(ci)]
    lib.fa_current_arch.restype = ci
    dp = ctypes.POINTER(FaDecodeParams)
    lib.fa_decode_num_splits.argtypes = [dp]
    lib.fa_decode_num_splits.restype = ci
    lib.fa_decode_workspace_bytes.argtypes = [ci, dp]
    lib.fa_decode_workspace_bytes.restype = ctypes.c_size_t
    lib.fa_decode.argtypes = [ci, vp, vp, vp, vp, vp, vp, dp, vp]
    lib.fa_decode.restype = ci
    lib.fa_decode_noalloc.argtypes = [ci, vp, vp, vp, vp, vp, dp, vp]
    lib.fa_decode_noalloc.restype = ci
    lib.fa_error_string.argtypes = [ci]
    lib.fa_error_string.restype = ctypes.c_char_p
    if path is None:
        _lib = lib
    return lib


def params(B: int, H: int, Hkv: int, N: int, D: int, scale: float, causal: bool) -> FaParams:
    return FaParams(B, H, Hkv, N, D, float(scale), bool(causal))


def current_arch() -> int:
    a = ctypes.c_int(0)
    rc = load().fa_current_arch(ctypes.byref(a))
    if rc != HIP_SUCCESS:
        raise RuntimeError(f"fa_current_arch failed: {error_string(rc)}")
    return a.value


def s5_plan(dtype: int, p: FaParams) -> tuple[int, int, int]:
    """``fa_s5_plan``: stage 5's (BR, BC, S) for ``p`` on the current device."""
    br, bc, s = ctypes.c_int(0), ctypes.c_int(0), ctypes.c_int(0)
    rc = load().fa_s5_plan(dtype, ctypes.byref(p), ctypes.byref(br), ctypes.byref(bc),
                           ctypes.byref(s))
    if rc != HIP_SUCCESS:
        raise RuntimeError(f"fa_s5_plan failed: {error_string(rc)}")
    return br.value, bc.value, s.value


def error_string(rc: int) -> str:
    return load().fa_error_string(rc).decode()


def forward_raw(impl: int, dtype: int, q: int, k: int, v: int, o: int, lse: int, workspace: int,
                p: FaParams, stream: int) -> int:
    """``fa_forward`` on raw device addresses; returns the hipError_t value."""
    return load().fa_forward(impl, dtype, q, k, v, o, lse, workspace, ctypes.byref(p), stream)


def workspace_bytes(impl: int, q: torch.Tensor, k: torch.Tensor, is_causal: bool,
                    scale: float) -> int:
    """``fa_workspace_bytes`` for these operands (stage 5: bytes that enable split key walks)."""
    b, h, n, d = q.shape
    p = params(b, h, k.shape[1], n, d, scale, is_causal)
    return int(load().fa_workspace_bytes(impl, DTYPE_CODES.get(q.dtype, -1), ctypes.byref(p)))


def workspace_for(stream: torch.cuda.Stream, nbytes: int,
                  device: torch.device) -> torch.Tensor | None:
    """A workspace of ``nbytes`` for a launch on ``stream`` (None for 0 bytes).

    Lifetime rule: it is allocated *on the launch stream*. The caching allocator keeps a freed
    block in the pool of the stream it was allocated on and hands it out again only to later
    allocations on that stream, whose work the stream orders after the launch. A caller may
    therefore drop the tensor as soon as the launch is queued. Allocated on another stream (for
    instance torch's current one while the launch goes to ``stream``), its bytes could be reused
    while the kernel still writes them."""
    if not nbytes:
        return None
    with torch.cuda.stream(stream):
        return torch.empty(nbytes, dtype=torch.uint8, device=device)


def forward(impl: int, q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, o: torch.Tensor,
            lse: torch.Tensor | None, is_causal: bool, scale: float,
            stream: torch.cuda.Stream | None = None,
            workspace: torch.Tensor | None | str = "auto") -> int:
    """``fa_forward`` on torch device tensors (caller-allocated o and lse, like any C caller).
    Launches on ``stream`` (default: torch's current stream) and returns the hipError_t value.
    ``workspace``: "auto" allocates the bytes ``fa_workspace_bytes`` asks for (none for most
    problems) on the launch stream (see ``workspace_for``), None passes a null workspace, a
    tensor is passed as is."""
    b, h, n, d = q.shape
    p = params(b, h, k.shape[1], n, d, scale, is_causal)
    s = stream if stream is not None else torch.cuda.current_stream(q.device)
    if isinstance(workspace, str):
        workspace = workspace_for(s, workspace_bytes(impl, q, k, is_causal, scale), q.device)
    ws = 0 if workspace is None else workspace.data_ptr()
    return forward_raw(impl, DTYPE_CODES[q.dtype], q.data_ptr(), k.data_ptr(), v.data_ptr(),
                       o.data_ptr(), 0 if lse is None else lse.data_ptr(), ws, p, s.cuda_stream)


def strides_of(t: torch.Tensor) -> FaStrides:
    return FaStrides(t.stride(0), t.stride(1), t.stride(2))


def forward_strided(impl: int, q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, o: torch.Tensor,
                    lse: torch.Tensor, is_causal: bool, scale: float,
                    stream: torch.cuda.Stream | None = None,
                    workspace: torch.Tensor | None | str = "auto") -> int:
    """``fa_forward_strided`` on torch views (their own strides); returns the hipError_t value.
    ``workspace`` as for ``forward``."""
    b, h, n, d = q.shape
    p = params(b, h, k.shape[1], n, d, scale, is_causal)
    s = stream if stream is not None else torch.cuda.current_stream(q.device)
    if isinstance(workspace, str):
        workspace = workspace_for(s, workspace_bytes(impl, q, k, is_causal, scale), q.device)
    qs, ks, vs, os_ = strides_of(q), strides_of(k), strides_of(v), strides_of(o)
    return load().fa_forward_strided(impl, DTYPE_CODES[q.dtype], q.data_ptr(), ctypes.byref(qs),
                                     k.data_ptr(), ctypes.byref(ks), v.data_ptr(),
                                     ctypes.byref(vs), o.data_ptr(), ctypes.byref(os_),
                                     lse.data_ptr(),
                                     None if workspace is None else workspace.data_ptr(),
                                     ctypes.byref(p), s.cuda_stream)


def decode_params(q: torch.Tensor, k: torch.Tensor, is_causal: bool, scale: float,
                  num_splits: int = 0) -> FaDecodeParams:
    """``fa_decode_params`` for q [B, H, Nq, D] and k [B, Hkv, Nkv, D]."""
    b, h, nq, d = q.shape
    return FaDecodeParams(b, h, k.shape[1], nq, k.shape[2], d, scale, is_causal, num_splits)


def decode(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, o: torch.Tensor, lse: torch.Tensor,
           is_causal: bool, scale: float, num_splits: int = 0, workspace: torch.Tensor | None = None,
           stream: torch.cuda.Stream | None = None) -> int:
    """``fa_decode`` on torch device tensors; allocates the workspace the library asks for on the
    launch stream (see ``workspace_for``) unless one is given. Returns the hipError_t value."""
    lib = load()
    p = decode_params(q, k, is_causal, scale, num_splits)
    s = stream if stream is not None else torch.cuda.current_stream(q.device)
    if workspace is None:
        nbytes = lib.fa_decode_workspace_bytes(DTYPE_CODES.get(q.dtype, -1), ctypes.byref(p))
        workspace = workspace_for(s, nbytes, q.device)
    return lib.fa_decode(DTYPE_CODES.get(q.dtype, -1), q.data_ptr(), k.data_ptr(), v.data_ptr(),
                         o.data_ptr(), lse.data_ptr(),
                         None if workspace is None else workspace.data_ptr(), ctypes.byref(p),
                         s.cuda_stream)


def decode_noalloc(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, o: torch.Tensor,
                   lse: torch.Tensor, is_causal: bool, scale: float, num_splits: int = 0,
                   stream: torch.cuda.Stream | None = None) -> int:
    """``fa_decode_noalloc``: the decode with its split partials in the library's per-GPU scratch
    array (``DECODE_SCRATCH_BYTES``) -- nothing is allocated, here or in the library. Calls that
    may overlap on one GPU share that array and must be serialised. Returns the hipError_t
    value."""
    p = decode_params(q, k, is_causal, scale, num_splits)
    s = stream if stream is not None else torch.cuda.current_stream(q.device)
    return load().fa_decode_noalloc(DTYPE_CODES.get(q.dtype, -1), q.data_ptr(), k.data_ptr(),
                                    v.data_ptr(), o.data_ptr(), lse.data_ptr(), ctypes.byref(p),
                                    s.cuda_stream)
