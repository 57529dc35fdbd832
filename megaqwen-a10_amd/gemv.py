"""INT8 weight-only matvec (int8_decoder.py:100-115, ``int8_gemv``) on gfx950.

``int8_gemv(x, w_int8, scale)`` returns ``y[j] = scale[j] * sum_i x[i] * w[j, i]``
as fp32 [M]. ``x`` is fp32 [K] (the reference's Triton
kernel took fp16), ``w_int8`` int8 [M, K] row-major with K a multiple of 16,
``scale`` fp32 [M]. One launch of csrc/gemv.hip on the current stream.
"""
from __future__ import annotations

import torch

from . import _lib


def int8_gemv(x: torch.Tensor, w_int8: torch.Tensor, scale: torch.Tensor, out: torch.Tensor | None = None):
    if w_int8.dim() != 2 or w_int8.dtype != torch.int8:
        raise TypeError("w_int8 must be an int8 [M, K] tensor")
    M, K = w_int8.shape
    if x.dtype != torch.float32 or tuple(x.shape) != (K,):
        raise TypeError(f"x must be fp32 [{K}]")
    if scale.dtype != torch.float32 or tuple(scale.shape) != (M,):
        raise TypeError(f"scale must be fp32 [{M}]")
    for name, t in (("x", x), ("w_int8", w_int8), ("scale", scale)):
        if not t.is_cuda or not t.is_contiguous():
            raise ValueError(f"{name} must be a contiguous tensor on a HIP device")
    if out is None:
        out = torch.empty(M, dtype=torch.float32, device=w_int8.device)
    lib = _lib.load()
    _lib.check(lib.mq_int8_gemv(x.data_ptr(), w_int8.data_ptr(), scale.data_ptr(), out.data_ptr(), M, K,
                                _lib.stream_handle(w_int8.device)), "mq_int8_gemv")
    return out


def int8_gemv_repeat(x: torch.Tensor, w_copies: torch.Tensor, scale: torch.Tensor, reps: int,
                     out: torch.Tensor | None = None):
    """Steady-state form of ``int8_gemv`` (mq_int8_gemv_repeat; no counterpart in the
    reference): one launch computes ``reps`` matvecs, rep i against copy i % n of
    ``w_copies`` (int8 [n, M, K], contiguous), and returns y fp32 [n, M] with
    ``y[c] = scale * (w_copies[c] @ x)``. Timing the launch and dividing by ``reps`` gives
    the per-matvec time without launch gaps (int8_decoder.py:351-434 times single calls)."""
    if w_copies.dim() != 3 or w_copies.dtype != torch.int8:
        raise TypeError("w_copies must be an int8 [n, M, K] tensor")
    n, M, K = w_copies.shape
    if x.dtype != torch.float32 or tuple(x.shape) != (K,):
        raise TypeError(f"x must be fp32 [{K}]")
    if scale.dtype != torch.float32 or tuple(scale.shape) != (M,):
        raise TypeError(f"scale must be fp32 [{M}]")
    if not isinstance(reps, int) or reps < 1:
        raise ValueError(f"reps must be a positive int, got {reps!r}")
    for name, t in (("x", x), ("w_copies", w_copies), ("scale", scale)):
        if not t.is_cuda or not t.is_contiguous():
            raise ValueError(f"{name} must be a contiguous tensor on a HIP device")
    if out is None:
        out = torch.empty((n, M), dtype=torch.float32, device=w_copies.device)
    elif out.dtype != torch.float32 or tuple(out.shape) != (n, M) or not out.is_contiguous():
        raise ValueError(f"out must be a contiguous fp32 [{n}, {M}] tensor")
    lib = _lib.load()
    _lib.check(lib.mq_int8_gemv_repeat(x.data_ptr(), w_copies.data_ptr(), M * K, n, scale.data_ptr(), out.data_ptr(),
                                       M, K, reps, _lib.stream_handle(w_copies.device)), "mq_int8_gemv_repeat")
    return out
