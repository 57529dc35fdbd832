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
