"""Other weight formats on gfx950: FP8 E4M3 per-row and INT4 per-group (128) weights.

The reference has INT8 and BF16 weights only (its one other-format figure is a
llama.cpp Q4_K_M comparison, README.md:19). These follow its INT8 quantizer's
pattern (bench_int8.py:19-24):

* ``quantize_fp8(w)``  -> (codes uint8 [M, K], scale fp32 [M]): s = amax / 448,
  codes = OCP E4M3FN of w / s (round to nearest even, saturating);
* ``quantize_int4(w)`` -> (packed uint8 [M, K/2], scale fp32 [M, K/128]):
  s = bf16(amax_group / 7), q = clamp(rint(w / s), -8, 7), low nibble = even element;
* ``fp8_gemv`` / ``int4_gemv``: y = dequant(w) @ x, fp32 x and y;
* ``fp8_gemv_repeat`` / ``int4_gemv_repeat``: the steady-state form (one launch,
  ``reps`` matvecs over rotating weight copies), as ``int8_gemv_repeat``.

Each call is one launch of csrc/formats.hip on the current stream.
"""
from __future__ import annotations

import torch

from . import _lib

INT4_GROUP = 128


def _check_dev(**tensors):
    for name, t in tensors.items():
        if not t.is_cuda or not t.is_contiguous():
            raise ValueError(f"{name} must be a contiguous tensor on a HIP device")


def quantize_fp8(w: torch.Tensor):
    if w.dim() != 2 or w.dtype != torch.bfloat16:
        raise TypeError("w must be a bf16 [M, K] tensor")
    _check_dev(w=w)
    M, K = w.shape
    q = torch.empty((M, K), dtype=torch.uint8, device=w.device)
    s = torch.empty(M, dtype=torch.float32, device=w.device)
    _lib.check(_lib.load().mq_quantize_fp8_rows_bf16(w.data_ptr(), M, K, q.data_ptr(), s.data_ptr(),
                                                     _lib.stream_handle(w.device)), "mq_quantize_fp8_rows_bf16")
    return q, s


def quantize_int4(w: torch.Tensor):
    if w.dim() != 2 or w.dtype != torch.bfloat16:
        raise TypeError("w must be a bf16 [M, K] tensor")
    _check_dev(w=w)
    M, K = w.shape
    if K % INT4_GROUP:
        raise ValueError(f"K must be a multiple of {INT4_GROUP}, got {K}")
    q = torch.empty((M, K // 2), dtype=torch.uint8, device=w.device)
    s = torch.empty((M, K // INT4_GROUP), dtype=torch.float32, device=w.device)
    _lib.check(_lib.load().mq_quantize_int4_groups_bf16(w.data_ptr(), M, K, q.data_ptr(), s.data_ptr(),
                                                        _lib.stream_handle(w.device)), "mq_quantize_int4_groups_bf16")
    return q, s


def _shapes(x, w, scale, int4: bool, copies: bool):
    if w.dtype != torch.uint8 or w.dim() != (3 if copies else 2):
        raise TypeError(f"w must be a uint8 {'[n, M, Kw]' if copies else '[M, Kw]'} tensor")
    M, Kw = w.shape[-2:]
    K = 2 * Kw if int4 else Kw
    if x.dtype != torch.float32 or tuple(x.shape) != (K,):
        raise TypeError(f"x must be fp32 [{K}]")
    want = (M, K // INT4_GROUP) if int4 else (M,)
    if scale.dtype != torch.float32 or tuple(scale.shape) != want:
        raise TypeError(f"scale must be fp32 {list(want)}")
    _check_dev(x=x, w=w, scale=scale)
    return M, K, Kw


def _gemv(fn, x, w, scale, out, int4):
    M, K, _ = _shapes(x, w, scale, int4, False)
    if out is None:
        out = torch.empty(M, dtype=torch.float32, device=w.device)
    lib = _lib.load()
    _lib.check(getattr(lib, fn)(x.data_ptr(), w.data_ptr(), scale.data_ptr(), out.data_ptr(), M, K,
                                _lib.stream_handle(w.device)), fn)
    return out


def _gemv_repeat(fn, x, w_copies, scale, reps, out, int4):
    M, K, Kw = _shapes(x, w_copies, scale, int4, True)
    n = w_copies.shape[0]
    if not isinstance(reps, int) or reps < 1:
        raise ValueError(f"reps must be a positive int, got {reps!r}")
    if out is None:
        out = torch.empty((n, M), dtype=torch.float32, device=w_copies.device)
    elif out.dtype != torch.float32 or tuple(out.shape) != (n, M) or not out.is_contiguous():
        raise ValueError(f"out must be a contiguous fp32 [{n}, {M}] tensor")
    lib = _lib.load()
    _lib.check(getattr(lib, fn)(x.data_ptr(), w_copies.data_ptr(), M * Kw, n, scale.data_ptr(), out.data_ptr(),
                                M, K, reps, _lib.stream_handle(w_copies.device)), fn)
    return out


def fp8_gemv(x, w, scale, out=None):
    return _gemv("mq_fp8_gemv", x, w, scale, out, False)


def int4_gemv(x, w, scale, out=None):
    return _gemv("mq_int4_gemv", x, w, scale, out, True)


def fp8_gemv_repeat(x, w_copies, scale, reps, out=None):
    return _gemv_repeat("mq_fp8_gemv_repeat", x, w_copies, scale, reps, out, False)


def int4_gemv_repeat(x, w_copies, scale, reps, out=None):
    return _gemv_repeat("mq_int4_gemv_repeat", x, w_copies, scale, reps, out, True)
