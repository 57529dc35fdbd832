"""Per-output-channel symmetric INT8 quantization (bench_int8.py:19-24) on the GPU.

``quantize_per_channel(w)`` keeps the reference's name and contract — a bf16
weight [M, K] in, ``(int8 [M, K], fp32 scale [M])`` out, with
``scale = bf16(absmax / 127)`` widened to fp32 and clamped to >= 1e-12, and
``q = clamp(round_half_even(w / scale), -128, 127)`` — and runs as one HIP
kernel (csrc/quant.hip). The input must be a bf16 tensor on a HIP device.
"""
from __future__ import annotations

import torch

from . import _lib


def quantize_per_channel(tensor: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    if tensor.dim() != 2:
        raise ValueError(f"expected a 2-D weight [out, in], got shape {tuple(tensor.shape)}")
    if tensor.dtype != torch.bfloat16:
        raise TypeError(f"expected a bfloat16 weight, got {tensor.dtype}")
    if not tensor.is_cuda:
        raise ValueError("quantize_per_channel runs on the GPU: move the weight to a HIP device first")
    w = tensor.contiguous()
    M, K = w.shape
    q = torch.empty((M, K), dtype=torch.int8, device=w.device)
    scale = torch.empty((M,), dtype=torch.float32, device=w.device)
    lib = _lib.load()
    with torch.cuda.device(w.device):
        _lib.check(lib.mq_quantize_per_channel_bf16(w.data_ptr(), M, K, q.data_ptr(), scale.data_ptr(),
                                                    _lib.stream_handle()), "mq_quantize_per_channel_bf16")
    return q, scale
