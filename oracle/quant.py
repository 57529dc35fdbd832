"""Per-output-channel symmetric INT8 quantizer — CPU restatement (test infrastructure).

Follows bench_int8.py:19-24 (identical copies at int8_decoder.py:45-56 and
build_int8_kernel.py:54-57). The arithmetic happens in three distinct
precisions, and each one matters for bit-exactness:

1. ``amax`` is the row maximum of |w| in w's own dtype (bf16 for the
   reference's weights) — exact.
2. ``amax / 127`` is evaluated in that same dtype: for bf16 that is an fp32
   division rounded to bf16 (round-to-nearest-even), so every scale is
   bf16-representable. It is then widened to fp32 and clamped to >= 1e-12.
3. ``w / scale`` promotes to fp32 (IEEE division), rounds half-to-even,
   clamps to [-128, 127] and narrows to int8.
"""
from __future__ import annotations

import torch

SCALE_FLOOR = 1e-12


def quantize_per_channel(w: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """Return ``(q int8 [M,K], scale fp32 [M])`` for a 2-D weight ``w`` [M,K]."""
    if w.dim() != 2:
        raise ValueError(f"expected a 2-D weight, got shape {tuple(w.shape)}")
    w = w.cpu()
    row_max = torch.amax(torch.abs(w), dim=1)            # dtype of w, exact
    step = torch.div(row_max, 127.0)                     # evaluated in w's dtype
    scale = step.to(torch.float32).clamp(min=SCALE_FLOOR)
    ratio = torch.div(w.to(torch.float32), scale.unsqueeze(1))
    q = torch.clamp(torch.round(ratio), -128, 127).to(torch.int8)
    return q, scale


def dequantize(q: torch.Tensor, scale: torch.Tensor, dtype=torch.float64) -> torch.Tensor:
    """``q[j,k] * scale[j]`` in ``dtype`` (exact in float64)."""
    return q.to(dtype) * scale.to(dtype).unsqueeze(1)
