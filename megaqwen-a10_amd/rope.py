"""RoPE cos/sin tables (setup data handed to the decode kernels).

* ``precompute_rope_freqs`` — verify_correctness_a10.py:23-33: theta = 1e6,
  split-half layout (``cat[cos, cos]``: column i and i+64 share a frequency),
  fp32 angles, bf16 storage. This is the table the kernels' rotation (element
  i paired with i+64) is correct for, and the default here.
* ``make_rope`` — bench_int8.py:270-279: the legacy theta = 1e4 table with
  pair-duplicated columns that the reference's speed runs used.

Tables are computed once on the host in fp32 (deterministic across machines)
and then copied to ``device``.
"""
from __future__ import annotations

import torch


def precompute_rope_freqs(head_dim: int, max_seq_len: int, theta: float = 1000000.0, device="cpu"):
    exponent = torch.arange(0, head_dim, 2, dtype=torch.float32) / head_dim
    inv_freq = 1.0 / (theta ** exponent)
    t = torch.arange(max_seq_len, dtype=torch.float32)
    freqs = t[:, None] * inv_freq[None, :]
    cos = freqs.cos().to(torch.bfloat16)
    sin = freqs.sin().to(torch.bfloat16)
    return torch.cat([cos, cos], dim=-1).to(device), torch.cat([sin, sin], dim=-1).to(device)


def make_rope(max_seq_len: int, head_dim: int, device="cpu", theta: float = 10000.0):
    pos = torch.arange(max_seq_len, dtype=torch.float64)[:, None]
    denom = torch.tensor([theta ** (d / head_dim) for d in range(0, head_dim, 2)], dtype=torch.float64)
    ang = pos / denom[None, :]
    cos = torch.repeat_interleave(torch.cos(ang), 2, dim=1)
    sin = torch.repeat_interleave(torch.sin(ang), 2, dim=1)
    return (cos.to(torch.float32).to(torch.bfloat16).to(device),
            sin.to(torch.float32).to(torch.bfloat16).to(device))


__all__ = ["precompute_rope_freqs", "make_rope"]
