"""RoPE cos/sin tables — CPU restatement (test infrastructure).

* ``split_half_tables`` follows verify_correctness_a10.py:23-33 (also
  a10_chat.py:24-32): inv_freq = 1/theta^(2i/D) and the angles p*inv_freq
  are fp32, cos/sin are taken in fp32, rounded to bf16, and the 64 columns
  are repeated (``cat[cos, cos]``) so column i and i+64 share a frequency.
  This is the HF Qwen3 convention and the table the decode kernels assume
  (they rotate element i with element i+64, a10_int8_decode_kernel.cu:180-192).
* ``pair_duplicated_tables`` follows bench_int8.py:270-279 (and
  a10_decode.py:329-339): theta=1e4, Python-double angles, columns 2j and
  2j+1 share frequency j. The reference's speed runs used it; it does not
  match the kernels' split-half pairing, so it only matters for timing.
"""
from __future__ import annotations

import math

import torch


def split_half_tables(max_seq_len: int, head_dim: int = 128, theta: float = 1e6):
    half = head_dim // 2
    exponent = torch.arange(0, head_dim, 2, dtype=torch.float32) / head_dim
    inv_freq = 1.0 / (theta ** exponent)                             # fp32 pow
    positions = torch.arange(max_seq_len, dtype=torch.float32)
    angles = positions.unsqueeze(1) * inv_freq.unsqueeze(0)          # [S, half] fp32
    assert angles.shape[1] == half
    c = torch.cos(angles).to(torch.bfloat16)
    s = torch.sin(angles).to(torch.bfloat16)
    return torch.cat([c, c], dim=1), torch.cat([s, s], dim=1)


def pair_duplicated_tables(max_seq_len: int, head_dim: int = 128, theta: float = 1e4):
    c = torch.zeros(max_seq_len, head_dim, dtype=torch.float64)
    s = torch.zeros(max_seq_len, head_dim, dtype=torch.float64)
    for d in range(0, head_dim, 2):
        denom = theta ** (d / head_dim)
        for p in range(max_seq_len):
            a = p / denom
            c[p, d] = c[p, d + 1] = math.cos(a)
            s[p, d] = s[p, d + 1] = math.sin(a)
    # A Python float stored into a bf16 tensor goes double -> float -> bf16.
    return c.to(torch.float32).to(torch.bfloat16), s.to(torch.float32).to(torch.bfloat16)
