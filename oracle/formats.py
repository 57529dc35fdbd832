"""CPU oracle for the other weight formats: FP8 E4M3 per-row and INT4 per-group.

Test infrastructure only: imported by tests/, never by the product path.

The reference has no FP8 or INT4 weights (its only other-format figure is a
llama.cpp Q4_K_M comparison, README.md:19), so there is no reference expression
to restate. The formats follow the INT8 quantizer's pattern
(bench_int8.py:19-24: per-channel symmetric scale from the absolute maximum,
IEEE division, round half to even, clamp), with the definitions below; every
function here is pinned in tests/test_oracle_pins.py by brute force over the
code tables or by an independent torch formulation.

FP8 E4M3 (OCP "E4M3FN", the format gfx950's v_cvt_pk_f32_fp8 decodes): sign,
4 exponent bits (bias 7), 3 mantissa bits; subnormals m * 2^-9; no
infinities; 0x7F / 0xFF are NaN; largest finite 448.
  per row:  s = fp32(max_k |w|) / 448  (IEEE fp32), floored at 1e-12
            q = encode(fp32(w) / s)    round to nearest, ties to even mantissa,
                                       |x| >= 448 saturates to +-448
INT4 per group of G = 128 consecutive elements of a row (two's complement nibbles):
            s = bf16(amax_group / 7)   (fp32 division rounded to bf16, as the INT8
                                       quantizer's bf16 division), floored at 1e-12
            q = clamp(rint(fp32(w) / s), -8, 7)
            byte i of a row = (q[2i] & 15) | (q[2i + 1] & 15) << 4
Matvec: y[j] = sum_k dequant(w)[j, k] x[k], in float64 here.
"""
from __future__ import annotations

import numpy as np
import torch

FP8_MAX = 448.0
INT4_GROUP = 128


# ---- FP8 E4M3 --------------------------------------------------------------------------
def fp8_decode_table() -> np.ndarray:
    """float64 value of every code 0..255 (NaN for 0x7F, 0xFF)."""
    c = np.arange(256)
    sign = np.where(c & 0x80, -1.0, 1.0)
    e = (c >> 3) & 0xF
    m = c & 7
    val = np.where(e == 0, m * 2.0 ** -9, (1.0 + m / 8.0) * 2.0 ** (e.astype(np.float64) - 7.0))
    val = sign * val
    val[(e == 15) & (m == 7)] = np.nan
    return val


def fp8_encode(x: np.ndarray) -> np.ndarray:
    """Codes of float32 values x (round to nearest even, saturating at +-448)."""
    x = np.asarray(x, dtype=np.float32)
    u = x.view(np.uint32)
    sign = ((u >> np.uint32(24)) & np.uint32(0x80)).astype(np.uint32)
    a = np.abs(x)
    out = np.zeros(x.shape, dtype=np.uint32)
    sat = ~(a < np.float32(FP8_MAX))
    sub = (a < np.float32(2.0 ** -6)) & ~sat
    nor = ~sat & ~sub
    out[sat] = 0x7E
    out[sub] = np.rint(a[sub] * np.float32(512.0)).astype(np.uint32)         # exact scaling, RNE
    ua = a[nor].view(np.uint32)
    r = (ua + np.uint32(0x7FFFF) + ((ua >> np.uint32(20)) & np.uint32(1))) & np.uint32(0xFFF00000)
    exp = (r >> np.uint32(23)).astype(np.int64) - 127
    out[nor] = (((exp + 7) << 3) | ((r >> np.uint32(20)) & np.uint32(7)).astype(np.int64)).astype(np.uint32)
    return (out | sign).astype(np.uint8)


def quantize_fp8_rows(w: torch.Tensor):
    """bf16 [M, K] -> (codes uint8 [M, K], scale fp32 [M])."""
    wf = w.float().numpy()
    amax = np.abs(wf).max(axis=1).astype(np.float32)
    s = np.maximum(amax / np.float32(FP8_MAX), np.float32(1e-12)).astype(np.float32)
    q = fp8_encode((wf / s[:, None]).astype(np.float32))
    return torch.from_numpy(q), torch.from_numpy(s)


def dequant_fp8(q: torch.Tensor, s: torch.Tensor) -> np.ndarray:
    return fp8_decode_table()[q.numpy().astype(np.int64)] * s.numpy().astype(np.float64)[:, None]


# ---- INT4 per group ----------------------------------------------------------------------
def quantize_int4_groups(w: torch.Tensor, group: int = INT4_GROUP):
    """bf16 [M, K] (K % group == 0) -> (packed uint8 [M, K / 2], scales fp32 [M, K / group])."""
    M, K = w.shape
    wf = w.float().numpy().reshape(M, K // group, group)
    amax = np.abs(wf).max(axis=2).astype(np.float32)                          # bf16 values: exact
    s = (amax / np.float32(7.0)).astype(np.float32)
    s = torch.from_numpy(s).to(torch.bfloat16).float().numpy()               # round to bf16 (RNE)
    s = np.maximum(s, np.float32(1e-12)).astype(np.float32)
    q = np.clip(np.rint((wf / s[:, :, None]).astype(np.float32)), -8, 7).astype(np.int64).reshape(M, K)
    packed = ((q[:, 0::2] & 15) | ((q[:, 1::2] & 15) << 4)).astype(np.uint8)
    return torch.from_numpy(packed), torch.from_numpy(s)


def unpack_int4(packed: torch.Tensor) -> np.ndarray:
    """uint8 [M, K / 2] -> int64 [M, K] nibble values in [-8, 7]."""
    p = packed.numpy().astype(np.int64)
    lo, hi = p & 15, (p >> 4) & 15
    q = np.empty((p.shape[0], 2 * p.shape[1]), dtype=np.int64)
    q[:, 0::2] = np.where(lo >= 8, lo - 16, lo)
    q[:, 1::2] = np.where(hi >= 8, hi - 16, hi)
    return q


def dequant_int4(packed: torch.Tensor, s: torch.Tensor, group: int = INT4_GROUP) -> np.ndarray:
    q = unpack_int4(packed).astype(np.float64)
    M, K = q.shape
    return (q.reshape(M, K // group, group) * s.numpy().astype(np.float64)[:, :, None]).reshape(M, K)


def matvec_f64(wd: np.ndarray, x: torch.Tensor) -> np.ndarray:
    """float64 product of a dequantized [M, K] matrix with x."""
    return wd @ x.numpy().astype(np.float64)
