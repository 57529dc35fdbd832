"""Model shapes served by the decode kernels.

The reference hard-codes Qwen3-0.6B as compile-time constants (config.cuh:33-40,
bench_int8.py:11-16); here the shape is data, and the kernels are compiled
for the two shapes the benchmarks use.
"""
from __future__ import annotations

from dataclasses import dataclass, replace


@dataclass(frozen=True)
class ModelConfig:
    name: str
    hidden_size: int = 1024
    intermediate_size: int = 3072
    num_q_heads: int = 16
    num_kv_heads: int = 8
    head_dim: int = 128
    num_layers: int = 28
    vocab_size: int = 151936
    rms_eps: float = 1e-6
    rope_theta: float = 1e6
    tie_word_embeddings: bool = True

    @property
    def q_size(self) -> int:
        return self.num_q_heads * self.head_dim

    @property
    def kv_size(self) -> int:
        return self.num_kv_heads * self.head_dim

    def with_(self, **kw) -> "ModelConfig":
        return replace(self, **kw)

    def int8_step_bytes(self, cache_len: int = 0) -> int:
        """Algorithmic HBM bytes of one INT8 decode step: every int8 weight,
        fp32 scale and bf16 norm weight once, one embedding row, the LM head
        and its scales, plus the K/V rows attended to and written."""
        H, I, Q, KV, L, V, D = (self.hidden_size, self.intermediate_size, self.q_size, self.kv_size,
                                self.num_layers, self.vocab_size, self.head_dim)
        proj = Q * H + 2 * KV * H + H * Q + 2 * I * H + H * I
        scales = 4 * (Q + 2 * KV + H + 2 * I + H)
        norms = 2 * (2 * H + 2 * D)
        per_layer = proj + scales + norms
        lm = V * H + 4 * V
        kv = L * 2 * self.num_kv_heads * D * 2 * (cache_len + 1)
        return L * per_layer + lm + 2 * H + 2 * H + kv

    def int4_step_bytes(self, cache_len: int = 0) -> int:
        """The same for INT4 layer projections per group of 128 (half a byte per weight, an
        fp32 scale per group) with the LM head INT8 per row."""
        H, I, Q, KV, L, V, D = (self.hidden_size, self.intermediate_size, self.q_size, self.kv_size,
                                self.num_layers, self.vocab_size, self.head_dim)
        proj = Q * H + 2 * KV * H + H * Q + 2 * I * H + H * I
        per_layer = proj // 2 + 4 * (proj // 128) + 2 * (2 * H + 2 * D)
        lm = V * H + 4 * V
        kv = L * 2 * self.num_kv_heads * D * 2 * (cache_len + 1)
        return L * per_layer + lm + 2 * H + 2 * H + kv

    def bf16_step_bytes(self, cache_len: int = 0) -> int:
        H, I, Q, KV, L, V, D = (self.hidden_size, self.intermediate_size, self.q_size, self.kv_size,
                                self.num_layers, self.vocab_size, self.head_dim)
        proj = 2 * (Q * H + 2 * KV * H + H * Q + 2 * I * H + H * I)
        norms = 2 * (2 * H + 2 * D)
        lm = 2 * V * H
        kv = L * 2 * self.num_kv_heads * D * 2 * (cache_len + 1)
        return L * (proj + norms) + lm + 2 * H + 2 * H + kv


QWEN3_0_6B = ModelConfig("qwen3-0.6b")
QWEN3_1_7B = ModelConfig("qwen3-1.7b", hidden_size=2048, intermediate_size=6144)
