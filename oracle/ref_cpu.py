"""One batch-1 decode step on the CPU — restatement of the reference kernel (test infrastructure).

Follows a10_int8_decode_kernel.cu (INT8) and a10_decode_kernel.cu (BF16,
the same pipeline with unit scales) stage by stage; the line numbers below
are in the INT8 file:

    h      = embed[t]                                              :21-33
    per layer:
      r    = fp32(h);  n = r * rsqrt(mean(r^2) + eps) * in_ln        :54-84
      q|k|v= (W_qkv @ n) * s_qkv                                     :88-135
      per head: y = x * rsqrt(mean(x^2) + eps) * {q,k}_norm          :165-178, :202-218
                y'[i]   = y[i] c[i] - y[i+64] s[i]        (i < 64)   :180-192
                y'[i]   = y[i-64] s[i] + y[i] c[i]        (i >= 64)
      Kc[pos] = bf16(k'), Vc[pos] = bf16(v)                          :233-235
      attn_h = softmax_j(q'_h . Kc[j] * attn_scale) @ Vc, kv head = h // 2,
               j < cache_len = pos + 1 (the current K/V read back from the
               bf16 cache)                                           :298-359
      x    = (W_o @ attn) * s_o + r                                  :393-418
      n2   = x * rsqrt(mean(x^2) + eps) * post_ln                    :421-457
      m    = silu((W_g @ n2) * s_g) * ((W_u @ n2) * s_u)            :460-534
             silu(z) = z / (1 + exp(-z))                             config.cuh:81-83
      h    = bf16((W_d @ m) * s_d + x)                               :538-572
    n      = fp32(h) * rsqrt(mean(h^2) + eps) * final_norm           :581-615
    token  = argmax_v (W_lm @ n)[v] * s_lm[v]                        :702-815

Argmax ties resolve to the lowest index (torch.argmax); the reference's
result on exact ties depends on its reduction order.

Numerics: with ``dtype=torch.float64`` every reduction is done in float64
and rounded to fp32 wherever the kernel stores an fp32 intermediate, and to
bf16 where the kernel stores bf16 (layer output, K/V cache). That makes the
oracle independent of BLAS summation order; the fp32 kernel differs from it
by accumulation error only. ``dtype=torch.float32`` is the plain fp32 port
(``(q.float() @ x) * scale``) used as the CPU baseline. ``rounding=False``
drops the bf16/fp32 rounding points so the architecture can be compared
with HF transformers' Qwen3 in float64.
"""
from __future__ import annotations

from dataclasses import dataclass

import torch

LAYER_FIELDS = ("in_ln", "q", "k", "v", "q_norm", "k_norm", "o", "post_ln", "gate", "up", "down")
SCALE_FIELDS = ("q", "k", "v", "o", "gate", "up", "down")


@dataclass
class Dims:
    hidden_size: int = 1024
    intermediate_size: int = 3072
    num_q_heads: int = 16
    num_kv_heads: int = 8
    head_dim: int = 128
    vocab_size: int = 151936
    rms_eps: float = 1e-6


class RefDecoder:
    """CPU decoder with the reference's ``decode_step`` / ``reset`` / ``position`` surface.

    ``layer_tensors`` is the reference's flat list of 11 tensors per layer
    (bench_int8.py:291-320 order) and ``layer_scales`` the flat list of 7
    scale vectors per layer (bench_int8.py:322-330), or None for bf16.
    """

    def __init__(self, dims: Dims, embed, layer_tensors, layer_scales, final_norm,
                 lm_head, lm_head_scale, cos_table, sin_table, num_layers: int,
                 max_seq_len: int, dtype=torch.float64, rounding: bool = True):
        self.d = dims
        self.dtype = dtype
        self.rounding = rounding
        self.num_layers = num_layers
        self.max_seq_len = max_seq_len
        # The reference passes the fp32 constant 1.0f / sqrtf(128.0f) (bench_int8.py:190).
        self.attn_scale = float(torch.tensor(1.0 / dims.head_dim ** 0.5, dtype=torch.float32))
        if len(layer_tensors) != 11 * num_layers:
            raise ValueError("expected 11 tensors per layer")
        if layer_scales is not None and len(layer_scales) != 7 * num_layers:
            raise ValueError("expected 7 scale vectors per layer")
        cv = lambda t: t.detach().cpu().to(dtype)
        self.embed = embed.detach().cpu()              # kept in its storage dtype (bf16)
        self.layers = []
        for l in range(num_layers):
            lt = layer_tensors[11 * l: 11 * l + 11]
            layer = {name: cv(t) for name, t in zip(LAYER_FIELDS, lt)}
            if layer_scales is not None:
                ls = layer_scales[7 * l: 7 * l + 7]
                layer.update({f"{n}_s": cv(s) for n, s in zip(SCALE_FIELDS, ls)})
            self.layers.append(layer)
        self.final_norm = cv(final_norm)
        self.lm_head = cv(lm_head)
        self.lm_scale = None if lm_head_scale is None else cv(lm_head_scale)
        self.cos = cos_table.detach().cpu()
        self.sin = sin_table.detach().cpu()
        kv_shape = (num_layers, dims.num_kv_heads, max_seq_len, dims.head_dim)
        cache_dtype = torch.bfloat16 if rounding else dtype
        self.k_cache = torch.zeros(kv_shape, dtype=cache_dtype)
        self.v_cache = torch.zeros(kv_shape, dtype=cache_dtype)
        self._pos = 0
        self.last = {}

    # -- reference surface (bench_int8.py:193-227) ---------------------------------------
    def reset(self):
        self._pos = 0
        self.k_cache.zero_()
        self.v_cache.zero_()

    def position(self) -> int:
        return self._pos

    def load_kv(self, k_cache, v_cache, position: int) -> None:
        """Start from a given cache (e.g. a long-context pre-fill): rows [0, position)
        of every layer / KV head are copied, the next step decodes at ``position``."""
        self.reset()
        self.k_cache[:, :, :position] = k_cache[:, :, :position].detach().cpu().to(self.k_cache.dtype)
        self.v_cache[:, :, :position] = v_cache[:, :, :position].detach().cpu().to(self.v_cache.dtype)
        self._pos = position

    def decode_step(self, token: int) -> int:
        logits = self.step_logits(token)
        return int(torch.argmax(logits))

    # -- rounding points -------------------------------------------------------------------
    def _f32(self, x):
        return x.to(torch.float32).to(self.dtype) if self.rounding else x

    def _bf16(self, x):
        return x.to(torch.float32).to(torch.bfloat16).to(self.dtype) if self.rounding else x

    def _rmsnorm(self, x, w):
        ms = torch.mean(x * x, dim=-1, keepdim=True)
        return x * torch.rsqrt(ms + self.d.rms_eps) * w

    def _linear(self, layer, name, x):
        y = torch.mv(layer[name], x)
        s = layer.get(f"{name}_s")
        return y if s is None else y * s

    # -- one step --------------------------------------------------------------------------
    def step_logits(self, token: int) -> torch.Tensor:
        d = self.d
        if not 0 <= token < d.vocab_size:
            raise ValueError(f"token id {token} outside [0, {d.vocab_size})")
        pos = self._pos
        if pos >= self.max_seq_len:
            raise ValueError(f"position {pos} >= max_seq_len {self.max_seq_len}")
        D, nq, nkv = d.head_dim, d.num_q_heads, d.num_kv_heads
        group = nq // nkv
        half = D // 2
        c = self.cos[pos].to(self.dtype)
        s = self.sin[pos].to(self.dtype)
        h = self.embed[token].to(self.dtype)                           # bf16 values

        def rope(y):                                                   # y: [heads, D]
            lo, hi = y[:, :half], y[:, half:]
            out_lo = lo * c[:half] - hi * s[:half]
            out_hi = lo * s[half:] + hi * c[half:]
            return torch.cat([out_lo, out_hi], dim=1)

        for l, w in enumerate(self.layers):
            r = h
            n = self._f32(self._rmsnorm(r, w["in_ln"]))
            q = self._f32(self._linear(w, "q", n)).view(nq, D)
            k = self._f32(self._linear(w, "k", n)).view(nkv, D)
            v = self._f32(self._linear(w, "v", n)).view(nkv, D)
            q = self._f32(rope(self._rmsnorm(q, w["q_norm"])))
            k = self._f32(rope(self._rmsnorm(k, w["k_norm"])))
            self.k_cache[l, :, pos] = self._bf16(k).to(self.k_cache.dtype)
            self.v_cache[l, :, pos] = self._bf16(v).to(self.v_cache.dtype)
            keys = self.k_cache[l, :, :pos + 1].to(self.dtype)         # [nkv, L, D]
            vals = self.v_cache[l, :, :pos + 1].to(self.dtype)
            kv_of_q = torch.arange(nq) // group
            scores = torch.einsum("hd,hld->hl", q, keys[kv_of_q]) * self.attn_scale
            p = torch.softmax(scores, dim=-1)
            attn = self._f32(torch.einsum("hl,hld->hd", p, vals[kv_of_q])).reshape(-1)
            x = self._f32(self._linear(w, "o", attn) + r)
            n2 = self._f32(self._rmsnorm(x, w["post_ln"]))
            g = self._linear(w, "gate", n2)
            u = self._linear(w, "up", n2)
            m = self._f32(g / (1.0 + torch.exp(-g)) * u)
            h = self._bf16(self._linear(w, "down", m) + x)
            if l == self.num_layers - 1:
                self.last = {"q": q.reshape(-1), "k": k.reshape(-1), "v": v.reshape(-1),
                             "attn_out": attn, "residual": x, "activations": n2,
                             "mlp_intermediate": m, "hidden": h}
        nf = self._f32(self._rmsnorm(h, self.final_norm))
        logits = torch.mv(self.lm_head, nf)
        if self.lm_scale is not None:
            logits = logits * self.lm_scale
        logits = self._f32(logits)
        self.last["normalized"] = nf
        self.last["logits"] = logits
        self._pos += 1
        return logits


def top2_margin(logits: torch.Tensor) -> float:
    top = torch.topk(logits.to(torch.float64), 2).values
    return float(top[0] - top[1])


def greedy_generate(dec: RefDecoder, prompt, num_tokens: int):
    """Prefill one token per step, then feed back argmax (verify_correctness_a10.py:323-339):
    the last prefill step's output is generated token 1. Returns (tokens, margins)."""
    dec.reset()
    toks, margins = [], []
    logits = None
    for t in prompt:
        logits = dec.step_logits(int(t))
    nxt = int(torch.argmax(logits))
    toks.append(nxt)
    margins.append(top2_margin(logits))
    while len(toks) < num_tokens:
        logits = dec.step_logits(nxt)
        nxt = int(torch.argmax(logits))
        toks.append(nxt)
        margins.append(top2_margin(logits))
    return toks, margins


# ---- sampling (no counterpart in the reference: its generate() accepts a temperature
# and ignores it, a10_decode.py:358) -------------------------------------------------
_GOLDEN = 0x9E3779B97F4A7C15
_M64 = (1 << 64) - 1


def splitmix64_mix(z):
    """The SplitMix64 output function (Steele, Lea, Flood, OOPSLA 2014), on Python ints or
    numpy uint64 arrays (wrapping arithmetic)."""
    import numpy as np
    if isinstance(z, np.ndarray):
        z = z.astype(np.uint64)
        z = (z ^ (z >> np.uint64(30))) * np.uint64(0xBF58476D1CE4E5B9)
        z = (z ^ (z >> np.uint64(27))) * np.uint64(0x94D049BB133111EB)
        return z ^ (z >> np.uint64(31))
    z &= _M64
    z = ((z ^ (z >> 30)) * 0xBF58476D1CE4E5B9) & _M64
    z = ((z ^ (z >> 27)) * 0x94D049BB133111EB) & _M64
    return z ^ (z >> 31)


def gumbel_noise(seed: int, pos: int, rows):
    """Gumbel noise of vocabulary rows ``rows`` at position ``pos``: u = (m + 0.5) 2^-23
    from the top 23 bits m of splitmix64_mix(seed ^ ((pos << 32 | row) * golden)), then
    g = -log(-log(u)) in float64. The kernels compute the same u exactly and g in fp32."""
    import numpy as np
    rows = np.asarray(rows, dtype=np.uint64)
    key = (np.uint64(pos) << np.uint64(32)) | rows
    with np.errstate(over="ignore"):
        z = splitmix64_mix(np.uint64(seed) ^ (key * np.uint64(_GOLDEN)))
    u = ((z >> np.uint64(41)).astype(np.float64) + 0.5) * 2.0 ** -23
    return -np.log(-np.log(u))


def sampled_choice(logits, temperature: float, seed: int, pos: int):
    """Gumbel-max sample of softmax(logits / temperature) at position ``pos``: returns
    (token, margin), margin being the gap between the two largest perturbed values."""
    import numpy as np
    v = np.asarray(logits, dtype=np.float64) / temperature + gumbel_noise(seed, pos, np.arange(len(logits)))
    top2 = np.partition(v, -2)[-2:]
    return int(np.argmax(v)), float(top2[1] - top2[0])
