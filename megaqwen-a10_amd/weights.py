"""Seeded random-init weights and the reference's tensor packing.

No checkpoint is available offline, so the benchmarks and tests run on
random-init weights of the Qwen3 architecture (the BASELINE recipe):

* one ``torch.Generator('cpu').manual_seed(seed)`` stream;
* tensors drawn in HF Qwen3 state-dict order — ``model.embed_tokens.weight``,
  then per layer q, k, v, o, gate, up, down projections — each as
  ``randn(fp32) * 0.02`` rounded to bf16 (the reference holds bf16 weights,
  bench_int8.py:31);
* every RMSNorm gain (input, post-attention, q_norm, k_norm, final) is 1
  unless ``norm_jitter > 0``, which draws ``1 + norm_jitter * randn`` from a
  second generator seeded ``seed + 1`` (so the main stream is unchanged);
* the LM head is tied to the embedding;
* after the weights, the same generator draws the prompt,
  ``randint(0, vocab, (prompt_len,))``.

``pack_int8`` / ``pack_bf16`` produce the reference's flat lists: 11 tensors
per layer in LayerWeights order (bench_int8.py:291-320) and 7 scale vectors
per layer (bench_int8.py:322-330).
"""
from __future__ import annotations

import hashlib

import torch

from .config import ModelConfig
from .quant import quantize_per_channel

PROJ = ("self_attn.q_proj", "self_attn.k_proj", "self_attn.v_proj", "self_attn.o_proj",
        "mlp.gate_proj", "mlp.up_proj", "mlp.down_proj")


def _proj_shapes(cfg: ModelConfig):
    H, I, Q, KV = cfg.hidden_size, cfg.intermediate_size, cfg.q_size, cfg.kv_size
    return {"self_attn.q_proj": (Q, H), "self_attn.k_proj": (KV, H), "self_attn.v_proj": (KV, H),
            "self_attn.o_proj": (H, Q), "mlp.gate_proj": (I, H), "mlp.up_proj": (I, H),
            "mlp.down_proj": (H, I)}


def random_init_state(cfg: ModelConfig, seed: int = 0, prompt_len: int = 8, norm_jitter: float = 0.0):
    """Returns ``(state, prompt)``: a dict of bf16 CPU tensors under HF key names
    and the int64 prompt token ids."""
    g = torch.Generator("cpu").manual_seed(seed)

    def rnd(shape):
        return (torch.randn(shape, generator=g, dtype=torch.float32) * 0.02).to(torch.bfloat16)

    gn = torch.Generator("cpu").manual_seed(seed + 1)

    def gain(n):
        if norm_jitter <= 0.0:
            return torch.ones(n, dtype=torch.bfloat16)
        return (1.0 + norm_jitter * torch.randn(n, generator=gn, dtype=torch.float32)).to(torch.bfloat16)

    H, D = cfg.hidden_size, cfg.head_dim
    shapes = _proj_shapes(cfg)
    state = {"model.embed_tokens.weight": rnd((cfg.vocab_size, H))}
    for i in range(cfg.num_layers):
        p = f"model.layers.{i}"
        for proj in PROJ:
            state[f"{p}.{proj}.weight"] = rnd(shapes[proj])
    for i in range(cfg.num_layers):
        p = f"model.layers.{i}"
        state[f"{p}.input_layernorm.weight"] = gain(H)
        state[f"{p}.self_attn.q_norm.weight"] = gain(D)
        state[f"{p}.self_attn.k_norm.weight"] = gain(D)
        state[f"{p}.post_attention_layernorm.weight"] = gain(H)
    state["model.norm.weight"] = gain(H)
    state["lm_head.weight"] = state["model.embed_tokens.weight"]
    prompt = torch.randint(0, cfg.vocab_size, (prompt_len,), generator=g, dtype=torch.int64)
    return state, prompt


def state_digest(state: dict) -> str:
    """sha256 over the raw bytes of every tensor (sorted keys) — detects drift in the generator."""
    h = hashlib.sha256()
    for k in sorted(state):
        t = state[k].contiguous().cpu()
        h.update(k.encode())
        h.update(t.view(torch.uint8).numpy().tobytes() if t.dtype != torch.uint8 else t.numpy().tobytes())
    return h.hexdigest()


def quantize_state(state: dict, cfg: ModelConfig, device, weight_format: str = "int8") -> dict:
    """bench_int8.py:27-55 without the HF load: every projection and the LM head
    become ``(int8, fp32 scale)`` pairs computed on ``device``. No counterpart in the
    reference: ``weight_format="fp8"`` gives ``(FP8 E4M3 codes, fp32 row scale)`` pairs;
    ``"int4"`` gives the seven layer projections as ``(packed nibbles uint8 [out, in / 2],
    fp32 group scales [out, in / 128])`` and keeps the LM head INT8 per row. Norms and the
    embedding stay bf16 (moved to ``device``). ``pack_int8`` packs any of them."""
    if weight_format not in ("int8", "fp8", "int4"):
        raise ValueError(f"weight_format must be 'int8', 'fp8' or 'int4', got {weight_format!r}")
    from .formats import quantize_fp8, quantize_int4
    quant = {"int8": quantize_per_channel, "fp8": quantize_fp8, "int4": quantize_int4}[weight_format]
    q = {}
    for k, v in state.items():
        if k == "lm_head.weight":
            q[k] = (quantize_per_channel if weight_format == "int4" else quant)(v.to(device))
        elif any(k.endswith(f"{p}.weight") for p in PROJ):
            q[k] = quant(v.to(device))
        else:
            q[k] = v.to(device)
    return q


def _layer_list(state: dict, cfg: ModelConfig, pick):
    out = []
    for i in range(cfg.num_layers):
        p = f"model.layers.{i}"
        out.append(state[f"{p}.input_layernorm.weight"].contiguous())
        for proj in ("self_attn.q_proj", "self_attn.k_proj", "self_attn.v_proj"):
            out.append(pick(state[f"{p}.{proj}.weight"]).contiguous())
        out.append(state[f"{p}.self_attn.q_norm.weight"].contiguous())
        out.append(state[f"{p}.self_attn.k_norm.weight"].contiguous())
        out.append(pick(state[f"{p}.self_attn.o_proj.weight"]).contiguous())
        out.append(state[f"{p}.post_attention_layernorm.weight"].contiguous())
        for proj in ("mlp.gate_proj", "mlp.up_proj", "mlp.down_proj"):
            out.append(pick(state[f"{p}.{proj}.weight"]).contiguous())
    return out


def pack_int8(qstate: dict, cfg: ModelConfig):
    """Returns ``(embed, layer_tensors[11L], layer_scales[7L], lm_int8, lm_scale, final_norm)``."""
    layers = _layer_list(qstate, cfg, lambda t: t[0] if isinstance(t, tuple) else t)
    scales = []
    for i in range(cfg.num_layers):
        p = f"model.layers.{i}"
        for proj in PROJ:
            scales.append(qstate[f"{p}.{proj}.weight"][1].contiguous())
    lm_q, lm_s = qstate["lm_head.weight"]
    return (qstate["model.embed_tokens.weight"].contiguous(), layers, scales, lm_q.contiguous(),
            lm_s.contiguous(), qstate["model.norm.weight"].contiguous())


def pack_bf16(state: dict, cfg: ModelConfig, device=None):
    """Returns ``(embed, layer_tensors[11L], final_norm, lm_head)`` (a10_decode.py:289-325 order)."""
    mv = (lambda t: t.to(device)) if device is not None else (lambda t: t)
    st = {k: mv(v) for k, v in state.items()}
    layers = _layer_list(st, cfg, lambda t: t)
    return (st["model.embed_tokens.weight"].contiguous(), layers, st["model.norm.weight"].contiguous(),
            st["lm_head.weight"].contiguous())
