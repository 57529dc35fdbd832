"""Writes small HF-style checkpoint directories for the loader tests (no network).

A directory holds what ``A10Decoder(model_path)`` reads the way the reference's
``_load_model`` reads a Qwen3 checkpoint (a10_decode.py:281-325): safetensors
shards under HF key names, ``config.json``, and optionally a tokenizer
(``tokenizer.json`` + ``tokenizer_config.json``, a word-level vocabulary
``w0 .. w{V-1}`` so that token ids and text map one to one). ``oracle_tokens`` gives
the float64 oracle's greedy tokens for the state dict such a directory was written from.
"""
from __future__ import annotations

import json
from pathlib import Path

import torch


def write_checkpoint(path, state: dict, cfg, *, untie: bool = False, drop_qk_norm_layers=(),
                     fp32_shard: bool = True, tokenizer: bool = False, eos: int | None = None) -> Path:
    """Write ``state`` (bf16 tensors under HF keys) to ``path`` in two shards: the embedding,
    final norm and layer 0 in ``model-00001-of-00002.safetensors``, the rest in the second
    (stored as fp32 when ``fp32_shard``). ``lm_head.weight`` is left out (a tied checkpoint)
    unless ``untie``; the q/k-norm gains of ``drop_qk_norm_layers`` are left out. Returns
    ``path``."""
    from safetensors.torch import save_file
    path = Path(path)
    path.mkdir(parents=True, exist_ok=True)
    first, second = {}, {}
    for k, v in state.items():
        if k == "lm_head.weight" and not untie:
            continue
        if any(k in (f"model.layers.{i}.self_attn.q_norm.weight", f"model.layers.{i}.self_attn.k_norm.weight")
               for i in drop_qk_norm_layers):
            continue
        if k.startswith("model.layers.0.") or k in ("model.embed_tokens.weight", "model.norm.weight"):
            first[k] = v.contiguous().clone()
        else:
            second[k] = (v.float() if fp32_shard else v).contiguous().clone()
    save_file(first, str(path / "model-00001-of-00002.safetensors"))
    save_file(second, str(path / "model-00002-of-00002.safetensors"))
    (path / "config.json").write_text(json.dumps({
        "architectures": ["Qwen3ForCausalLM"], "model_type": "qwen3",
        "num_hidden_layers": cfg.num_layers, "hidden_size": cfg.hidden_size,
        "intermediate_size": cfg.intermediate_size, "num_attention_heads": cfg.num_q_heads,
        "num_key_value_heads": cfg.num_kv_heads, "head_dim": cfg.head_dim, "vocab_size": cfg.vocab_size,
        "rms_norm_eps": cfg.rms_eps, "rope_theta": cfg.rope_theta, "tie_word_embeddings": not untie,
        "torch_dtype": "bfloat16"}))
    if tokenizer:
        write_tokenizer(path, cfg.vocab_size, eos)
    return path


def write_tokenizer(path, vocab_size: int, eos: int | None = None) -> None:
    """A word-level tokenizer over ``w0 .. w{vocab_size-1}`` (whitespace split), EOS ``w{eos}``."""
    from tokenizers import Tokenizer, decoders, models, pre_tokenizers
    path = Path(path)
    tok = Tokenizer(models.WordLevel({f"w{i}": i for i in range(vocab_size)}, unk_token="w0"))
    tok.pre_tokenizer = pre_tokenizers.WhitespaceSplit()
    tok.decoder = decoders.WordPiece(prefix="##")       # joins words with single spaces
    tok.save(str(path / "tokenizer.json"))
    conf = {"tokenizer_class": "PreTrainedTokenizerFast", "unk_token": "w0"}
    if eos is not None:
        conf["eos_token"] = f"w{eos}"
    (path / "tokenizer_config.json").write_text(json.dumps(conf))


def text_of(ids) -> str:
    return " ".join(f"w{int(t)}" for t in ids)


def tied_state_with_defaults(state: dict, cfg, drop_qk_norm_layers=()) -> dict:
    """What a loader must return for a checkpoint written from ``state`` with the head tied
    and the listed layers' q/k-norm gains dropped: the head is the embedding and the dropped
    gains are ones (a10_decode.py:304-309)."""
    want = dict(state)
    want["lm_head.weight"] = state["model.embed_tokens.weight"]
    for i in drop_qk_norm_layers:
        for n in ("q_norm", "k_norm"):
            want[f"model.layers.{i}.self_attn.{n}.weight"] = torch.ones(cfg.head_dim, dtype=torch.bfloat16)
    return want


def oracle_tokens(mq, cfg, state, prompt, n_new: int, max_seq_len: int, int8: bool, with_margins: bool = False):
    """Greedy tokens of the float64 oracle for ``prompt`` from a (tied, defaulted) bf16 state
    dict; with ``int8`` the oracle quantizes every projection and the head with its own CPU
    restatement (bench_int8.py:19-24). With ``with_margins`` also the top-2 logit margins."""
    from oracle.quant import quantize_per_channel as ref_quantize
    from oracle.ref_cpu import Dims, RefDecoder, greedy_generate
    layers = []
    scales = [] if int8 else None
    for i in range(cfg.num_layers):
        p = f"model.layers.{i}"
        layers.append(state[f"{p}.input_layernorm.weight"])
        for n in ("q", "k", "v"):
            layers.append(state[f"{p}.self_attn.{n}_proj.weight"])
        layers.append(state[f"{p}.self_attn.q_norm.weight"])
        layers.append(state[f"{p}.self_attn.k_norm.weight"])
        layers.append(state[f"{p}.self_attn.o_proj.weight"])
        layers.append(state[f"{p}.post_attention_layernorm.weight"])
        for n in ("gate", "up", "down"):
            layers.append(state[f"{p}.mlp.{n}_proj.weight"])
    lm, lm_s = state["lm_head.weight"], None
    if int8:
        for i in range(cfg.num_layers):
            for j in (1, 2, 3, 6, 8, 9, 10):             # projections in each layer's 11 tensors
                q, s = ref_quantize(layers[11 * i + j])
                layers[11 * i + j] = q
                scales.append(s)
        lm, lm_s = ref_quantize(lm)
    cos, sin = mq.precompute_rope_freqs(cfg.head_dim, max_seq_len, cfg.rope_theta)
    ref = RefDecoder(Dims(vocab_size=cfg.vocab_size), state["model.embed_tokens.weight"], layers, scales,
                     state["model.norm.weight"], lm, lm_s, cos, sin, cfg.num_layers, max_seq_len)
    toks, margins = greedy_generate(ref, prompt, n_new)
    return (toks, margins) if with_margins else toks
