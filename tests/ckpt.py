"""Writes small HF-style checkpoint directories for the loader tests (no network).

A directory holds what ``A10Decoder(model_path)`` reads the way the reference's
``_load_model`` reads a Qwen3 checkpoint (a10_decode.py:281-325): safetensors
shards under HF key names, ``config.json``, and optionally a tokenizer
(``tokenizer.json`` + ``tokenizer_config.json``, a word-level vocabulary
``w0 .. w{V-1}`` so that token ids and text map one to one).
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
