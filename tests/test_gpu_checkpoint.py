"""A10Decoder from a checkpoint directory on the GPU (run with -m gpu).

The reference's A10Decoder loads an HF checkpoint and its tokenizer and generates
from a text prompt (a10_decode.py:281-327, 358-393; INT8 quantization at load,
bench_int8.py:27-55). Here a 2-layer checkpoint of the Qwen3-0.6B layer shape
(4096-word vocabulary, tied head, layer 1 without q/k-norm gains, one shard stored
fp32, a word-level tokenizer with an EOS word) is written under ``tmp_path`` and
loaded through ``A10Decoder(model_path, int8=...)``. Gates: the generated tokens
equal the float64 oracle's greedy tokens computed from the state dict the checkpoint
was written from (the oracle quantizes with its own CPU restatement for INT8), the
text is the tokenizer's decoding of prompt + tokens, and generation stops after the
EOS token.
"""
from __future__ import annotations

import pytest
import torch

from oracle.quant import quantize_per_channel as ref_quantize
from oracle.ref_cpu import Dims, RefDecoder, greedy_generate

from .ckpt import text_of, tied_state_with_defaults, write_checkpoint

pytestmark = pytest.mark.gpu

N_NEW = 16
S = 64


def _oracle_tokens(mq, cfg, state, prompt, int8):
    """Greedy tokens of the float64 oracle from a (tied, defaulted) bf16 state dict."""
    layers = []
    scales = [] if int8 else None
    for i in range(cfg.num_layers):
        p = f"model.layers.{i}"
        layers.append(state[f"{p}.input_layernorm.weight"])
        for n in ("q", "k", "v"):
            w = state[f"{p}.self_attn.{n}_proj.weight"]
            layers.append(w)
        layers.append(state[f"{p}.self_attn.q_norm.weight"])
        layers.append(state[f"{p}.self_attn.k_norm.weight"])
        layers.append(state[f"{p}.self_attn.o_proj.weight"])
        layers.append(state[f"{p}.post_attention_layernorm.weight"])
        for n in ("gate", "up", "down"):
            layers.append(state[f"{p}.mlp.{n}_proj.weight"])
    lm, lm_s = state["lm_head.weight"], None
    if int8:
        qi = [1, 2, 3, 6, 8, 9, 10]                  # projections in each layer's 11 tensors
        for i in range(cfg.num_layers):
            for j in qi:
                q, s = ref_quantize(layers[11 * i + j])
                layers[11 * i + j] = q
                scales.append(s)
        lm, lm_s = ref_quantize(lm)
    cos, sin = mq.precompute_rope_freqs(cfg.head_dim, S, cfg.rope_theta)
    ref = RefDecoder(Dims(vocab_size=cfg.vocab_size), state["model.embed_tokens.weight"], layers, scales,
                     state["model.norm.weight"], lm, lm_s, cos, sin, cfg.num_layers, S)
    toks, _ = greedy_generate(ref, prompt, N_NEW)
    return toks


@pytest.fixture(scope="module")
def seeded(mq):
    cfg = mq.QWEN3_0_6B.with_(name="ckpt-gpu", num_layers=2, vocab_size=4096)
    state, prompt = mq.random_init_state(cfg, seed=11, norm_jitter=0.2)
    return cfg, state, prompt.tolist()


@pytest.mark.parametrize("int8", [True, False])
def test_a10decoder_from_checkpoint_with_tokenizer(mq, dev, seeded, tmp_path, int8):
    cfg, state, prompt = seeded
    want_state = tied_state_with_defaults(state, cfg, drop_qk_norm_layers=(1,))
    want = _oracle_tokens(mq, cfg, want_state, prompt, int8)
    # EOS: the first token from the eleventh on that does not occur before it (else none)
    k = next((i for i in range(10, N_NEW) if want[i] not in want[:i]), None)
    eos = want[k] if k is not None else None
    path = write_checkpoint(tmp_path / "ckpt", state, cfg, drop_qk_norm_layers=(1,), fp32_shard=True,
                            tokenizer=True, eos=eos)
    print(f"checkpoint decoder int8={int8} eos={eos}", flush=True)
    dec = mq.A10Decoder(path, max_seq_len=S, int8=int8, device=dev)
    assert dec.config.num_layers == 2 and dec.config.vocab_size == 4096
    assert dec.tokenizer is not None and dec.tokenizer.eos_token_id == eos

    ids, tok_s, _ = dec.generate(prompt, N_NEW)                     # token ids in, ids out
    stop = want[:k + 1] if k is not None else want
    assert ids[:len(prompt)] == prompt
    assert ids[len(prompt):] == stop, (ids[len(prompt):], want)
    assert tok_s > 0

    text, _, _ = dec.generate(text_of(prompt), N_NEW)               # text in, text out
    assert text == text_of([t for t in prompt + stop if t != eos])
    del dec
    torch.cuda.empty_cache()
