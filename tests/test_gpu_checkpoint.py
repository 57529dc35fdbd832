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

from .ckpt import oracle_tokens, text_of, tied_state_with_defaults, write_checkpoint

pytestmark = pytest.mark.gpu

N_NEW = 16
S = 64


@pytest.fixture(scope="module")
def seeded(mq):
    cfg = mq.QWEN3_0_6B.with_(name="ckpt-gpu", num_layers=2, vocab_size=4096)
    state, prompt = mq.random_init_state(cfg, seed=11, norm_jitter=0.2)
    return cfg, state, prompt.tolist()


@pytest.mark.parametrize("int8", [True, False])
def test_a10decoder_from_checkpoint_with_tokenizer(mq, dev, seeded, tmp_path, int8):
    cfg, state, prompt = seeded
    want_state = tied_state_with_defaults(state, cfg, drop_qk_norm_layers=(1,))
    want = oracle_tokens(mq, cfg, want_state, prompt, N_NEW, S, int8)
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
