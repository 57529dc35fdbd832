"""A10Chat on the GPU (run with -m gpu): the reference's chat front end (a10_chat.py:222-604).

The model is a 2-layer checkpoint of the Qwen3-0.6B layer shape (4096-word vocabulary,
tied head) with a word-level tokenizer whose EOS word is chosen from the oracle's
continuation. It is loaded through ``A10Chat(model_path, int8=...)``. The gates:

* ``generate`` returns the float64 oracle's greedy tokens up to and including EOS, as
  text. Its steps run in launches of 32 steps, with the INT8 prompt prefilled in one
  launch once it is long enough.
* ``generate_stream`` (one launch per step) prints and returns the same text.
* Over two turns, ``chat`` holds the oracle's reply to each turn's ChatML prompt,
  cleaned, and the second turn's prompt carries the first turn's reply. The prompts
  come from the tokenizer, so most template words are its unknown word.
"""
from __future__ import annotations

import pytest
import torch

from .ckpt import oracle_tokens, text_of, tied_state_with_defaults, write_checkpoint

pytestmark = pytest.mark.gpu

N_NEW = 24
S = 160


@pytest.fixture(scope="module")
def seeded(mq):
    cfg = mq.QWEN3_0_6B.with_(name="chat-gpu", num_layers=2, vocab_size=4096)
    state, prompt = mq.random_init_state(cfg, seed=13, norm_jitter=0.2)
    return cfg, state, prompt.tolist()


def _cut(toks, eos):
    return toks[:toks.index(eos) + 1] if eos in toks else toks


@pytest.mark.parametrize("int8", [True, False])
def test_a10chat_matches_the_oracle(mq, dev, seeded, tmp_path, int8, capsys):
    cfg, state, prompt = seeded
    want_state = tied_state_with_defaults(state, cfg)
    want = oracle_tokens(mq, cfg, want_state, prompt, N_NEW, S, int8)
    # EOS: the first token from the eleventh on that does not occur before it
    k = next(i for i in range(10, N_NEW) if want[i] not in want[:i])
    eos = want[k]
    path = write_checkpoint(tmp_path / "ckpt", state, cfg, fp32_shard=False, tokenizer=True, eos=eos)
    print(f"A10Chat int8={int8} eos={eos}", flush=True)
    chat = mq.A10Chat(path, max_seq_len=S, int8=int8, device=dev)
    tok = chat.tokenizer

    text = chat.generate(text_of(prompt), N_NEW, show_speed=False)
    assert chat.last_stats["tokens"] == want[:k + 1], (chat.last_stats["tokens"], want)
    assert text == text_of(want[:k])

    capsys.readouterr()
    assert chat.generate_stream(text_of(prompt), N_NEW) == text
    assert capsys.readouterr().out.startswith(text)

    turns = [text_of(prompt[:3]), text_of(prompt[3:7])]
    conv = []
    for line in turns:
        conv.append({"role": "user", "content": line})
        ids = tok.encode(mq.chat_prompt(conv))
        toks = _cut(oracle_tokens(mq, cfg, want_state, ids, N_NEW, S, int8), eos)
        conv.append({"role": "assistant", "content": mq.clean_reply(tok.decode(toks, skip_special_tokens=True))})
    feed = iter(turns + ["exit"])
    got = chat.chat(lambda _p: next(feed), max_new_tokens=N_NEW)
    assert got == conv, (got, conv)
    del chat
    torch.cuda.empty_cache()
