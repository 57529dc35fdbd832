"""A10Chat's host logic on the CPU (a10_chat.py:222-604).

``chat_prompt`` is checked against the ChatML text that a10_chat.py:584-591 builds,
written out literally here. ``clean_reply`` is checked on the cases of
a10_chat.py:593-601, and ``fit_prompt`` on the truncation rule of
a10_chat.py:339-342. The token bookkeeping of ``generate``, ``generate_stream`` and
``chat`` runs over a stand-in for the kernel decoder. There, each step's token is a
hash of every token fed since the last reset, so a token fed out of order, twice, or
not at all changes every later token. The expected tokens come from stepping that rule
one token at a time. The real kernel under A10Chat is checked against the oracle in
tests/test_gpu_chat.py.
"""
from __future__ import annotations

import hashlib
from types import SimpleNamespace

import pytest

from .ckpt import text_of, write_tokenizer

V = 64


def _rule(fed) -> int:
    return hashlib.sha256(bytes(str(fed), "ascii")).digest()[0] % V


class FakeSteps:
    """The kernel decoder's surface that A10Chat uses, on the CPU."""
    PREFILL_MIN = 16

    def __init__(self, max_seq_len=256, prefill=False):
        self.max_seq_len = max_seq_len
        self.can_prefill = prefill
        self.sessions = []
        self.calls = []
        self.pending = None

    def reset(self):
        self.sessions.append([])

    def set_sampling(self, temperature=0.0, seed=0):
        self.calls.append(("sampling", temperature, seed))

    def prefill_supported(self):
        return self.can_prefill

    def _feed(self, t):
        fed = self.sessions[-1]
        assert len(fed) < self.max_seq_len, "position past max_seq_len"
        fed.append(int(t))
        return _rule(fed)

    def prefill(self, ids):
        self.calls.append(("prefill", len(ids)))
        for t in ids:
            self._feed(t)

    def launch_step(self, t):
        self.pending = self._feed(t)

    def wait_token(self):
        tok, self.pending = self.pending, None
        return tok

    def decode_step(self, t):
        self.launch_step(t)
        return self.wait_token()

    def generate(self, ids, n):
        self.calls.append(("generate", len(ids), n))
        out = []
        for t in ids:
            tok = self._feed(t)
        out.append(tok)
        while len(out) < n:
            out.append(self._feed(out[-1]))
        return out


def _stepped(ids, n):
    """The tokens of one decode step per token: the prompt, then each token fed back."""
    fed = list(ids)
    out = [_rule(fed)]
    while len(out) < n:
        fed.append(out[-1])
        out.append(_rule(fed))
    return out


def _eos_after(ids, at_least):
    """A token that first appears at index >= at_least of the stepped continuation, and where."""
    toks = _stepped(ids, 400)
    k = next(i for i in range(at_least, 400) if toks[i] not in toks[:i])
    return toks[k], k


@pytest.fixture()
def make_chat(mq, tmp_path):
    def make(eos=None, max_seq_len=256, prefill=False, **kw):
        d = tmp_path / f"tok{eos}"
        d.mkdir(exist_ok=True)
        write_tokenizer(d, V, eos)
        tok = mq.load_tokenizer(d)
        steps = FakeSteps(max_seq_len, prefill)
        model = SimpleNamespace(decoder=steps, tokenizer=tok, max_seq_len=max_seq_len)
        return mq.A10Chat(decoder=model, **kw), steps, tok
    return make


def test_chat_prompt_is_the_chatml_text(mq):
    conv = [{"role": "user", "content": "hi"}, {"role": "assistant", "content": "hello there"},
            {"role": "user", "content": "and now?"}]
    assert mq.chat_prompt(conv) == (
        "<|im_start|>system\nYou are a helpful assistant. Be concise and direct. /nothink<|im_end|>\n"
        "<|im_start|>user\nhi<|im_end|>\n"
        "<|im_start|>assistant\nhello there<|im_end|>\n"
        "<|im_start|>user\nand now?<|im_end|>\n"
        "<|im_start|>assistant\n")
    assert mq.chat_prompt([], system="S") == "<|im_start|>system\nS<|im_end|>\n<|im_start|>assistant\n"
    # any role that is not "user" is written as the assistant's (a10_chat.py:589-590)
    assert "<|im_start|>assistant\nx<|im_end|>" in mq.chat_prompt([{"role": "tool", "content": "x"}])


@pytest.mark.parametrize("text, want", [
    ("  Paris.  ", "Paris."),
    ("Paris.<|im_end|>\n<|im_start|>user\nmore", "Paris."),
    ("<think>\nlet me see\n</think>\n\nParis.", "Paris."),
    ("A <think>x</think>B<think>y\nz</think> C", "A B C"),
    ("Paris. <think> still going", "Paris."),
    ("<think> never closed", None),
    ("", None),
    ("<think>a</think><|im_end|>tail", None),
])
def test_clean_reply(mq, text, want):
    assert mq.clean_reply(text) == (mq.chat.THINKING_PLACEHOLDER if want is None else want)


def test_fit_prompt(mq):
    fit = mq.chat.fit_prompt
    ids = list(range(100))
    assert fit(ids[:87], 128, 40) == ids[:87]           # 87 < 128 - 40: kept whole
    assert fit(ids[:88], 128, 40) == ids[1:88]          # 88 >= 128 - 40: the last 87 tokens
    assert fit(ids, 128, 40) == ids[13:]
    assert fit([5], 3, 1) == [5]
    for bad in (0, -1, 2.0, 127, 128):
        with pytest.raises(ValueError):
            fit(ids, 128, bad)


def test_speed_line(mq):
    line = mq.chat.speed_line(10, 0.5, 5, 2.0, 2.5)
    assert line == "[prefill: 10 tok @ 20 tok/s | decode: 5 tok @ 2 tok/s | total: 2500ms]"
    assert mq.chat.speed_line(10, 0.5, 1, 0.0, 0.5) == "[prefill: 10 tok @ 20 tok/s | decode: 1 tok | total: 500ms]"


def test_generate_follows_the_steps_and_stops_after_eos(make_chat):
    prompt = [3, 9, 27, 17, 50]
    eos, k = _eos_after(prompt, 40)                  # EOS past the first launch of 32 steps
    chat, steps, tok = make_chat(eos)
    text = chat.generate(text_of(prompt), max_new_tokens=200, show_speed=False)
    want = _stepped(prompt, k + 1)
    assert chat.last_stats["tokens"] == want and want[-1] == eos
    assert text == text_of(want[:-1])                # EOS is a special token: not in the text
    # every generated token but EOS fed back once; the launch that made EOS ran its other steps
    fed = steps.sessions[-1]
    assert fed[:len(prompt) + k] == prompt + want[:-1] and len(fed) < len(prompt) + k + 32
    gens = [c for c in steps.calls if c[0] == "generate"]
    assert all(c[1] == 1 for c in gens) and gens[0][2] == 32
    assert ("sampling", 0.0, 0) in steps.calls

    # a budget shorter than the reply: exactly max_new_tokens tokens, no EOS
    text = chat.generate(text_of(prompt), max_new_tokens=k - 3, show_speed=False)
    assert chat.last_stats["tokens"] == _stepped(prompt, k - 3)
    assert chat.generate(text_of(prompt), max_new_tokens=1, show_speed=False) == text_of(_stepped(prompt, 1))


def test_generate_stream_prints_what_generate_returns(make_chat, capsys):
    prompt = [7, 1, 60, 33]
    eos, k = _eos_after(prompt, 20)
    chat, steps, tok = make_chat(eos)
    want = chat.generate(text_of(prompt), 100, show_speed=False)
    capsys.readouterr()
    got = chat.generate_stream(text_of(prompt), 100)
    printed = capsys.readouterr().out
    assert got == want
    assert printed.startswith(want) and printed[len(want):].startswith("\n[prefill: 4 tok")
    # one launch per step: it stops feeding at EOS, and fed what generate fed up to there
    assert steps.sessions[-1] == steps.sessions[-2][:len(prompt) + k]


def test_long_prompt_is_prefilled_then_stepped(make_chat):
    prompt = [(5 * i + 2) % V for i in range(40)]
    chat, steps, tok = make_chat(None, prefill=True)
    chat.generate(text_of(prompt), 10, show_speed=False)
    assert ("prefill", 39) in steps.calls
    assert chat.last_stats["tokens"] == _stepped(prompt, 10)
    # short prompts (fewer than PREFILL_MIN + 1 tokens) run as decode steps
    steps.calls.clear()
    chat.generate(text_of(prompt[:16]), 10, show_speed=False)
    assert not [c for c in steps.calls if c[0] == "prefill"]
    assert chat.last_stats["tokens"] == _stepped(prompt[:16], 10)


def test_prompt_truncation(make_chat, capsys):
    prompt = [(3 * i + 1) % V for i in range(60)]
    chat, steps, tok = make_chat(None, max_seq_len=64)
    chat.generate(text_of(prompt), 8, show_speed=False)
    assert "prompt too long (60 tokens)" in capsys.readouterr().out
    kept = prompt[-(64 - 8 - 1):]
    assert steps.sessions[-1][:len(kept)] == kept
    assert chat.last_stats["tokens"] == _stepped(kept, 8)
    assert len(steps.sessions[-1]) == len(kept) + 7 <= 64
    with pytest.raises(ValueError):
        chat.generate(text_of(prompt), 63)
    with pytest.raises(ValueError):
        chat.generate_stream(text_of(prompt), 0)


def _inputs(lines):
    it = iter(lines)

    def read(_prompt):
        try:
            return next(it)
        except StopIteration:
            raise EOFError from None
    return read


def test_chat_loop_history_clear_and_exit(mq, make_chat, capsys):
    chat, steps, tok = make_chat(None)
    conv = chat.chat(_inputs(["", "w1 w2", "w5", "clear", "w3", "QUIT", "w9"]), max_new_tokens=6)
    out = capsys.readouterr().out
    assert "[Conversation cleared]" in out and out.rstrip().endswith("Goodbye!")
    assert len(steps.sessions) == 3                  # the empty line and the line after quit never ran
    first = [{"role": "user", "content": "w1 w2"}]
    assert steps.sessions[0][:len(tok.encode(mq.chat_prompt(first)))] == tok.encode(mq.chat_prompt(first))
    reply1 = mq.clean_reply(tok.decode(_stepped(tok.encode(mq.chat_prompt(first)), 6), skip_special_tokens=True))
    second = first + [{"role": "assistant", "content": reply1}, {"role": "user", "content": "w5"}]
    p2 = tok.encode(mq.chat_prompt(second))
    assert steps.sessions[1][:len(p2)] == p2         # the second turn carries the first turn's reply
    third = [{"role": "user", "content": "w3"}]
    p3 = tok.encode(mq.chat_prompt(third))
    assert steps.sessions[2][:len(p3)] == p3         # cleared: history restarts
    reply3 = mq.clean_reply(tok.decode(_stepped(p3, 6), skip_special_tokens=True))
    assert conv == third + [{"role": "assistant", "content": reply3}]
    assert f"\n{reply3}\n" in out

    # end of input ends the loop too
    chat2, steps2, _ = make_chat(None)
    assert chat2.chat(_inputs(["w4"]), max_new_tokens=3)[0] == {"role": "user", "content": "w4"}
    assert len(steps2.sessions) == 1


def test_chat_needs_a_tokenizer(mq):
    with pytest.raises(ValueError):
        mq.A10Chat()
    with pytest.raises(ValueError):
        mq.A10Chat(decoder=SimpleNamespace(decoder=FakeSteps(), tokenizer=None, max_seq_len=256))
