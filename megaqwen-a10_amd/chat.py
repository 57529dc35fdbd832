"""Chat front end over the decode step: the reference's ``A10Chat`` (a10_chat.py:222-604).

The reference loads Qwen3-0.6B and its tokenizer and then does three things. It
formats the conversation in the Qwen ChatML template under a fixed system message
(a10_chat.py:584-591). It decodes one token per launch of its BF16 kernel,
prefilling the prompt one step per token and printing each token as it comes
(a10_chat.py:413-510). It keeps the cleaned replies as history for the next turn
(a10_chat.py:593-604).

``A10Chat`` here keeps that surface (``generate``, ``generate_stream``, ``chat``) on
top of ``A10Decoder``: BF16 weights by default, as the reference, or per-row INT8
with ``int8=True``. Every turn starts from an empty KV cache, as in the reference
(a10_chat.py:331).

The prompt is prefilled in one prompt-batched launch where the decoder supports it
(INT8), else as decode steps queued back to back with one wait at the end.
``generate`` runs its steps in launches of ``GENERATE_CHUNK`` steps each (tokens
handed on on the device) and stops after the launch that produced EOS.
``generate_stream`` runs one launch per step and queues the next step before it
decodes and prints the text of the last, so the host's tokenizer work overlaps
the step. All paths give the same tokens as one decode step per token.

    python megaqwen-a10_amd/chat.py --model DIR [--int8] [--max-new-tokens 500]
"""
from __future__ import annotations

if __name__ == "__main__" and not __package__:
    # run as a script: load the package (its directory name is not an identifier) and hand over
    import sys as _sys
    from pathlib import Path as _Path
    _sys.path.insert(0, str(_Path(__file__).resolve().parents[1]))
    import __graft_entry__ as _entry
    _sys.exit(_entry.load_package().chat.main())

import re
import sys
import time

SYSTEM_PROMPT = "You are a helpful assistant. Be concise and direct. /nothink"    # a10_chat.py:585
THINKING_PLACEHOLDER = "[Model is thinking... try asking more directly]"           # a10_chat.py:601
GENERATE_CHUNK = 32      # decode steps per launch in generate(): EOS is looked for between launches

_THINK = re.compile(r"<think>.*?</think>", re.DOTALL)


def chat_prompt(conversation, system: str = SYSTEM_PROMPT) -> str:
    """The ChatML text of ``conversation`` (a list of ``{"role", "content"}``), as
    a10_chat.py:584-591 builds it. It has the system turn, then each message as
    ``<|im_start|>ROLE\\nCONTENT<|im_end|>\\n``, then an open assistant turn. Any role
    other than ``"user"`` is written as ``assistant``, as there."""
    parts = [f"<|im_start|>system\n{system}<|im_end|>\n"]
    for msg in conversation:
        role = "user" if msg["role"] == "user" else "assistant"
        parts.append(f"<|im_start|>{role}\n{msg['content']}<|im_end|>\n")
    parts.append("<|im_start|>assistant\n")
    return "".join(parts)


def clean_reply(text: str) -> str:
    """The reply kept in the history (a10_chat.py:593-601). The text is cut at the first
    ``<|im_end|>`` and every ``<think>...</think>`` block is removed. An unclosed
    ``<think>`` is dropped with everything after it. The result is stripped, and
    ``THINKING_PLACEHOLDER`` is returned when nothing is left."""
    reply = text.split("<|im_end|>")[0].strip()
    reply = _THINK.sub("", reply).strip()
    if "<think>" in reply:
        reply = reply.split("<think>")[0].strip()
    return reply or THINKING_PLACEHOLDER


def fit_prompt(ids, max_seq_len: int, max_new_tokens: int) -> list:
    """The prompt ids that fit with ``max_new_tokens`` generated tokens (a10_chat.py:339-342).
    A prompt of at least ``max_seq_len - max_new_tokens`` tokens keeps its last
    ``max_seq_len - max_new_tokens - 1``. Raises ``ValueError`` when ``max_new_tokens``
    is not positive, or too large to leave a prompt token."""
    if not isinstance(max_new_tokens, int) or max_new_tokens <= 0:
        raise ValueError(f"max_new_tokens must be a positive int, got {max_new_tokens!r}")
    keep = max_seq_len - max_new_tokens - 1
    if keep < 1:
        raise ValueError(f"max_new_tokens {max_new_tokens} leaves no room for a prompt in max_seq_len {max_seq_len}")
    ids = list(ids)
    return ids[-keep:] if len(ids) >= max_seq_len - max_new_tokens else ids


def speed_line(prompt_tokens: int, prefill_s: float, new_tokens: int, decode_s: float, total_s: float) -> str:
    """The line printed after a reply (a10_chat.py:404-406). Prefill is the prompt's
    tokens over the time to the first generated token; decode is the generated tokens
    after the first over the time they took."""
    pre = f"prefill: {prompt_tokens} tok @ {prompt_tokens / prefill_s:.0f} tok/s" if prefill_s > 0 else \
        f"prefill: {prompt_tokens} tok"
    if new_tokens > 1 and decode_s > 0:
        dec = f"decode: {new_tokens} tok @ {(new_tokens - 1) / decode_s:.0f} tok/s"
    else:
        dec = f"decode: {new_tokens} tok"
    return f"[{pre} | {dec} | total: {total_s * 1e3:.0f}ms]"


class A10Chat:
    """a10_chat.py:222-604 over ``A10Decoder``.

    ``A10Chat(model_path, max_seq_len=2048, int8=False)`` loads a local checkpoint
    directory with its tokenizer (``A10Decoder``). ``decoder=`` takes an already
    built ``A10Decoder`` instead. ``temperature`` / ``seed`` set the token choice of
    every reply (``set_sampling``); the default 0 is the reference's greedy argmax.
    Raises ``ValueError`` when the model has no tokenizer."""

    def __init__(self, model_path=None, max_seq_len: int = 2048, *, int8: bool = False, device="cuda",
                 decoder=None, system: str = SYSTEM_PROMPT, temperature: float = 0.0, seed: int = 0):
        if decoder is None:
            if model_path is None:
                raise ValueError("A10Chat needs a checkpoint directory (model_path) or a decoder")
            from .decoder import A10Decoder
            decoder = A10Decoder(model_path, max_seq_len, int8=int8, device=device)
        if getattr(decoder, "tokenizer", None) is None:
            raise ValueError("A10Chat needs a model with a tokenizer")
        self.model = decoder
        self.tokenizer = decoder.tokenizer
        self.max_seq_len = decoder.max_seq_len
        self.system = system
        self.temperature = temperature
        self.seed = seed
        self.conversation = []
        self.last_stats = None

    # -- host pieces -----------------------------------------------------------------------
    def _prompt_ids(self, prompt: str, max_new_tokens: int, warn: bool, out) -> list:
        ids = self.tokenizer.encode(prompt)
        if not ids:
            raise ValueError("the prompt encodes to no tokens")
        fitted = fit_prompt(ids, self.max_seq_len, max_new_tokens)
        if warn and len(fitted) < len(ids):
            print(f"Warning: prompt too long ({len(ids)} tokens), truncating", file=out)
        return fitted

    def _first_token(self, ids) -> int:
        """Runs the prompt from position 0 and returns the last prompt step's token."""
        k = self.model.decoder
        k.reset()
        k.set_sampling(self.temperature, self.seed)
        if len(ids) - 1 >= k.PREFILL_MIN and k.prefill_supported():
            k.prefill(ids[:-1])
        else:
            for t in ids[:-1]:
                k.launch_step(t)           # no wait: only the last prompt step's token is needed
        return k.decode_step(ids[-1])

    def _finish(self, toks, prompt_tokens, t0, t1, out, show_speed) -> str:
        t2 = time.perf_counter()
        self.last_stats = {"prompt_tokens": prompt_tokens, "prefill_s": t1 - t0, "new_tokens": len(toks),
                           "decode_s": t2 - t1, "total_s": t2 - t0, "tokens": list(toks)}
        if show_speed:
            print("\n" + speed_line(prompt_tokens, t1 - t0, len(toks), t2 - t1, t2 - t0), file=out)
        return self.tokenizer.decode(toks, skip_special_tokens=True)

    # -- reference surface -----------------------------------------------------------------
    def generate(self, prompt: str, max_new_tokens: int = 100, show_speed: bool = True) -> str:
        """The reply text to ``prompt`` (a10_chat.py:325-407). At most ``max_new_tokens``
        tokens are generated, stopping after EOS. The prompt is truncated from the front
        when it does not fit (``fit_prompt``). Returns the generated tokens decoded
        without special tokens, and prints the speed line when ``show_speed``."""
        out = sys.stdout
        ids = self._prompt_ids(prompt, max_new_tokens, True, out)
        eos = self.tokenizer.eos_token_id
        k = self.model.decoder
        t0 = time.perf_counter()
        toks = [self._first_token(ids)]
        t1 = time.perf_counter()
        while toks[-1] != eos and len(toks) < max_new_tokens:
            n = min(GENERATE_CHUNK, max_new_tokens - len(toks))
            more = k.generate([toks[-1]], n)       # feeds the last token: its step's token and n - 1 more
            if eos is not None and eos in more:
                more = more[:more.index(eos) + 1]
            toks += more
        return self._finish(toks, len(ids), t0, t1, out, show_speed)

    def generate_stream(self, prompt: str, max_new_tokens: int = 500, show_speed: bool = True) -> str:
        """``generate`` with the reply printed as it is generated (a10_chat.py:409-510).
        Each step is its own launch. The next step is queued before the text of the
        last token is decoded and printed. Printing holds back an incomplete multi-byte
        character (the reference decodes and prints each token alone). Returns the same
        text as ``generate``."""
        out = sys.stdout
        ids = self._prompt_ids(prompt, max_new_tokens, False, out)
        eos = self.tokenizer.eos_token_id
        k = self.model.decoder
        shown = ""

        def show():
            nonlocal shown
            text = self.tokenizer.decode(toks, skip_special_tokens=True)
            if text.startswith(shown) and not text.endswith("\ufffd"):
                out.write(text[len(shown):])
                out.flush()
                shown = text

        t0 = time.perf_counter()
        toks = [self._first_token(ids)]
        t1 = time.perf_counter()
        while toks[-1] != eos and len(toks) < max_new_tokens:
            k.launch_step(toks[-1])
            show()
            toks.append(k.wait_token())
        show()
        return self._finish(toks, len(ids), t0, t1, out, show_speed)

    def chat(self, input_fn=input, max_new_tokens: int = 500) -> list:
        """The interactive loop (a10_chat.py:558-604). Each line read by ``input_fn`` is
        one user turn. ``quit`` / ``exit``, end of input or an interrupt end the loop;
        ``clear`` empties the history; an empty line is skipped. The reply is streamed,
        then printed cleaned (``clean_reply``) and kept in the history. Returns the
        conversation."""
        bar = "=" * 60
        print(f"\n{bar}\nQwen3 chat (MI355X decode kernel)\n{bar}\n"
              "Type 'quit' or 'exit' to end the conversation.\n"
              f"Type 'clear' to start a new conversation.\n{bar}\n")
        while True:
            try:
                line = input_fn("You: ").strip()
            except (KeyboardInterrupt, EOFError):
                print("\nGoodbye!")
                break
            if not line:
                continue
            if line.lower() in ("quit", "exit"):
                print("Goodbye!")
                break
            if line.lower() == "clear":
                self.conversation = []
                print("\n[Conversation cleared]\n")
                continue
            self.conversation.append({"role": "user", "content": line})
            print("Assistant: ", end="", flush=True)
            reply = clean_reply(self.generate_stream(chat_prompt(self.conversation, self.system), max_new_tokens))
            print(reply)
            self.conversation.append({"role": "assistant", "content": reply})
            print()
        return self.conversation


def main(argv=None) -> int:
    """Command line: chat with a local checkpoint directory (a10_chat.py:607-613)."""
    import argparse
    ap = argparse.ArgumentParser(description="Chat with a local Qwen3 checkpoint on the MI355X decode kernel")
    ap.add_argument("--model", required=True, help="checkpoint directory (safetensors, config.json, tokenizer)")
    ap.add_argument("--int8", action="store_true", help="per-row INT8 weights (default BF16, as the reference)")
    ap.add_argument("--max-seq-len", type=int, default=2048)
    ap.add_argument("--max-new-tokens", type=int, default=500)
    ap.add_argument("--temperature", type=float, default=0.0)
    ap.add_argument("--seed", type=int, default=0)
    args = ap.parse_args(argv)
    A10Chat(args.model, args.max_seq_len, int8=args.int8, temperature=args.temperature,
            seed=args.seed).chat(max_new_tokens=args.max_new_tokens)
    return 0
