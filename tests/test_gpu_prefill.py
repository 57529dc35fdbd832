"""Prompt-batched prefill on the GPU (run with -m gpu).

The reference prefills a prompt with one decode step per token (a10_decode.py:367-368,
verify_correctness_a10.py:326-328). ``prefill`` / mq_int8_prefill writes the same K/V
cache rows with each layer's weights read once for all prompt positions. Gates:

* against the device's own per-token prefill (P decode steps) on the config-1 model
  (28 layers, INT8 Qwen3-0.6B shape) at P = 8, 64 and 512: every K and V row of every
  layer within one bf16 ulp, and at least 99.99 % of the values bit-identical (the two
  paths sum in different fp64 orders, which can move an fp32 rounding: about once in
  2^20 values);
* against the float64 oracle's per-token prefill on a 2-layer model (non-unit norm
  gains, 4096-word vocabulary) at P = 8, 64 and 512: the same bounds on the caches, and
  the first generated token (the decode step of the prompt's last token) equal to the
  oracle's argmax;
* the config-1 fixture's 32 greedy tokens through ``generate`` with the batched prefill,
  one launch and one launch per step;
* chunked prefills (a workspace smaller than the prompt) and a prefill after decode
  steps bit-identical to one chunk / to the per-token path's rows;
* a prompt of 1,500 positions (three chunks, attention past the decode kernel's
  64-position slots) against the per-token path;
* refusals before anything is launched (token range, positions past max_seq_len).
"""
from __future__ import annotations

import ctypes

import pytest
import torch

from oracle.ref_cpu import Dims, RefDecoder

from .test_gpu_decode import _fixture

pytestmark = pytest.mark.gpu


def _decoder(mq, dev, name, S):
    d = _fixture(name)
    cfg = mq.ModelConfig(**d["config"])
    state, prompt = mq.random_init_state(cfg, seed=d["seed"], norm_jitter=d["norm_jitter"])
    cos, sin = mq.precompute_rope_freqs(cfg.head_dim, S, cfg.rope_theta, device=dev)
    qstate = mq.quantize_state(state, cfg, dev)
    embed, layers, scales, lm_q, lm_s, fnorm = mq.pack_int8(qstate, cfg)
    dec = mq.A10Int8MegakernelDecoder(embed, layers, scales, lm_q, lm_s, fnorm, cos, sin, cfg.num_layers, S)
    keep = (embed, layers, scales, lm_q, lm_s, fnorm, cos, sin)
    return dec, d, prompt.tolist(), cfg, keep


def _tokens(n, vocab, seed):
    g = torch.Generator().manual_seed(seed)
    return torch.randint(0, vocab, (n,), generator=g).tolist()


def _rows(dec, n):
    torch.cuda.synchronize()
    return dec.k_cache[:, :, :n].cpu().clone(), dec.v_cache[:, :, :n].cpu().clone()


def _ordered(t):
    """bf16 values as integers ordered like the values (adjacent bf16 values differ by 1)."""
    u = t.contiguous().view(torch.int16).to(torch.int32) & 0xFFFF
    return torch.where(u < 0x8000, u, 0x8000 - u)


def _check_rows(got, want, what):
    """Every value within one bf16 ulp, at least 99.99 % bit-identical."""
    for g, w, kv in zip(got, want, "KV"):
        w = w.to(torch.bfloat16)
        d = (_ordered(g) - _ordered(w)).abs()
        same = float((d == 0).double().mean())
        assert int(d.max()) <= 1, f"{what} {kv}: a value differs by {int(d.max())} bf16 ulps"
        assert same >= 0.9999, f"{what} {kv}: only {same:.6f} of the values bit-identical"


def _per_token(dec, ids):
    dec.reset()
    tok = None
    for t in ids:
        tok = dec.decode_step(int(t))
    return tok


@pytest.fixture(scope="module")
def full(mq, dev):
    return _decoder(mq, dev, "qwen3_0.6b_int8", 1024)


@pytest.fixture(scope="module")
def small(mq, dev):
    return _decoder(mq, dev, "small_int8", 2048)


@pytest.mark.parametrize("P", [8, 64, 512])
def test_prefill_matches_per_token_steps(full, P):
    dec, d, prompt, cfg, _ = full
    ids = _tokens(P, cfg.vocab_size, 100 + P)
    print(f"config-1 model: prefill of {P} positions vs {P} decode steps", flush=True)
    _per_token(dec, ids)
    want = _rows(dec, P)
    dec.reset()
    dec.prefill(ids)
    assert dec.position() == P
    _check_rows(_rows(dec, P), want, f"P={P}")


@pytest.mark.parametrize("P", [8, 64, 512])
def test_prefill_matches_oracle(mq, small, P):
    dec, d, prompt, cfg, keep = small
    embed, layers, scales, lm_q, lm_s, fnorm, cos, sin = keep
    ids = _tokens(P, cfg.vocab_size, 7 + P)
    c = lambda t: t.cpu()
    ref = RefDecoder(Dims(vocab_size=cfg.vocab_size), c(embed), [c(t) for t in layers], [c(t) for t in scales],
                     c(fnorm), c(lm_q), c(lm_s), c(cos[:P + 1]), c(sin[:P + 1]), cfg.num_layers, P + 1)
    print(f"2-layer model: prefill of {P - 1} positions + one decode step vs the float64 oracle", flush=True)
    logits = None
    for t in ids:
        logits = ref.step_logits(int(t))
    want_tok = int(torch.argmax(logits))
    dec.reset()
    dec.prefill(ids[:-1])
    tok = dec.decode_step(int(ids[-1]))
    got = _rows(dec, P)
    _check_rows(got, (ref.k_cache[:, :, :P], ref.v_cache[:, :, :P]), f"P={P} vs oracle")
    top = torch.topk(logits.double(), 2).values
    assert tok == want_tok, f"first token {tok} != oracle {want_tok} (top-2 margin {float(top[0] - top[1]):.3g})"


@pytest.mark.parametrize("device_loop", [True, False])
def test_generate_with_batched_prefill_reproduces_fixture(full, device_loop):
    dec, d, prompt, cfg, _ = full
    print(f"config 1: generate with the batched prefill, device_loop={device_loop}", flush=True)
    dec.reset()
    dec.set_sampling(0.0)
    dec.PREFILL_MIN = 1                     # the 8-token prompt's first 7 through prefill()
    try:
        got = dec.generate(prompt, 32, device_loop=device_loop, batched_prefill=True)
    finally:
        del dec.PREFILL_MIN
    assert got == d["tokens"]
    assert dec.position() == len(prompt) + 31


def test_chunked_prefill_equals_one_chunk(small):
    dec, d, prompt, cfg, _ = small
    ids = _tokens(200, cfg.vocab_size, 3)
    print("2-layer model: 200 positions in one chunk and in chunks of 64", flush=True)
    dec.reset()
    dec.prefill(ids)
    one = _rows(dec, 200)
    old = dec.PREFILL_CHUNK
    try:
        dec.PREFILL_CHUNK = 64
        dec._pf_cap = 0                      # reallocate the workspace at the smaller chunk
        dec.reset()
        dec.prefill(ids)
        many = _rows(dec, 200)
    finally:
        dec.PREFILL_CHUNK = old
        dec._pf_cap = 0
    assert torch.equal(one[0], many[0]) and torch.equal(one[1], many[1])


def test_prefill_after_decode_steps(small):
    dec, d, prompt, cfg, _ = small
    ids = _tokens(45, cfg.vocab_size, 5)
    print("2-layer model: 5 decode steps, then a prefill of 40 positions, vs 45 decode steps", flush=True)
    _per_token(dec, ids)
    want = _rows(dec, 45)
    dec.reset()
    for t in ids[:5]:
        dec.decode_step(int(t))
    dec.prefill(ids[5:])
    assert dec.position() == 45
    _check_rows(_rows(dec, 45), want, "continued prefill")


def test_long_prompt_three_chunks(small):
    dec, d, prompt, cfg, _ = small
    P = 1500
    ids = _tokens(P, cfg.vocab_size, 11)
    print(f"2-layer model: prefill of {P} positions (chunks of 512) vs {P} decode steps", flush=True)
    _per_token(dec, ids)
    want = _rows(dec, P)
    dec.reset()
    dec.prefill(ids)
    _check_rows(_rows(dec, P), want, f"P={P}")


def test_prefill_refuses_before_launch(mq, small):
    dec, d, prompt, cfg, _ = small
    from megaqwen_a10_amd import _lib
    dec.reset()
    with pytest.raises(ValueError):
        dec.prefill([0, cfg.vocab_size])
    with pytest.raises(ValueError):
        dec.prefill([1] * (dec.max_seq_len + 1))
    assert dec.position() == 0
    lib = _lib.load()
    dec.prefill([1, 2])                                      # sets up the workspace
    torch.cuda.synchronize()
    before = _rows(dec, 4)
    bad = (ctypes.c_int * 2)(5, -1)
    a = dec._args
    a.position = 2
    st = lib.mq_int8_prefill(ctypes.byref(a), ctypes.cast(bad, ctypes.c_void_p), 2,
                             ctypes.c_void_p(dec._pf_ws.data_ptr()), dec._pf_ws.numel(),
                             ctypes.c_void_p(_lib.stream_handle()))
    assert st == _lib.MQ_ERR_INVALID_ARGUMENT and "tokens[1]" in _lib.last_error()
    a.position = dec.max_seq_len - 1
    ok = (ctypes.c_int * 2)(5, 6)
    st = lib.mq_int8_prefill(ctypes.byref(a), ctypes.cast(ok, ctypes.c_void_p), 2,
                             ctypes.c_void_p(dec._pf_ws.data_ptr()), dec._pf_ws.numel(),
                             ctypes.c_void_p(_lib.stream_handle()))
    assert st == _lib.MQ_ERR_INVALID_ARGUMENT
    st = lib.mq_int8_prefill(ctypes.byref(a), ctypes.cast(ok, ctypes.c_void_p), 2,
                             ctypes.c_void_p(dec._pf_ws.data_ptr()), 1000, ctypes.c_void_p(_lib.stream_handle()))
    assert st == _lib.MQ_ERR_INVALID_ARGUMENT
    after = _rows(dec, 4)
    assert torch.equal(before[0], after[0]) and torch.equal(before[1], after[1])
