"""GPU check of the allocation-free decode step (mq_int8_decode_step_noalloc).

It must give the same results as mq_int8_decode_step, which runs the same kernels
on a caller-provided workspace: identical greedy tokens and bit-identical KV caches
over a prefill and greedy steps of one model, then the same for a smaller model
(fewer layers, smaller vocabulary, shorter cache) right after it, on the same
static scratch array (which every call clears before use).
"""
from __future__ import annotations

import ctypes
import json

import pytest
import torch

from .conftest import GOLDEN

pytestmark = pytest.mark.gpu


def _model(mq, dev, cfg, seed, S):
    state, prompt = mq.random_init_state(cfg, seed=seed, norm_jitter=0.1)
    qstate = mq.quantize_state(state, cfg, dev)
    packed = mq.pack_int8(qstate, cfg)
    cos, sin = mq.precompute_rope_freqs(cfg.head_dim, S, cfg.rope_theta, device=dev)
    dec = mq.A10Int8MegakernelDecoder(*packed, cos, sin, cfg.num_layers, S)
    return dec, prompt.tolist(), (packed, cos, sin)


def _noalloc_run(mq, dec, prompt, n):
    """Prefill + n greedy steps through mq_int8_decode_step_noalloc on fresh KV caches, with
    the decoder's own (weights, tables) arguments and no workspace."""
    lib = mq._lib.load()
    dev = dec.device
    a = type(dec._args).from_buffer_copy(dec._args)
    kc, vc = torch.zeros_like(dec.k_cache), torch.zeros_like(dec.v_cache)
    out = torch.full((1,), -2, dtype=torch.int32, device=dev)
    a.k_cache, a.v_cache, a.output_token_id = kc.data_ptr(), vc.data_ptr(), out.data_ptr()
    a.workspace, a.workspace_bytes = None, 0
    stream = ctypes.c_void_p(mq._lib.stream_handle(dev))
    seq, toks, pos = list(prompt), [], 0
    while len(toks) < n:
        a.input_token_id, a.position, a.cache_len = int(seq[pos]), pos, pos + 1
        st = lib.mq_int8_decode_step_noalloc(ctypes.byref(a), stream)
        assert st == 0, mq._lib.last_error()
        tok = int(out.item())
        pos += 1
        if pos >= len(prompt):
            toks.append(tok)
            seq.append(tok)
    return toks, kc, vc


def _class_run(dec, prompt, n):
    dec.reset()
    tok = None
    for t in prompt:
        tok = dec.decode_step(int(t))
    toks = [tok]
    while len(toks) < n:
        tok = dec.decode_step(tok)
        toks.append(tok)
    return toks


def test_noalloc_matches_workspace_entry_point(mq, dev):
    fixture = json.loads((GOLDEN / "tokens_small_int8.json").read_text())
    big_cfg = mq.ModelConfig(**fixture["config"])
    small_cfg = mq.QWEN3_0_6B.with_(name="noalloc_b", num_layers=1, vocab_size=1024)
    for cfg, seed, S, n in ((big_cfg, fixture["seed"], 64, 16), (small_cfg, 3, 24, 8)):
        print(f"{cfg.name}: {cfg.num_layers} layers, vocab {cfg.vocab_size}, cache {S}", flush=True)
        dec, prompt, keep = _model(mq, dev, cfg, seed, S)
        got, kc, vc = _noalloc_run(mq, dec, prompt, n)
        want = _class_run(dec, prompt, n)
        assert got == want, (cfg.name, got, want)
        assert torch.equal(kc, dec.k_cache) and torch.equal(vc, dec.v_cache), cfg.name
        if cfg is big_cfg:
            assert got == fixture["tokens"][:n]
        del dec, keep, kc, vc
        torch.cuda.empty_cache()
