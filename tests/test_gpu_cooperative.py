"""Cooperative launches of the persistent kernels (mq_decode_set_cooperative; run with -m gpu).

By default the decode, generation, batched and prefill kernels are launched plainly:
their workgroups wait on each other, so co-residency is checked with the occupancy
calculator but not guaranteed when other work holds compute units (the bounded waits
then end the step with MQ_ERR_TIMEOUT). With set_cooperative_launch(True) the runtime
starts them only when every workgroup can be resident. Gates: the same results as
plain launches on every kernel: the config-1 fixture's 32 tokens on the async-wave and
XCD-aware kernels and in one launch, a prefill's K/V rows, a batched step's tokens.
"""
from __future__ import annotations

import pytest
import torch

from .test_gpu_decode import _build, _greedy, _use_variant

pytestmark = pytest.mark.gpu


@pytest.fixture
def coop(mq):
    mq.set_cooperative_launch(True)
    try:
        yield
    finally:
        mq.set_cooperative_launch(False)


def test_cooperative_decode_reproduces_fixture(mq, dev, coop):
    dec, d, prompt, cfg, keep = _build(mq, dev, "qwen3_0.6b_int8")
    print("cooperative launches: async-wave kernel, per step and in one launch", flush=True)
    assert _greedy(dec, prompt, 32) == d["tokens"]
    dec.reset()
    assert dec.generate(prompt, 32, device_loop=True, batched_prefill=False) == d["tokens"]
    print("cooperative launches: XCD-aware kernel", flush=True)
    gen = _use_variant(mq, "xcd")
    next(gen)
    try:
        assert _greedy(dec, prompt, 32) == d["tokens"]
    finally:
        next(gen, None)
    del dec, keep
    torch.cuda.empty_cache()


def test_cooperative_prefill_and_batch_match_plain(mq, dev):
    cfg = mq.QWEN3_0_6B.with_(num_layers=2, vocab_size=4096)
    state, prompt = mq.random_init_state(cfg, seed=4, norm_jitter=0.1)
    S = 256
    cos, sin = mq.precompute_rope_freqs(cfg.head_dim, S, cfg.rope_theta, device=dev)
    packed = mq.pack_int8(mq.quantize_state(state, cfg, dev), cfg)
    dec = mq.A10Int8MegakernelDecoder(*packed[:6], cos, sin, cfg.num_layers, S)
    ids = torch.randint(0, cfg.vocab_size, (200,), generator=torch.Generator().manual_seed(9)).tolist()
    rows = []
    for on in (False, True):
        mq.set_cooperative_launch(on)
        try:
            dec.reset()
            dec.prefill(ids)
            torch.cuda.synchronize()
            rows.append((dec.k_cache[:, :, :200].cpu().clone(), dec.v_cache[:, :, :200].cpu().clone()))
        finally:
            mq.set_cooperative_launch(False)
    assert torch.equal(rows[0][0], rows[1][0]) and torch.equal(rows[0][1], rows[1][1])
    del dec
    # batched step (1.7B layer shape, 2 layers)
    bcfg = mq.QWEN3_1_7B.with_(num_layers=2, vocab_size=4096)
    bstate, _ = mq.random_init_state(bcfg, seed=5, norm_jitter=0.1)
    bpacked = mq.pack_int8(mq.quantize_state(bstate, bcfg, dev), bcfg)
    bcos, bsin = mq.precompute_rope_freqs(bcfg.head_dim, 32, bcfg.rope_theta, device=dev)
    prompts = torch.randint(0, bcfg.vocab_size, (4, 8), generator=torch.Generator().manual_seed(2)).tolist()
    toks = []
    for on in (False, True):
        mq.set_cooperative_launch(on)
        try:
            bdec = mq.A10Int8BatchDecoder(*bpacked, bcos, bsin, bcfg.num_layers, 32, 4)
            out = None
            for i in range(8):
                out = bdec.decode_step([p[i] for p in prompts])
            seq = [out]
            for _ in range(4):
                out = bdec.decode_step(out)
                seq.append(out)
            toks.append(seq)
            del bdec
        finally:
            mq.set_cooperative_launch(False)
    assert toks[0] == toks[1]
    torch.cuda.empty_cache()
