"""One-launch generation on the XCD-aware kernel's multi-step form (run with -m gpu).

The async-wave kernel runs a whole generation in one launch for INT8 weights of the
Qwen3-0.6B shape up to 10240 positions; everything else (bf16 weights, the reference's own
A10Decoder.generate path, a10_decode.py:358-393; FP8 weights; the Qwen3-1.7B shape; longer
contexts) runs on the XCD-aware kernel, whose multi-step instantiation loops over the steps
inside one launch and hands each token to every workgroup through one tagged word. Gates:
the bf16 and FP8 32-token float64-oracle fixtures from one launch; the config-1 INT8
fixture from one launch on the XCD-aware kernel; one launch equal to one launch per step
(tokens and KV caches) on the 1.7B shape and at two temperatures; A10Decoder(int8=False)
running its generate in one launch; an expired in-kernel wait leaving the position where
the launch started.
"""
from __future__ import annotations

import pytest
import torch

from .test_gpu_decode import _build, _greedy, _use_variant

pytestmark = pytest.mark.gpu


def _caches(dec):
    torch.cuda.synchronize()
    return dec.k_cache.clone(), dec.v_cache.clone()


def _one_launch_vs_steps(dec, prompt, n, want=None):
    dec.reset()
    got = dec._generate_one_launch(prompt, n)
    assert got is not None, "a multi-step kernel covers this request"
    assert dec.position() == len(prompt) + n - 1
    k1, v1 = _caches(dec)
    per_step = _greedy(dec, prompt, n)
    k2, v2 = _caches(dec)
    assert got == per_step
    assert torch.equal(k1, k2) and torch.equal(v1, v2)
    if want is not None:
        assert got == want
    return got


@pytest.mark.parametrize("name", ["qwen3_0.6b_bf16", "qwen3_0.6b_fp8"])
def test_fixture_in_one_launch(mq, dev, name):
    dec, d, prompt, cfg, keep = _build(mq, dev, name)
    print(f"{name}: 8 prompt + 31 generated steps in one launch (XCD-aware kernel)", flush=True)
    dec.set_sampling(0.0)
    _one_launch_vs_steps(dec, prompt, 32, d["tokens"])
    del dec, keep
    torch.cuda.empty_cache()


@pytest.fixture
def xcd(mq, dev):
    yield from _use_variant(mq, "xcd")


def test_int8_fixture_in_one_launch_on_xcd_kernel(mq, dev, xcd):
    dec, d, prompt, cfg, keep = _build(mq, dev, "qwen3_0.6b_int8")
    print("config 1 on the XCD-aware kernel: one launch", flush=True)
    dec.set_sampling(0.0)
    _one_launch_vs_steps(dec, prompt, 32, d["tokens"])
    del dec, keep
    torch.cuda.empty_cache()


@pytest.mark.parametrize("temperature,seed", [(0.7, 3), (1.3, 2 ** 40 + 1)])
def test_sampled_one_launch_equals_per_step(mq, dev, xcd, temperature, seed):
    dec, d, prompt, cfg, keep = _build(mq, dev, "small_int8")
    print(f"2-layer model on the XCD-aware kernel, T={temperature}", flush=True)
    dec.set_sampling(temperature, seed)
    _one_launch_vs_steps(dec, prompt, 40)
    del dec, keep
    torch.cuda.empty_cache()


def test_1p7b_shape_one_launch(mq, dev):
    cfg = mq.QWEN3_1_7B.with_(name="1p7b-2l", num_layers=2, vocab_size=4096)
    state, prompt = mq.random_init_state(cfg, seed=5, norm_jitter=0.1)
    S = 96
    cos, sin = mq.precompute_rope_freqs(cfg.head_dim, S, cfg.rope_theta, device=dev)
    qstate = mq.quantize_state(state, cfg, dev)
    embed, layers, scales, lm_q, lm_s, fnorm = mq.pack_int8(qstate, cfg)
    dec = mq.A10Int8MegakernelDecoder(embed, layers, scales, lm_q, lm_s, fnorm, cos, sin, cfg.num_layers, S)
    print("1.7B shape, 2 layers: 8 + 79 steps in one launch (split attention past 48)", flush=True)
    _one_launch_vs_steps(dec, prompt.tolist(), S - len(prompt) + 1)
    del dec
    torch.cuda.empty_cache()


def test_a10decoder_bf16_generate_is_one_launch(mq, dev):
    """The reference's generate path (bf16 A10Decoder) runs in one launch and gives the bf16
    fixture; with device_loop=False it gives the same tokens one launch per step."""
    from .test_gpu_decode import _fixture
    d = _fixture("qwen3_0.6b_bf16")
    dec = mq.A10Decoder(seed=d["seed"], int8=False, max_seq_len=d["max_seq_len"], device=dev)
    calls = []
    orig = dec.decoder._generate_one_launch

    def spy(ids, n):
        out = orig(ids, n)
        calls.append(out is not None)
        return out

    dec.decoder._generate_one_launch = spy
    ids, tok_s, _ = dec.generate(d["prompt"], 32)
    assert calls == [True]
    assert ids[8:] == d["tokens"]
    ids2, _, _ = dec.generate(d["prompt"], 32, device_loop=False)
    assert ids2 == ids and calls == [True]
    del dec
    torch.cuda.empty_cache()


def test_expired_wait_in_multi_step_launch(mq, dev, xcd):
    dec, d, prompt, cfg, keep = _build(mq, dev, "small_int8")
    dec.set_sampling(0.0)
    dec.reset()
    dec.set_spin_limit(1)
    try:
        with pytest.raises(mq._lib.MQTimeoutError):
            dec.generate(prompt, 16)
    finally:
        dec.set_spin_limit(0)
    assert dec.position() == 0
    assert dec.generate(prompt, 16) == d["tokens"][:16]
    del dec, keep
    torch.cuda.empty_cache()
