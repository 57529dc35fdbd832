"""GPU tests of the device-side generation loop and of sampling (run with -m gpu).

mq_int8_decode_generate runs the prefill and every generated step in one launch
(the reference launches one step per token and reads each back,
bench_int8.py:218, a10_decode.py:358-393). Gates: the config-1 fixture's 32
greedy tokens from one launch; one launch and one launch per step agreeing
bitwise (tokens and KV caches), greedy and sampled; sampled tokens against the
float64 oracle's Gumbel-max choice wherever its top-2 margin exceeds fp32
logit error; a launch past one workgroup's 64-position slot (split attention);
one launch past the async-wave kernel's 10240 positions (the XCD-aware kernel's
multi-step form);
argument validation; a forced in-kernel wait expiry that leaves the decoder
where it started; a P-token prefill in one launch (P = 8 and 64) whose whole KV
cache and first generated token match the oracle's per-token prefill
(a10_decode.py:367-368).
"""
from __future__ import annotations

import pytest
import torch

from oracle.ref_cpu import sampled_choice

from .test_gpu_decode import _build, _greedy, _ref_for

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def small(mq, dev):
    return _build(mq, dev, "small_int8")


@pytest.fixture(scope="module")
def full(mq, dev):
    return _build(mq, dev, "qwen3_0.6b_int8")


def _caches(dec):
    torch.cuda.synchronize()
    return dec.k_cache.clone(), dec.v_cache.clone()


def test_one_launch_reproduces_fixture(full):
    dec, d, prompt, cfg, _ = full
    dec.set_sampling(0.0)
    dec.reset()
    print("config 1: 8 prompt + 31 generated steps in one launch", flush=True)
    got = dec._generate_one_launch(prompt, 32)
    assert got is not None, "the request is within the async-wave kernel's range"
    assert got == d["tokens"]
    assert dec.position() == len(prompt) + 31
    k1, v1 = _caches(dec)
    assert _greedy(dec, prompt, 32) == d["tokens"]             # one launch per step
    k2, v2 = _caches(dec)
    assert torch.equal(k1, k2) and torch.equal(v1, v2)


@pytest.mark.parametrize("temperature,seed", [(0.0, 0), (0.8, 1234), (1.5, 2 ** 63 + 5)])
def test_one_launch_equals_per_step(small, temperature, seed):
    dec, d, prompt, cfg, _ = small
    dec.set_sampling(temperature, seed)
    dec.reset()
    a = dec.generate(prompt, 24)
    ka, va = _caches(dec)
    dec.reset()
    b = dec.generate(prompt, 24, device_loop=False)
    kb, vb = _caches(dec)
    dec.set_sampling(0.0)
    print(f"T={temperature} seed={seed}: {a[:8]}", flush=True)
    assert a == b
    assert torch.equal(ka, kb) and torch.equal(va, vb)
    if temperature == 0.0:
        assert a == d["tokens"][:24]


def test_sampled_tokens_match_oracle(small):
    """Teacher-forced with the GPU's own tokens: at every step whose perturbed top-2 margin
    (float64 oracle) exceeds 1e-3 (fp32 logit error is ~1e-6 here), the sampled token must be
    the oracle's Gumbel-max choice."""
    dec, d, prompt, cfg, _ = small
    T, seed = 0.8, 99
    dec.set_sampling(T, seed)
    dec.reset()
    toks = dec.generate(prompt, 32)
    dec.set_sampling(0.0)
    ref = _ref_for(small)
    ref.reset()
    logits = None
    for t in prompt:
        logits = ref.step_logits(int(t))
    checked = 0
    for i, got in enumerate(toks):
        pos = len(prompt) - 1 + i
        want, margin = sampled_choice(logits.numpy(), T, seed, pos)
        if margin > 1e-3:
            assert got == want, (i, got, want, margin)
            checked += 1
        logits = ref.step_logits(int(got))
    print(f"sampled steps checked: {checked}/32", flush=True)
    assert checked >= 28
    assert len(set(toks)) > 1


def test_one_launch_past_one_slot(mq, dev, small):
    """Past the 64 positions of one workgroup's LDS slot the launch splits attention over the
    32 workgroups of an XCD: 8 prompt + 112 generated steps in one launch equal one launch
    per step, tokens and KV caches."""
    dec0, d, prompt, cfg, keep = small
    embed, layers, scales, lm_q, lm_s, fnorm, _, _ = keep
    S = 128
    cos, sin = mq.precompute_rope_freqs(cfg.head_dim, S, cfg.rope_theta, device=dev)
    dec = mq.A10Int8MegakernelDecoder(embed, layers, scales, lm_q, lm_s, fnorm, cos, sin, cfg.num_layers, S)
    n = S - len(prompt) + 1
    got = dec._generate_one_launch(prompt, n)
    assert got is not None
    k1, v1 = _caches(dec)
    want = _greedy(dec, prompt, n)
    k2, v2 = _caches(dec)
    assert got == want
    assert torch.equal(k1, k2) and torch.equal(v1, v2)
    del dec
    torch.cuda.empty_cache()


def test_one_launch_across_async_chunks(mq, dev, small):
    """On the async-wave kernel a rank's slice streams through its LDS slot in chunks of 64
    positions past 2048 cached positions: from a seeded cache of depth 2030, 150 steps in one
    launch (one chunk per rank, then two from cache_len 2049) equal one launch per step,
    tokens and KV caches."""
    dec0, d, prompt, cfg, keep = small
    embed, layers, scales, lm_q, lm_s, fnorm, _, _ = keep
    S, depth, n = 2200, 2030, 150
    cos, sin = mq.precompute_rope_freqs(cfg.head_dim, S, cfg.rope_theta, device=dev)
    dec = mq.A10Int8MegakernelDecoder(embed, layers, scales, lm_q, lm_s, fnorm, cos, sin, cfg.num_layers, S)
    mq.set_decode_variant("async")
    try:
        print(f"2-layer model: depth {depth}, {n} steps in one launch", flush=True)
        dec.prefill_random_kv(depth, seed=5)
        got = dec._generate_one_launch([int(prompt[0])], n)
        assert got is not None
        assert dec.position() == depth + n
        k1, v1 = _caches(dec)
        dec.prefill_random_kv(depth, seed=5)
        tok, want = int(prompt[0]), []
        for _ in range(n):
            tok = dec.decode_step(tok)
            want.append(tok)
        k2, v2 = _caches(dec)
    finally:
        mq.set_decode_variant("auto")
    assert got == want
    assert torch.equal(k1, k2) and torch.equal(v1, v2)
    del dec
    torch.cuda.empty_cache()


def test_one_launch_beyond_async_range(mq, dev, small):
    """Past the async-wave kernel's 10240 positions the launch runs on the XCD-aware kernel's
    multi-step form (split attention): one launch gives the tokens of one launch per step on
    that kernel, and the same KV cache rows wherever both take the same arithmetic path:
    positions below 2048, where each workgroup's slice holds at most 64 positions. (Past that,
    the one-step kernel takes a slice's scores on the bf16 matrix cores with fp32 sums and the
    multi-step form, which has no registers for those slices, in fp64, so later rows can round
    differently in their last bits.)"""
    dec0, d, prompt, cfg, keep = small
    embed, layers, scales, lm_q, lm_s, fnorm, _, _ = keep
    S = 10240 + 16
    cos, sin = mq.precompute_rope_freqs(cfg.head_dim, S, cfg.rope_theta, device=dev)
    dec = mq.A10Int8MegakernelDecoder(embed, layers, scales, lm_q, lm_s, fnorm, cos, sin, cfg.num_layers, S)
    n = S - len(prompt) + 1
    print(f"2-layer model: {len(prompt)} + {n - 1} steps in one launch past 10240 positions", flush=True)
    got = dec._generate_one_launch(prompt, n)
    assert got is not None
    assert dec.position() == S
    k1, v1 = _caches(dec)
    mq.set_decode_variant("xcd")
    try:
        assert got == _greedy(dec, prompt, n)
    finally:
        mq.set_decode_variant("auto")
    k2, v2 = _caches(dec)
    assert torch.equal(k1[:, :, :2048], k2[:, :, :2048]) and torch.equal(v1[:, :, :2048], v2[:, :, :2048])
    del dec
    torch.cuda.empty_cache()


def test_generate_validation(small):
    dec, d, prompt, cfg, _ = small
    dec.reset()
    with pytest.raises(ValueError):
        dec.generate([cfg.vocab_size], 4)
    with pytest.raises(ValueError):
        dec.generate([], 4)
    with pytest.raises(ValueError):
        dec.generate(prompt, 0)
    with pytest.raises(ValueError):
        dec.generate(prompt, d["max_seq_len"])               # runs past the KV cache
    with pytest.raises(ValueError):
        dec.set_sampling(-1.0)
    with pytest.raises(ValueError):
        dec.set_sampling(float("nan"))
    assert dec.position() == 0


def test_expired_wait_leaves_position(mq, small):
    dec, d, prompt, cfg, _ = small
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


@pytest.mark.parametrize("P", [8, 64])
def test_prefill_one_launch_matches_oracle(small, P):
    """P prompt tokens and the first generated token from one launch: every cached K and V
    row of every layer within one bf16 ulp of the float64 oracle's per-token prefill, most
    of them bit-identical, and the generated token the oracle's argmax (its top-2 margin
    checked to exceed fp32 logit error)."""
    dec, d, prompt, cfg, _ = small
    g = torch.Generator().manual_seed(4242 + P)
    ids = torch.randint(0, cfg.vocab_size, (P,), generator=g).tolist()
    dec.set_sampling(0.0)
    dec.reset()
    print(f"prefill P={P} in one launch", flush=True)
    got = dec._generate_one_launch(ids, 1)
    assert got is not None, "P <= 64 positions is within the async-wave kernel's range"
    assert dec.position() == P
    kc, vc = _caches(dec)
    ref = _ref_for(small)
    ref.reset()
    logits = None
    for t in ids:
        logits = ref.step_logits(int(t))
    top2 = torch.topk(logits.double(), 2).values
    assert float(top2[0] - top2[1]) > 1e-4
    assert got == [int(torch.argmax(logits))]
    for name, gpu, want in (("K", kc, ref.k_cache), ("V", vc, ref.v_cache)):
        a = gpu[:, :, :P].cpu().float()
        b = want[:, :, :P].float()
        err = (a - b).abs()
        ulp = b.abs().clamp_min(2.0 ** -126) * 2.0 ** -7
        print(f"{name}: max |err|/ulp {float((err / ulp).max()):.3f}, "
              f"bit-identical {float((err == 0).double().mean()):.4f}", flush=True)
        assert bool((err <= ulp).all()), name
        assert float((err == 0).double().mean()) > 0.95, name
        assert int(gpu[:, :, P:].abs().sum()) == 0            # nothing written past the prompt
