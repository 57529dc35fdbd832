"""GPU parity of long-context decode and of the split attention
(run with -m gpu).

From ``attn_split_min`` positions on, the XCD-aware kernel gives each of the 32
workgroups sharing a KV head 1/32 of the cached positions and merges their
softmax partials (max, probability sum, weighted V) with a log-sum-exp rescale.
The checks: tokens identical to the committed fixture with the split forced at
every length (empty slices included), attention outputs of the split and the
unsplit paths within 1e-6 relative L2 of each other, and, after a seeded N(0,1) bf16 KV
pre-fill to depths past the unsplit limit of 1024, greedy tokens identical to
the float64 oracle started from the same cache. The async-wave kernel splits
the same way from 65 positions (slices of at most 64, held in its LDS slot) up to
2048: the same fixture, split-vs-unsplit and oracle checks run on it.
"""
from __future__ import annotations

import pytest
import torch

from oracle.ref_cpu import Dims, RefDecoder, top2_margin

from .test_gpu_decode import _build, _greedy

pytestmark = pytest.mark.gpu


@pytest.fixture
def xcd(mq):
    mq.set_decode_variant("xcd")
    yield
    mq.set_decode_variant("auto")


@pytest.fixture
def asyncv(mq):
    mq.set_decode_variant("async")
    yield
    mq.set_decode_variant("auto")


@pytest.fixture(scope="module")
def small(mq, dev):
    return _build(mq, dev, "small_int8")


@pytest.mark.parametrize("split_min", [1, 5, 17])
def test_split_tokens_match_fixture(xcd, small, split_min):
    """split_min 1: every step splits, so most of the 32 slices are empty early on;
    5 / 17: the switch happens inside the prompt / inside generation."""
    dec, d, prompt, cfg, _ = small
    dec.set_attn_split(split_min)
    try:
        print(f"small_int8 32 steps, split from {split_min}", flush=True)
        assert _greedy(dec, prompt, 32) == d["tokens"]
    finally:
        dec.set_attn_split(0)


def test_split_attention_matches_unsplit(xcd, small):
    """Same prompt with and without the split: same tokens, and the last layer's attention
    output agrees to far below fp32 accumulation error (both paths sum in fp64 and round
    once to fp32; earlier layers' outputs may differ in a last bit, which then moves
    later values by about 1e-7)."""
    dec, d, prompt, cfg, _ = small
    dec.enable_debug()
    outs = []
    try:
        for split_min in (-1, 1):
            dec.set_attn_split(split_min)
            toks = _greedy(dec, prompt, 20)
            outs.append((toks, dec.get_attn_out().clone(), dec.get_q().clone()))
    finally:
        dec.set_attn_split(0)
        dec.enable_debug(False)
    (ta, aa, qa), (tb, ab, qb) = outs
    assert ta == tb
    e = float(torch.linalg.norm((aa - ab).double()) / torch.linalg.norm(aa.double()))
    print(f"split vs unsplit attention: rel L2 {e:.2e}, identical {float((aa == ab).double().mean()):.3f}")
    assert e < 1e-6, e


def _long_case(mq, dev, depth, num_layers=2, seed=3, base=None):
    cfg = (base or mq.QWEN3_0_6B).with_(num_layers=num_layers, vocab_size=4096)
    state, prompt = mq.random_init_state(cfg, seed=seed, norm_jitter=0.1)
    qstate = mq.quantize_state(state, cfg, dev)
    embed, layers, scales, lm_q, lm_s, fnorm = mq.pack_int8(qstate, cfg)
    S = depth + 16
    cos, sin = mq.precompute_rope_freqs(cfg.head_dim, S, cfg.rope_theta, device=dev)
    dec = mq.A10Int8MegakernelDecoder(embed, layers, scales, lm_q, lm_s, fnorm, cos, sin, num_layers, S)
    c = lambda t: t.cpu()
    ref = RefDecoder(Dims(hidden_size=cfg.hidden_size, intermediate_size=cfg.intermediate_size,
                          vocab_size=cfg.vocab_size), c(embed), [c(t) for t in layers], [c(t) for t in scales],
                     c(fnorm), c(lm_q), c(lm_s), c(cos), c(sin), num_layers, S)
    return dec, ref, prompt.tolist()


# 1000 unsplit / split; 1500 and 4100: slices staged in LDS; 8192: the config-4 depth;
# 10300: slices of 322 positions, past the LDS staging capacity (320) -> read from HBM in the loop
@pytest.mark.parametrize("depth,split_min", [(1000, -1), (1000, 0), (1500, 0), (4100, 0), (8192, 0), (10300, 0)])
def test_long_context_matches_oracle(xcd, mq, dev, depth, split_min):
    """Config 4 semantics on a 2-layer model: seeded N(0,1) bf16 K/V rows at positions
    [0, depth), then 6 greedy steps; the oracle starts from the same cache."""
    print(f"long context depth {depth} split_min {split_min}", flush=True)
    _check_long(mq, dev, *_long_case(mq, dev, depth), depth, split_min)


@pytest.mark.parametrize("depth", [4100, 8192])
def test_long_context_1p7b_matches_oracle(xcd, mq, dev, depth):
    """The Qwen3-1.7B layer shapes (H = 2048, LDS staging capacity 256 positions): 4100
    stages its slices in LDS, 8192 (slices of 257) reads them in the loop."""
    print(f"1.7B long context depth {depth}", flush=True)
    _check_long(mq, dev, *_long_case(mq, dev, depth, base=mq.QWEN3_1_7B, seed=4), depth, 0)


def _check_long(mq, dev, dec, ref, prompt, depth, split_min):
    dec.set_attn_split(split_min)
    dec.prefill_random_kv(depth, seed=11)
    assert dec.position() == depth
    assert float(dec.k_cache[:, :, :depth].float().std()) == pytest.approx(1.0, rel=0.02)
    assert int(dec.k_cache[:, :, depth:].abs().sum()) == 0
    ref.load_kv(dec.k_cache, dec.v_cache, depth)
    tok_g = tok_r = int(prompt[0])
    got, want, margins = [], [], []
    for _ in range(6):
        tok_g = dec.decode_step(tok_g)
        logits = ref.step_logits(tok_r)
        tok_r = int(torch.argmax(logits))
        got.append(tok_g)
        want.append(tok_r)
        margins.append(top2_margin(logits))
    print(f"tokens {got} oracle {want} margins {[f'{m:.2e}' for m in margins]}", flush=True)
    assert got == want, (got, want, margins)
    # the rows this run wrote match the oracle's cache
    kc = dec.k_cache[:, :, depth:depth + 6].cpu().float()
    rk = ref.k_cache[:, :, depth:depth + 6].float()
    assert float((kc - rk).abs().max()) <= float(rk.abs().max()) * 2.0 ** -7
    del dec, ref
    torch.cuda.empty_cache()


def test_bf16_split_tokens_match_fixture(xcd, mq, dev):
    """bf16 weights with the split forced on every step (slices of at most two positions, taken
    from the rows prefetched a layer ahead): the 32 tokens of the bf16 fixture."""
    dec, d, prompt, cfg, keep = _build(mq, dev, "qwen3_0.6b_bf16")
    dec.set_attn_split(1)
    try:
        print("qwen3_0.6b_bf16 32 steps, split from 1", flush=True)
        assert _greedy(dec, prompt, 32) == d["tokens"]
    finally:
        dec.set_attn_split(0)
    del dec, keep
    torch.cuda.empty_cache()


def test_bf16_long_context_matches_oracle(xcd, mq, dev):
    """bf16 weights at depth 4100: split slices of 129 positions, more than the 64 rows prefetched a
    layer ahead, so the bf16 kernel reads them from the cache inside the loop (it has no register
    slice path); 6 greedy steps against the float64 oracle started from the same cache."""
    depth = 4100
    cfg = mq.QWEN3_0_6B.with_(num_layers=2, vocab_size=4096)
    state, prompt = mq.random_init_state(cfg, seed=3, norm_jitter=0.1)
    embed, layers, fnorm, lm = mq.pack_bf16(state, cfg, dev)
    S = depth + 16
    cos, sin = mq.precompute_rope_freqs(cfg.head_dim, S, cfg.rope_theta, device=dev)
    dec = mq.A10MegakernelDecoder(embed, layers, fnorm, lm, cos, sin, cfg.num_layers, S)
    c = lambda t: t.cpu()
    ref = RefDecoder(Dims(hidden_size=cfg.hidden_size, intermediate_size=cfg.intermediate_size,
                          vocab_size=cfg.vocab_size), c(embed), [c(t) for t in layers], None, c(fnorm), c(lm), None,
                     c(cos), c(sin), cfg.num_layers, S)
    print(f"bf16 long context depth {depth}", flush=True)
    _check_long(mq, dev, dec, ref, prompt.tolist(), depth, 0)


@pytest.fixture(params=["xcd", "async"])
def kernel_variant(request, mq):
    mq.set_decode_variant(request.param)
    yield request.param
    mq.set_decode_variant("auto")


def test_full_model_long_context_matches_oracle(kernel_variant, mq, dev):
    """Qwen3-0.6B shape (28 layers, full vocabulary) at depth 4096: 4 greedy steps
    against the live float64 oracle from the same pre-filled cache, on the XCD-aware kernel
    and on the async-wave kernel (slices of 129 positions in three chunks)."""
    depth = 4096
    cfg = mq.QWEN3_0_6B
    print(f"building qwen3_0.6b_int8 at depth 4096 ({kernel_variant})", flush=True)
    state, prompt = mq.random_init_state(cfg, seed=0)
    qstate = mq.quantize_state(state, cfg, dev)
    del state
    embed, layers, scales, lm_q, lm_s, fnorm = mq.pack_int8(qstate, cfg)
    S = depth + 8
    cos, sin = mq.precompute_rope_freqs(cfg.head_dim, S, cfg.rope_theta, device=dev)
    dec = mq.A10Int8MegakernelDecoder(embed, layers, scales, lm_q, lm_s, fnorm, cos, sin, cfg.num_layers, S)
    dec.prefill_random_kv(depth, seed=0)
    c = lambda t: t.cpu()
    ref = RefDecoder(Dims(), c(embed), [c(t) for t in layers], [c(t) for t in scales], c(fnorm), c(lm_q), c(lm_s),
                     c(cos), c(sin), cfg.num_layers, S)
    ref.load_kv(dec.k_cache, dec.v_cache, depth)
    tok_g = tok_r = int(prompt[-1])
    got, want, margins = [], [], []
    for _ in range(4):
        tok_g = dec.decode_step(tok_g)
        logits = ref.step_logits(tok_r)
        tok_r = int(torch.argmax(logits))
        got.append(tok_g)
        want.append(tok_r)
        margins.append(top2_margin(logits))
    print(f"tokens {got} oracle {want} margins {[f'{m:.2e}' for m in margins]}", flush=True)
    assert got == want, (got, want, margins)
    del dec, ref
    torch.cuda.empty_cache()


def test_length_limits(mq, dev):
    """Past 1024 positions only the split path can attend: the single-level kernel and the
    XCD-aware kernel with the split switched off refuse the step before launching."""
    dec, ref, prompt = _long_case(mq, dev, 1100, num_layers=1)
    dec.prefill_random_kv(1100, seed=1)
    try:
        mq.set_decode_variant("flat")
        with pytest.raises(mq._lib.MQError, match="attention limit"):
            dec.decode_step(int(prompt[0]))
        mq.set_decode_variant("xcd")
        dec.set_attn_split(-1)
        with pytest.raises(mq._lib.MQError, match="attention limit"):
            dec.decode_step(int(prompt[0]))
        dec.set_attn_split(0)
        assert dec.position() == 1100
        dec.decode_step(int(prompt[0]))
        assert dec.position() == 1101
    finally:
        mq.set_decode_variant("auto")
    with pytest.raises(ValueError):
        dec.prefill_random_kv(1116)


# ---- the async-wave kernel's split attention (32 slices of <= 64 positions) -------------------
@pytest.mark.parametrize("split_min", [1, 5, 17])
def test_async_split_tokens_match_fixture(asyncv, small, split_min):
    """The split forced from cache_len 1 / 5 / 17: the 32-token fixture (empty slices included)."""
    dec, d, prompt, cfg, _ = small
    dec.set_attn_split(split_min)
    try:
        print(f"async: small_int8 32 steps, split from {split_min}", flush=True)
        assert _greedy(dec, prompt, 32) == d["tokens"]
    finally:
        dec.set_attn_split(0)


def test_async_split_attention_matches_unsplit(asyncv, small):
    dec, d, prompt, cfg, _ = small
    dec.enable_debug()
    outs = []
    try:
        for split_min in (-1, 1):
            dec.set_attn_split(split_min)
            toks = _greedy(dec, prompt, 20)
            outs.append((toks, dec.get_attn_out().clone()))
    finally:
        dec.set_attn_split(0)
        dec.enable_debug(False)
    (ta, aa), (tb, ab) = outs
    assert ta == tb
    e = float(torch.linalg.norm((aa - ab).double()) / torch.linalg.norm(aa.double()))
    print(f"async split vs unsplit attention: rel L2 {e:.2e}, identical {float((aa == ab).double().mean()):.3f}")
    assert e < 1e-6, e


@pytest.mark.parametrize("depth", [100, 1000, 2040, 2100, 4100, 8180, 10200])
def test_async_long_context_matches_oracle(asyncv, mq, dev, depth):
    """Past the 64 positions of one workgroup's slot: 6 greedy steps after a seeded N(0,1) KV
    pre-fill, against the oracle started from the same cache. A rank's slice streams through its
    slot in chunks of 64: one chunk up to 2048 positions, two at 2100, three at 4100, four at
    8180, five at 10200 (the last step at cache_len 10206)."""
    print(f"async long context depth {depth}", flush=True)
    _check_long(mq, dev, *_long_case(mq, dev, depth), depth, 0)



def test_automatic_kernel_by_context_length(mq, dev):
    """The automatic choice takes the async-wave kernel up to 6144 cached positions (rank slices
    of up to three 64-position chunks) and the XCD-aware kernel past them (where it is faster);
    the async-wave kernel, when forced, covers 10240 and refuses longer ones."""
    mq.set_decode_variant("auto")
    v = lambda n: mq.decode_variant(1024, 3072, int8=True, cache_len=n)
    assert v(1) == v(2048) == v(2049) == v(6144) == "async"
    assert v(6145) == v(7168) == v(10240) == v(20000) == "xcd"
    mq.set_decode_variant("async")
    try:
        assert v(10240) == "async"
        with pytest.raises(mq._lib.MQError, match="async-wave"):
            v(10241)
    finally:
        mq.set_decode_variant("auto")
    assert mq.decode_variant(2048, 6144, int8=True, cache_len=100) == "xcd"
