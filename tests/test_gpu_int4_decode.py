"""GPU tests of the INT4-g128 decode step (A10Int4MegakernelDecoder, mq_int4_decode_step; run with -m gpu).

The reference has INT8 and BF16 weights only. Here the seven layer projections are
INT4 per group of 128 inputs (quantize_int4: s = bf16(amax / 7), q = clamp(rint(w / s),
-8, 7)) and the LM head stays INT8 per row. The async-wave kernel expands the nibbles
to int8 matrix-core operands and scales each group's exact digit-plane sum by its
group scale in fp64. Its oracle is oracle.ref_cpu.RefDecoder fed the dequantized
weights (q x s, exact in fp64; oracle/formats.py) with row scales of 1, so the bar is
the INT8 one: the config-1 model's 32 greedy tokens identical to the float64 oracle's
fixture, per-stage values of a 1- and 2-layer model within 1e-5 / 1e-3 of the live
oracle, one launch for a generation equal to per-step launches.
"""
from __future__ import annotations

import pytest
import torch

from oracle import formats as of
from oracle.ref_cpu import Dims, RefDecoder

from .test_gpu_decode import _build, _greedy

pytestmark = pytest.mark.gpu


def test_full_int4_32_tokens(mq, dev):
    """Config-1 model with INT4-g128 weights: 32 greedy tokens identical to the float64 oracle's."""
    print("building qwen3_0.6b_int4", flush=True)
    dec, d, prompt, cfg, keep = _build(mq, dev, "qwen3_0.6b_int4")
    assert isinstance(dec, mq.A10Int4MegakernelDecoder)
    toks = _greedy(dec, prompt, 32)
    assert toks == d["tokens"], (toks, d["tokens"])
    # one launch for the prompt and 25 generated tokens: the same tokens
    dec.reset()
    assert dec.generate(prompt, 25, device_loop=True) == d["tokens"][:25]
    del dec, keep
    torch.cuda.empty_cache()


def _small_int4(mq, dev, num_layers, S=64):
    cfg = mq.QWEN3_0_6B.with_(num_layers=num_layers, vocab_size=4096)
    state, prompt = mq.random_init_state(cfg, seed=3, norm_jitter=0.1)
    cos, sin = mq.precompute_rope_freqs(cfg.head_dim, S, cfg.rope_theta, device=dev)
    qstate = mq.quantize_state(state, cfg, dev, weight_format="int4")
    embed, layers, scales, lm_q, lm_s, fnorm = mq.pack_int8(qstate, cfg)
    dec = mq.A10Int4MegakernelDecoder(embed, layers, scales, lm_q, lm_s, fnorm, cos, sin, cfg.num_layers, S)
    # the oracle: dequantized projections (row scales of 1), the INT8 LM head as it is
    proj = {1, 2, 3, 6, 8, 9, 10}
    ref_layers, ref_scales = [], []
    for i, t in enumerate(layers):
        if i % 11 in proj:
            s = scales[len(ref_scales)]
            ref_layers.append(torch.from_numpy(of.dequant_int4(t.cpu(), s.cpu())))
            ref_scales.append(torch.ones(t.shape[0], dtype=torch.float32))
        else:
            ref_layers.append(t.cpu())
    ref = RefDecoder(Dims(vocab_size=cfg.vocab_size), embed.cpu(), ref_layers, ref_scales, fnorm.cpu(),
                     lm_q.cpu(), lm_s.cpu(), cos.cpu(), sin.cpu(), cfg.num_layers, S)
    return dec, ref, prompt.tolist(), (embed, layers, scales, lm_q, lm_s, fnorm, cos, sin)


def test_int4_quantized_state_is_the_oracles(mq, dev):
    """quantize_state(weight_format="int4"): the GPU quantizer's nibbles and group scales equal
    the oracle's for every projection; the LM head is INT8 per row."""
    cfg = mq.QWEN3_0_6B.with_(num_layers=1, vocab_size=4096)
    state, _ = mq.random_init_state(cfg, seed=3, norm_jitter=0.1)
    qstate = mq.quantize_state(state, cfg, dev, weight_format="int4")
    for k, v in qstate.items():
        if not isinstance(v, tuple):
            continue
        q, s = v
        if k == "lm_head.weight":
            assert q.dtype == torch.int8 and s.shape == (cfg.vocab_size,)
            continue
        qr, sr = of.quantize_int4_groups(state[k])
        assert torch.equal(q.cpu(), qr) and torch.equal(s.cpu(), sr), k


@pytest.mark.parametrize("num_layers,steps,bound", [(1, 1, 1e-5), (2, 5, 1e-3)])
def test_int4_stages_match_oracle(mq, dev, num_layers, steps, bound):
    """Last layer's stored values (the reference's debug getters) against the live oracle."""
    dec, ref, prompt, keep = _small_int4(mq, dev, num_layers)
    print(f"int4 stages, {num_layers} layer(s), {steps} step(s)", flush=True)
    dec.enable_debug()
    dec.reset()
    ref.reset()
    for t in prompt[:steps]:
        got = dec.decode_step(int(t))
        logits = ref.step_logits(int(t))
        assert got == int(torch.argmax(logits))
    last = ref.last
    checks = {"q": dec.get_q(), "k": dec.get_k(), "v": dec.get_v(), "attn_out": dec.get_attn_out(),
              "residual": dec.get_residual(), "activations": dec.get_activations(),
              "mlp_intermediate": dec.get_mlp_int(), "normalized": dec.get_normalized()}
    for name, t in checks.items():
        a, b = t.detach().cpu().double(), last[name].double()
        e = float(torch.linalg.norm(a - b) / torch.linalg.norm(b))
        print(f"int4 stage {name}: rel L2 {e:.2e}", flush=True)
        assert e < bound, (name, e)
    p = dec.position() - 1
    kc = dec.k_cache[:, :, p].cpu().float()
    rk = ref.k_cache[:, :, p].float()
    assert float((kc - rk).abs().max()) <= float(rk.abs().max()) * 2.0 ** -7
    del dec, keep
    torch.cuda.empty_cache()


def test_int4_runs_on_the_async_kernel_only(mq, dev):
    """Forcing the single-level or XCD-aware kernel is refused before anything runs; the
    automatic choice runs, and one launch equals per-step launches."""
    dec, ref, prompt, keep = _small_int4(mq, dev, 2)
    for v in ("flat", "xcd"):
        mq.set_decode_variant(v)
        try:
            with pytest.raises(mq._lib.MQError):
                dec.decode_step(int(prompt[0]))
        finally:
            mq.set_decode_variant("auto")
        assert dec.position() == 0
    assert dec.decode_step(int(prompt[0])) == int(torch.argmax(ref.step_logits(int(prompt[0]))))
    dec.reset()
    assert dec.generate(prompt, 12, device_loop=True) == _greedy(dec, prompt, 12)
    assert not dec.prefill_supported()
    del dec, keep
    torch.cuda.empty_cache()


def test_int4_long_context_matches_oracle(mq, dev):
    """INT4 weights past 2048 cached positions, where a rank's slice streams through its LDS slot
    in two 64-position chunks: 6 greedy steps after a seeded N(0,1) KV pre-fill of depth 2100,
    tokens equal to the live oracle's from the same cache."""
    from .test_gpu_longctx import _check_long
    depth = 2100
    print(f"INT4 2-layer model at depth {depth}", flush=True)
    dec, ref, prompt, keep = _small_int4(mq, dev, 2, S=depth + 16)
    _check_long(mq, dev, dec, ref, prompt, depth, 0)
    del dec, ref, keep
    torch.cuda.empty_cache()
