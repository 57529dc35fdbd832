"""GPU tests of the FP8 E4M3 decode step (A10Fp8MegakernelDecoder, mq_fp8_decode_step; run with -m gpu).

The reference has INT8 and BF16 weights only; the FP8 path is the INT8 one with
every linear and the LM head as E4M3 codes and per-row scales, on the
XCD-aware kernel. Its oracle is oracle.ref_cpu.RefDecoder fed the codes'
exact values (oracle/formats.py): the products are exact in fp64 as for INT8,
so the bar is the INT8 one: the config-1 model's 32 greedy tokens identical to
the float64 oracle's fixture, and per-stage values of a 2-layer model within
1e-3 (1e-5 after one layer) of the live oracle.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import formats as of
from oracle.ref_cpu import Dims, RefDecoder

from .test_gpu_decode import _build, _greedy, _use_variant

pytestmark = pytest.mark.gpu


@pytest.fixture
def xcd(mq, dev):
    yield from _use_variant(mq, "xcd")


def test_full_fp8_32_tokens(mq, dev):
    """Config-1 model with FP8 weights: 32 greedy tokens identical to the float64 oracle's."""
    print("building qwen3_0.6b_fp8", flush=True)
    dec, d, prompt, cfg, keep = _build(mq, dev, "qwen3_0.6b_fp8")
    toks = _greedy(dec, prompt, 32)
    assert toks == d["tokens"], (toks, d["tokens"])
    # the GPU quantizer's codes are the oracle's (the fixture was made from the oracle's)
    embed, layers, scales, lm_q, lm_s, fnorm, cos, sin = keep
    assert lm_q.dtype == torch.uint8 and int(lm_q.max()) <= 0xFE
    del dec, keep
    torch.cuda.empty_cache()


def _small_fp8(mq, dev, num_layers):
    cfg = mq.QWEN3_0_6B.with_(num_layers=num_layers, vocab_size=4096)
    state, prompt = mq.random_init_state(cfg, seed=3, norm_jitter=0.1)
    S = 64
    cos, sin = mq.precompute_rope_freqs(cfg.head_dim, S, cfg.rope_theta, device=dev)
    qstate = mq.quantize_state(state, cfg, dev, weight_format="fp8")
    embed, layers, scales, lm_q, lm_s, fnorm = mq.pack_int8(qstate, cfg)
    dec = mq.A10Fp8MegakernelDecoder(embed, layers, scales, lm_q, lm_s, fnorm, cos, sin, cfg.num_layers, S)
    table = torch.from_numpy(of.fp8_decode_table())
    val = lambda t: table[t.cpu().long()] if t.dtype == torch.uint8 else t.cpu()
    ref = RefDecoder(Dims(vocab_size=cfg.vocab_size), embed.cpu(), [val(t) for t in layers],
                     [t.cpu() for t in scales], fnorm.cpu(), val(lm_q), lm_s.cpu(), cos.cpu(), sin.cpu(),
                     cfg.num_layers, S)
    return dec, ref, prompt.tolist(), (embed, layers, scales, lm_q, lm_s, fnorm, cos, sin)


@pytest.mark.parametrize("num_layers,steps,bound", [(1, 1, 1e-5), (2, 5, 1e-3)])
def test_fp8_stages_match_oracle(mq, dev, xcd, num_layers, steps, bound):
    """Last layer's stored values (the reference's debug getters) against the live oracle."""
    dec, ref, prompt, keep = _small_fp8(mq, dev, num_layers)
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
        print(f"fp8 stage {name}: rel L2 {e:.2e}", flush=True)
        assert e < bound, (name, e)
    p = dec.position() - 1
    kc = dec.k_cache[:, :, p].cpu().float()
    rk = ref.k_cache[:, :, p].float()
    assert float((kc - rk).abs().max()) <= float(rk.abs().max()) * 2.0 ** -7
    del dec, keep
    torch.cuda.empty_cache()


def test_fp8_needs_the_xcd_kernel(mq, dev):
    """FP8 runs on the XCD-aware kernel only: forcing the single-level or async kernel is refused."""
    dec, ref, prompt, keep = _small_fp8(mq, dev, 1)
    for v in ("flat", "async"):
        mq.set_decode_variant(v)
        try:
            with pytest.raises(mq._lib.MQError):
                dec.decode_step(int(prompt[0]))
        finally:
            mq.set_decode_variant("auto")
        assert dec.position() == 0
    assert dec.decode_step(int(prompt[0])) == int(torch.argmax(ref.step_logits(int(prompt[0]))))
    dec.reset()
    assert dec.generate(prompt, 3, device_loop=True) == _greedy(dec, prompt, 3)     # per-step launches
    del dec, keep
    torch.cuda.empty_cache()
