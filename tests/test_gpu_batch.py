"""GPU parity of the batched INT8 decode (run with -m gpu).

The reference has no batched path; its semantics are B independent copies of
the single-sequence step sharing the weights. Each sequence of a batch must
therefore produce the float64 oracle's greedy tokens for its own prompt, and a
sequence's tokens must not depend on which slot or batch size it runs in.
The batched kernel computes products on the int8 matrix cores with 28-bit
(four-digit) activations and applies the RMSNorm scale after the product, so
its intermediate values carry bf16-level differences from the oracle's (a
flipped bf16 rounding is 2^-8 relative), and those accumulate in the KV cache
over a long run. Parity is therefore checked teacher-forced: the oracle is fed
each sequence's own GPU tokens, and at every step the GPU's token must be the
oracle's argmax up to the bf16-activation tolerance carried to the logits
(its logit at most 2^-7 of the logits' standard deviation below the maximum,
twice the 2^-8 relative error of one bf16 rounding). After the last step the
hidden state must be within 2^-8 relative L2 of the oracle's. A wrong token
from a real fault falls short of the maximum by about 3 logit standard
deviations.
"""
from __future__ import annotations

import pytest
import torch

from oracle.ref_cpu import Dims, RefDecoder

pytestmark = pytest.mark.gpu

STEPS = 12
LOGIT_TOL = 2.0 ** -7  # x the logits' standard deviation at that step


def _model(mq, dev, S, seed=5):
    cfg = mq.QWEN3_1_7B.with_(num_layers=2, vocab_size=4096)
    state, _ = mq.random_init_state(cfg, seed=seed, norm_jitter=0.1)
    qstate = mq.quantize_state(state, cfg, dev)
    packed = mq.pack_int8(qstate, cfg)
    cos, sin = mq.precompute_rope_freqs(cfg.head_dim, S, cfg.rope_theta, device=dev)
    return cfg, packed, cos, sin, S


@pytest.fixture(scope="module")
def model(mq, dev):
    return _model(mq, dev, 64)


def _prompts(n, vocab, seed=21):
    g = torch.Generator().manual_seed(seed)
    return torch.randint(0, vocab, (n, 8), generator=g).tolist()


def _run_batch(mq, model, prompts, steps=STEPS, debug=False):
    cfg, (embed, layers, scales, lm_q, lm_s, fnorm), cos, sin, S = model
    dec = mq.A10Int8BatchDecoder(embed, layers, scales, lm_q, lm_s, fnorm, cos, sin, cfg.num_layers, S, len(prompts))
    if debug:
        dec.enable_debug()
    out = None
    for i in range(len(prompts[0])):
        out = dec.decode_step([p[i] for p in prompts])
    toks = [[t] for t in out]
    for _ in range(steps - 1):
        out = dec.decode_step(out)
        for b, t in enumerate(out):
            toks[b].append(t)
    return dec, toks


def _ref(model):
    cfg, (embed, layers, scales, lm_q, lm_s, fnorm), cos, sin, S = model
    c = lambda t: t.cpu()
    return RefDecoder(Dims(hidden_size=2048, intermediate_size=6144, vocab_size=cfg.vocab_size), c(embed),
                      [c(t) for t in layers], [c(t) for t in scales], c(fnorm), c(lm_q), c(lm_s), c(cos), c(sin),
                      cfg.num_layers, S)


@pytest.mark.parametrize("batch", [1, 3, 4, 8, 16])
def test_batch_matches_oracle_per_sequence(mq, dev, model, batch):
    prompts = _prompts(batch, model[0].vocab_size)
    print(f"batch {batch}", flush=True)
    _check_against_oracle(mq, model, prompts, STEPS)


def test_batch_long_positions_match_oracle(mq, dev):
    """Past the positions the config-5 benchmark reaches (8 prompt tokens + 128 steps) and past the
    192 positions whose K/V rows the attention rank loads straight into LDS (longer sequences take
    the path that reads the rows beyond the first 64 inside the attention loops): three sequences,
    8 prompt tokens and 200 greedy steps, up to position 207."""
    long_model = _model(mq, dev, 216, seed=6)
    prompts = _prompts(3, long_model[0].vocab_size, seed=29)
    print("batch 3, 200 steps", flush=True)
    _check_against_oracle(mq, long_model, prompts, 200)


def _check_against_oracle(mq, model, prompts, steps, shared_ref=None, check=None, hidden_tol=2.0 ** -8):
    """Teacher-forced parity of every sequence (module docstring), or of the sequences in
    `check`. With `shared_ref` one oracle instance is reset per sequence instead of built per
    sequence."""
    dec, toks = _run_batch(mq, model, prompts, steps, debug=True)
    assert dec.positions() == [8 + steps - 1] * len(prompts)
    hidden = dec.get_hidden().float().cpu().double()
    bad, worst, differ = [], 0.0, 0
    for b, p in enumerate(prompts):
        if check is not None and b not in check:
            continue
        ref = shared_ref if shared_ref is not None else _ref(model)
        ref.reset()
        for i, t in enumerate(list(p) + toks[b][:-1]):
            logits = ref.step_logits(int(t))
            j = i - (len(p) - 1)
            if j < 0:
                continue
            got = toks[b][j]
            deficit = float(logits.max() - logits[got]) / float(logits.std())
            worst = max(worst, deficit)
            differ += int(got != int(logits.argmax()))
            if deficit > LOGIT_TOL:
                bad.append((b, j, got, int(logits.argmax()), f"{deficit:.2e}"))
        want = ref.last["hidden"].double()
        e = float(torch.linalg.norm(hidden[b] - want) / torch.linalg.norm(want))
        if e >= hidden_tol:
            bad.append((b, "hidden rel L2", f"{e:.2e}"))
    print(f"{len(prompts) if check is None else len(check)} sequences x {steps} steps: {differ} tokens differ from the oracle's argmax, "
          f"largest logit deficit {worst:.2e} std", flush=True)
    assert not bad, bad


@pytest.fixture(scope="module")
def full_vocab(mq, dev):
    """One Qwen3-1.7B-shape layer with the real 151,936-row vocabulary, and one oracle for it."""
    cfg = mq.QWEN3_1_7B.with_(num_layers=1)
    state, _ = mq.random_init_state(cfg, seed=8, norm_jitter=0.1)
    qstate = mq.quantize_state(state, cfg, dev)
    del state
    packed = mq.pack_int8(qstate, cfg)
    S = 32
    cos, sin = mq.precompute_rope_freqs(cfg.head_dim, S, cfg.rope_theta, device=dev)
    model = (cfg, packed, cos, sin, S)
    return model, _ref(model)


@pytest.mark.parametrize("batch", [1, 16])
def test_batch_full_vocabulary_matches_oracle(mq, dev, full_vocab, batch):
    """At the real vocabulary each workgroup owns 593-594 LM-head rows: 38 tiles of 16 rows over
    the 8 waves (5 per wave), a ragged last tile, the two-deep weight ring and the argmax merged
    across waves and workgroups all run, which the 4,096-row models above never reach. Every
    sequence is checked teacher-forced against the oracle as in the other batched tests."""
    model, ref = full_vocab
    prompts = _prompts(batch, model[0].vocab_size, seed=51)
    print(f"full vocabulary, batch {batch}", flush=True)
    _check_against_oracle(mq, model, prompts, STEPS, shared_ref=ref)


def test_full_model_batch_16_matches_oracle(mq, dev):
    """The BASELINE config-5 model itself: Qwen3-1.7B shape with all 28 layers and the
    151,936-row vocabulary, 16 sequences for 8 prompt tokens and 4 greedy steps (the bench's
    batch), four of them (slots 0, 5, 10, 15) checked teacher-forced against the float64
    oracle as in the other batched tests. The hidden state's bound is 2^-5 relative L2, not
    the 2-layer models' 2^-8: the occasional flipped bf16 rounding (module docstring) compounds
    over 28 layers (measured: 1.2e-2 after the 11 steps), while a wrong row, scale or head
    moves it by order 1."""
    cfg = mq.QWEN3_1_7B
    state, _ = mq.random_init_state(cfg, seed=12, norm_jitter=0.1)
    qstate = mq.quantize_state(state, cfg, dev)
    del state
    packed = mq.pack_int8(qstate, cfg)
    del qstate
    S = 16
    cos, sin = mq.precompute_rope_freqs(cfg.head_dim, S, cfg.rope_theta, device=dev)
    model = (cfg, packed, cos, sin, S)
    prompts = _prompts(16, cfg.vocab_size, seed=61)
    print("full 28-layer 1.7B model, batch 16", flush=True)
    _check_against_oracle(mq, model, prompts, 4, shared_ref=_ref(model), check=(0, 5, 10, 15), hidden_tol=2.0 ** -5)
    del packed
    torch.cuda.empty_cache()


def test_batch_hidden_state_matches_oracle(mq, dev, model):
    """Every sequence's last-layer values against the oracle's after the same 8 prompt tokens.
    The batched path applies the RMSNorm scale after the matrix product instead of rounding
    the normalised input to fp32 first, so projections differ from the oracle's by ~1e-8
    relative; that flips an occasional bf16 rounding of a K/V row or hidden value (2^-8
    relative each), which moves later values by up to ~1e-3. The bound is one bf16 ulp
    (2^-8) relative L2 -- the north star's bf16-activation tolerance for config 5."""
    cfg, (embed, layers, scales, lm_q, lm_s, fnorm), cos, sin, S = model
    prompts = _prompts(16, cfg.vocab_size, seed=44)
    dec = mq.A10Int8BatchDecoder(embed, layers, scales, lm_q, lm_s, fnorm, cos, sin, cfg.num_layers, S, 16)
    dec.enable_debug()
    for i in range(8):
        dec.decode_step([p[i] for p in prompts])
    got = dec.get_hidden().float().cpu().double()
    c = lambda t: t.cpu()
    errs = []
    for b, p in enumerate(prompts):
        ref = RefDecoder(Dims(hidden_size=2048, intermediate_size=6144, vocab_size=cfg.vocab_size), c(embed),
                         [c(t) for t in layers], [c(t) for t in scales], c(fnorm), c(lm_q), c(lm_s), c(cos), c(sin),
                         cfg.num_layers, S)
        for t in p:
            ref.step_logits(int(t))
        want = ref.last["hidden"].double()
        e = float(torch.linalg.norm(got[b] - want) / torch.linalg.norm(want))
        diff = float((got[b] != want).double().mean())
        stages = {"attn_out": dec.get_attn_out()[b], "residual": dec.get_activations()[b],
                  "mlp_intermediate": dec.get_mlp_int()[b]}
        rel = {k: float(torch.linalg.norm(v.cpu().double() - ref.last[k].double()) / torch.linalg.norm(ref.last[k].double()))
               for k, v in stages.items()}
        print(f"sequence {b}: hidden rel L2 {e:.2e}, bf16 values differing {diff:.4f}, "
              + ", ".join(f"{k} {v:.2e}" for k, v in rel.items()), flush=True)
        errs.append((b, e, max(rel.values())))
    assert all(e < 2.0 ** -8 and st < 2.0 ** -8 for _, e, st in errs), errs


def test_sequence_independent_of_slot_and_batch(mq, dev, model):
    """The same prompt gives the same tokens alone, in slot 0 of a batch of 4 and in slot 11
    of a batch of 16 (per-sequence digit scales; per-column matrix-core sums)."""
    prompts = _prompts(16, model[0].vocab_size, seed=33)
    _, alone = _run_batch(mq, model, [prompts[11]])
    _, four = _run_batch(mq, model, [prompts[11]] + prompts[:3])
    _, sixteen = _run_batch(mq, model, prompts)
    assert alone[0] == four[0] == sixteen[11]


def test_batch_reset_and_validation(mq, dev, model):
    cfg, packed, cos, sin, S = model
    dec = mq.A10Int8BatchDecoder(*packed, cos, sin, cfg.num_layers, S, 2)
    with pytest.raises(ValueError):
        dec.decode_step([1])                    # wrong count
    with pytest.raises(ValueError):
        dec.decode_step([1, cfg.vocab_size])    # token out of range
    a = dec.decode_step([1, 2])
    assert dec.positions() == [1, 1]
    dec.reset()
    assert dec.positions() == [0, 0] and int(dec.k_cache.abs().sum()) == 0
    assert dec.decode_step([1, 2]) == a
    with pytest.raises(ValueError):
        mq.A10Int8BatchDecoder(*packed, cos, sin, cfg.num_layers, S, 17)
