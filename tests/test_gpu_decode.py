"""GPU parity of the persistent decode kernel (run with -m gpu).

Gates: greedy tokens identical to the float64 oracle's
committed fixtures for 32 steps (INT8 Qwen3-0.6B shape, BF16 Qwen3-0.6B
shape, a 2-layer INT8 case with non-unit norm gains), per-stage values within
fp32-accumulation tolerance of the oracle, bitwise run-to-run determinism, the
reference-signature C launcher agreeing with the class, and the host-forced
failure paths (bad token, full cache, expired in-kernel wait) raising cleanly.
"""
from __future__ import annotations

import ctypes
import json

import pytest
import torch

from oracle.ref_cpu import Dims, RefDecoder, greedy_generate

from .conftest import GOLDEN

pytestmark = pytest.mark.gpu


def _fixture(name):
    return json.loads((GOLDEN / f"tokens_{name}.json").read_text())


def _build(mq, dev, name):
    d = _fixture(name)
    cfg = mq.ModelConfig(**d["config"])
    state, prompt = mq.random_init_state(cfg, seed=d["seed"], norm_jitter=d["norm_jitter"])
    assert mq.state_digest(state) == d["weights_sha256"]
    S = d["max_seq_len"]
    cos, sin = mq.precompute_rope_freqs(cfg.head_dim, S, cfg.rope_theta, device=dev)
    if d["int8"]:
        fmt = d.get("weight_format", "int8")
        qstate = mq.quantize_state(state, cfg, dev, weight_format=fmt)
        embed, layers, scales, lm_q, lm_s, fnorm = mq.pack_int8(qstate, cfg)
        cls = {"fp8": mq.A10Fp8MegakernelDecoder, "int4": mq.A10Int4MegakernelDecoder}.get(fmt, mq.A10Int8MegakernelDecoder)
        dec = cls(embed, layers, scales, lm_q, lm_s, fnorm, cos, sin, cfg.num_layers, S)
        keep = (embed, layers, scales, lm_q, lm_s, fnorm, cos, sin)
    else:
        embed, layers, fnorm, lm = mq.pack_bf16(state, cfg, dev)
        dec = mq.A10MegakernelDecoder(embed, layers, fnorm, lm, cos, sin, cfg.num_layers, S)
        keep = (embed, layers, fnorm, lm, cos, sin)
    return dec, d, prompt.tolist(), cfg, keep


def _greedy(dec, prompt, n):
    dec.reset()
    tok = None
    for t in prompt:
        tok = dec.decode_step(int(t))
    out = [tok]
    while len(out) < n:
        tok = dec.decode_step(tok)
        out.append(tok)
    return out


def _use_variant(mq, name):
    mq.set_decode_variant(name)
    assert mq.decode_variant() == name
    yield name
    mq.set_decode_variant("auto")


@pytest.fixture(params=["xcd", "async"])
def variant(request, mq, dev):
    """Runs a test once per decode kernel the library selects on MI355X (XCD-aware /
    async-wave; the async-wave kernel covers the INT8 Qwen3-0.6B shape up to 2048 cached
    positions). The single-level fallback has its own fixture test below."""
    yield from _use_variant(mq, request.param)


@pytest.fixture(params=["xcd"])
def variant_any_shape(request, mq, dev):
    """The kernel that runs every compiled shape and weight format."""
    yield from _use_variant(mq, request.param)


@pytest.fixture(scope="module")
def small(mq, dev):
    return _build(mq, dev, "small_int8")


def _ref_for(small_case):
    dec, d, prompt, cfg, keep = small_case
    embed, layers, scales, lm_q, lm_s, fnorm, cos, sin = keep
    c = lambda t: t.cpu()
    return RefDecoder(Dims(vocab_size=cfg.vocab_size), c(embed), [c(t) for t in layers], [c(t) for t in scales],
                      c(fnorm), c(lm_q), c(lm_s), c(cos), c(sin), cfg.num_layers, d["max_seq_len"])


def test_small_int8_tokens_match_fixture(variant, small):
    dec, d, prompt, cfg, _ = small
    print("small_int8 32 greedy steps", flush=True)
    assert _greedy(dec, prompt, 32) == d["tokens"]


def test_small_int8_stages_match_oracle(variant, small):
    """Per-stage values of the last layer (the reference's debug getters) after several steps."""
    dec, d, prompt, cfg, _ = small
    ref = _ref_for(small)
    dec.enable_debug()
    dec.reset()
    ref.reset()
    for t in prompt[:5]:
        got_tok = dec.decode_step(int(t))
        ref_logits = ref.step_logits(int(t))
        assert got_tok == int(torch.argmax(ref_logits))
    last = ref.last

    def rel(name, t):
        a = t.detach().cpu().double()
        b = last[name].double()
        return float(torch.linalg.norm(a - b) / torch.linalg.norm(b))

    checks = {"q": dec.get_q(), "k": dec.get_k(), "v": dec.get_v(), "attn_out": dec.get_attn_out(),
              "residual": dec.get_residual(), "activations": dec.get_activations(),
              "mlp_intermediate": dec.get_mlp_int(), "normalized": dec.get_normalized()}
    # after earlier layers, fp32-order differences can flip single bf16 roundings of the
    # hidden state / KV cache, which moves later stages by ~1e-4; the bound is the
    # north-star per-matvec tolerance
    for name, t in checks.items():
        e = rel(name, t)
        print(f"stage {name}: rel L2 {e:.2e}")
        assert e < 1e-3, (name, e)
    h = dec.get_hidden().cpu().float().double()
    e = float(torch.linalg.norm(h - last["hidden"]) / torch.linalg.norm(last["hidden"]))
    assert e < 1e-3, ("hidden", e)
    assert float(((h - last["hidden"]).abs() > 0).double().mean()) < 0.05   # most elements bit-identical
    # the KV cache rows written at the last position match the oracle's bf16 cache
    p = dec.position() - 1
    kc = dec.k_cache[:, :, p].cpu().float()
    rk = ref.k_cache[:, :, p].float()
    assert float((kc - rk).abs().max()) <= float(rk.abs().max()) * 2.0 ** -7


def test_one_layer_stages_tight(variant, mq, dev):
    """One layer, first position: every stage input is bit-identical to the oracle's, so the
    fp32 stages must agree to accumulation error (1e-5) and the bf16 outputs to one ulp."""
    cfg = mq.QWEN3_0_6B.with_(num_layers=1, vocab_size=3000)
    state, prompt = mq.random_init_state(cfg, seed=9, norm_jitter=0.2)
    qstate = mq.quantize_state(state, cfg, dev)
    embed, layers, scales, lm_q, lm_s, fnorm = mq.pack_int8(qstate, cfg)
    S = 8
    cos, sin = mq.precompute_rope_freqs(cfg.head_dim, S, cfg.rope_theta, device=dev)
    dec = mq.A10Int8MegakernelDecoder(embed, layers, scales, lm_q, lm_s, fnorm, cos, sin, 1, S)
    dec.enable_debug()
    c = lambda t: t.cpu()
    ref = RefDecoder(Dims(vocab_size=cfg.vocab_size), c(embed), [c(t) for t in layers], [c(t) for t in scales],
                     c(fnorm), c(lm_q), c(lm_s), c(cos), c(sin), 1, S)
    for step in range(2):
        tok = int(prompt[step])
        got = dec.decode_step(tok)
        logits = ref.step_logits(tok)
        assert got == int(torch.argmax(logits))
        last = ref.last
        stages = {"q": dec.get_q(), "k": dec.get_k(), "v": dec.get_v(), "attn_out": dec.get_attn_out(),
                  "residual": dec.get_residual(), "activations": dec.get_activations(),
                  "mlp_intermediate": dec.get_mlp_int()}
        for name, t in stages.items():
            a, b = t.cpu().double(), last[name].double()
            e = float(torch.linalg.norm(a - b) / torch.linalg.norm(b))
            print(f"step {step} stage {name}: rel L2 {e:.2e}")
            assert e < 1e-5, (step, name, e)
        h = dec.get_hidden().cpu().double()
        assert torch.all((h - last["hidden"]).abs() <= last["hidden"].abs() * 2.0 ** -7)
        e = float(torch.linalg.norm(dec.get_normalized().cpu().double() - last["normalized"].double())
                  / torch.linalg.norm(last["normalized"].double()))
        assert e < 1e-3, e


def test_small_int8_deterministic(variant, small):
    dec, d, prompt, cfg, _ = small
    dec.enable_debug()
    runs = []
    for _ in range(2):
        toks = _greedy(dec, prompt, 12)
        runs.append((toks, dec.get_q().clone(), dec.get_attn_out().clone(), dec.get_mlp_int().clone(),
                     dec.get_hidden().clone(), dec.k_cache.clone(), dec.block_max_vals.clone()))
    a, b = runs
    assert a[0] == b[0]
    for x, y in zip(a[1:], b[1:]):
        assert torch.equal(x, y)
    # the debug and the plain kernels agree
    dec.enable_debug(False)
    assert _greedy(dec, prompt, 12) == a[0]


def test_trace_without_debug_outputs(variant, small, dev):
    """The timing trace alone selects the instrumented kernel with every debug
    output pointer null: it must write through none of them and give the same tokens."""
    dec, d, prompt, cfg, _ = small
    dec.enable_debug(False)
    L = cfg.num_layers
    buf = torch.zeros((L + 1) * 10 * 256, dtype=torch.int64, device=dev)
    dec.set_trace(buf)
    try:
        toks = _greedy(dec, prompt, 12)
    finally:
        dec.set_trace(None)
    assert toks == d["tokens"][:12]
    t = buf.view(L + 1, 10, 256)
    assert bool((t[:L, 0, :] > 0).all()) and bool((t[:L, 1, :] > 0).all())


def test_reset_and_position(small):
    dec, d, prompt, cfg, _ = small
    dec.reset()
    assert dec.position() == 0
    dec.decode_step(int(prompt[0]))
    dec.decode_step(int(prompt[1]))
    assert dec.position() == 2
    assert dec.k_cache.abs().sum() > 0
    dec.reset()
    assert dec.position() == 0 and int(dec.k_cache.abs().sum()) == 0 and int(dec.v_cache.abs().sum()) == 0


def test_invalid_inputs_raise(small):
    dec, d, prompt, cfg, _ = small
    dec.reset()
    with pytest.raises(ValueError):
        dec.decode_step(cfg.vocab_size)
    with pytest.raises(ValueError):
        dec.decode_step(-1)
    for i in range(d["max_seq_len"]):
        dec.launch_step(int(prompt[i % len(prompt)]))
    torch.cuda.synchronize()
    with pytest.raises(ValueError, match="full"):
        dec.decode_step(int(prompt[0]))
    dec.reset()


def test_expired_wait_reports_timeout_and_recovers(variant, mq, small):
    """A one-poll spin limit makes every cross-workgroup wait expire: the step must end,
    report MQ_ERR_TIMEOUT, and the decoder must work again after its workspace reset."""
    dec, d, prompt, cfg, _ = small
    dec.reset()
    dec.set_spin_limit(1)
    with pytest.raises(mq._lib.MQTimeoutError):
        for t in prompt:
            dec.decode_step(int(t))
    dec.set_spin_limit(0)
    assert _greedy(dec, prompt, 8) == d["tokens"][:8]


def test_full_int8_32_tokens(variant, mq, dev):
    """BASELINE config 1 gate: Qwen3-0.6B shape, INT8, seed 0, 32 greedy tokens identical to the oracle."""
    print("building qwen3_0.6b_int8", flush=True)
    dec, d, prompt, cfg, keep = _build(mq, dev, "qwen3_0.6b_int8")
    toks = _greedy(dec, prompt, 32)
    assert toks == d["tokens"], (toks, d["tokens"])
    # the reference-signature launcher on the same buffers reproduces the last step
    lib = mq._lib.load()
    embed, layers, scales, lm_q, lm_s, fnorm, cos, sin = keep
    dec.reset()
    out = torch.zeros(1, dtype=torch.int32, device=dev)
    stream = ctypes.c_void_p(mq._lib.stream_handle(dev))
    for pos, t in enumerate(prompt):
        lib.launch_a10_int8_decode(int(t), out.data_ptr(), embed.data_ptr(), dec.d_layer_weights.data_ptr(),
                                   fnorm.data_ptr(), lm_q.data_ptr(), lm_s.data_ptr(), cos.data_ptr(),
                                   sin.data_ptr(), dec.k_cache.data_ptr(), dec.v_cache.data_ptr(),
                                   None, None, None, None, None, None, None, None, None, None, None,
                                   cfg.num_layers, pos, pos + 1, d["max_seq_len"], dec.attn_scale,
                                   dec.d_layer_scales.data_ptr(), stream)
        assert mq._lib.last_error() == "", mq._lib.last_error()
    torch.cuda.synchronize()
    assert int(out.item()) == d["tokens"][0]
    del dec, keep
    torch.cuda.empty_cache()


def test_full_bf16_32_tokens(variant_any_shape, mq, dev):
    """BASELINE config 3 gate: Qwen3-0.6B shape, bf16 weights, 32 greedy tokens identical to the oracle."""
    print("building qwen3_0.6b_bf16", flush=True)
    dec, d, prompt, cfg, keep = _build(mq, dev, "qwen3_0.6b_bf16")
    toks = _greedy(dec, prompt, 32)
    assert toks == d["tokens"], (toks, d["tokens"])
    del dec, keep
    torch.cuda.empty_cache()


@pytest.mark.parametrize("name", ["small_int8", "qwen3_0.6b_int8", "qwen3_0.6b_bf16"])
def test_single_level_fallback_fixtures(mq, dev, name):
    """The single-level kernel (the fallback for devices whose workgroup placement does not
    fit the XCD-aware kernel; never selected on MI355X) against the 32-token fixtures."""
    print(f"single-level kernel, {name}", flush=True)
    dec, d, prompt, cfg, keep = _build(mq, dev, name)
    mq.set_decode_variant("flat")
    try:
        assert mq.decode_variant(cfg.hidden_size, cfg.intermediate_size, int8=d["int8"]) == "flat"
        assert _greedy(dec, prompt, 32) == d["tokens"]
    finally:
        mq.set_decode_variant("auto")
    del dec, keep
    torch.cuda.empty_cache()


def test_1p7b_int8_matches_oracle(variant_any_shape, mq, dev):
    """Qwen3-1.7B layer shapes (H=2048, I=6144), 2 layers, small vocabulary, live oracle."""
    cfg = mq.QWEN3_1_7B.with_(num_layers=2, vocab_size=2048)
    state, prompt = mq.random_init_state(cfg, seed=5, norm_jitter=0.1)
    qstate = mq.quantize_state(state, cfg, dev)
    embed, layers, scales, lm_q, lm_s, fnorm = mq.pack_int8(qstate, cfg)
    S = 32
    cos, sin = mq.precompute_rope_freqs(cfg.head_dim, S, cfg.rope_theta, device=dev)
    dec = mq.A10Int8MegakernelDecoder(embed, layers, scales, lm_q, lm_s, fnorm, cos, sin, cfg.num_layers, S)
    toks = _greedy(dec, prompt.tolist(), 12)
    c = lambda t: t.cpu()
    ref = RefDecoder(Dims(hidden_size=2048, intermediate_size=6144, vocab_size=cfg.vocab_size), c(embed),
                     [c(t) for t in layers], [c(t) for t in scales], c(fnorm), c(lm_q), c(lm_s), c(cos), c(sin),
                     cfg.num_layers, S)
    want, margins = greedy_generate(ref, prompt.tolist(), 12)
    assert toks == want, (toks, want, margins)


def test_failed_step_resumes_without_reset(mq, small):
    """A step whose in-kernel waits expire (spin limit of one poll; every kernel still exits)
    raises MQTimeoutError and leaves the decoder at that step's position: feeding the same
    token again continues the sequence, with no reset, to the fixture's tokens
    (bench_int8.py:193-219 semantics for position and cache)."""
    dec, d, prompt, cfg, _ = small
    dec.reset()
    for t in prompt[:3]:
        dec.decode_step(int(t))
    dec.set_spin_limit(1)
    with pytest.raises(mq._lib.MQTimeoutError):
        for t in prompt[3:]:
            dec.decode_step(int(t))
    dec.set_spin_limit(0)
    resume = dec.position()
    assert 3 <= resume < len(prompt), resume
    tok = None
    for t in prompt[resume:]:
        tok = dec.decode_step(int(t))
    out = [tok]
    while len(out) < 12:
        tok = dec.decode_step(tok)
        out.append(tok)
    assert out == d["tokens"][:12], (out, d["tokens"][:12])


def test_pipelined_steps_keep_their_own_tokens(small):
    """Steps launched back to back without reading their tokens (each has its own token word):
    the last one's token is the fixture's, however many are in flight."""
    dec, d, prompt, cfg, _ = small
    dec.reset()
    for t in prompt:
        dec.launch_step(int(t))
    assert dec.wait_token() == d["tokens"][0]
    with pytest.raises(RuntimeError):
        dec.wait_token()                        # nothing in flight any more


def _reference_scratch(dev, H, I, n_partials=1184):
    """The scratch buffers the reference's INT8 class allocates (bench_int8.py:176-188)."""
    f32 = lambda n: torch.zeros(n, dtype=torch.float32, device=dev)
    return {"hidden_buffer": torch.zeros(H, dtype=torch.bfloat16, device=dev), "g_activations": f32(H),
            "g_residual": f32(H), "g_q": f32(2048), "g_k": f32(1024), "g_v": f32(1024), "g_attn_out": f32(2048),
            "g_mlp_intermediate": f32(I), "g_normalized": f32(H), "block_max_vals": f32(n_partials),
            "block_max_idxs": torch.zeros(n_partials, dtype=torch.int32, device=dev)}


_SCRATCH_ORDER = ("hidden_buffer", "g_activations", "g_residual", "g_q", "g_k", "g_v", "g_attn_out",
                  "g_mlp_intermediate", "g_normalized", "block_max_vals", "block_max_idxs")


class _reference_dims:
    """The reference-signature launchers assume Qwen3-0.6B unless told otherwise
    (mq_reference_set_dims): declare a test model's dims for the duration of a block."""

    def __init__(self, mq, cfg):
        self.lib = mq._lib.load()
        self.dims = mq._lib.ModelDims(cfg.hidden_size, cfg.intermediate_size, 16, 8, 128, cfg.vocab_size)

    def __enter__(self):
        assert self.lib.mq_reference_set_dims(ctypes.byref(self.dims)) == 0

    def __exit__(self, *exc):
        self.lib.mq_reference_set_dims(None)


def _reference_drive(mq, dev, d, prompt, n, launch, scr):
    """Prefill + greedy decode through a reference-signature launcher, the way
    bench_int8.py:193-219 drives it (token buffer on the device, .item() per step)."""
    out_tok = torch.zeros(1, dtype=torch.int32, device=dev)
    toks, seq, pos = [], list(prompt), 0
    while len(toks) < n:
        launch(int(seq[pos]), out_tok, pos, [scr[k].data_ptr() for k in _SCRATCH_ORDER])
        assert mq._lib.last_error() == "", mq._lib.last_error()
        tok = int(out_tok.item())
        pos += 1
        if pos >= len(prompt):
            toks.append(tok)
            seq.append(tok)
    return toks


def test_reference_int8_launcher_with_scratch_buffers(mq, dev, small):
    """launch_a10_int8_decode called exactly as the reference's class calls it, every scratch
    buffer set (sized as bench_int8.py allocates them): 32 fixture tokens, and the debug
    buffers hold the last layer's values of the last step (run_benchmark.py:174-183)."""
    dec, d, prompt, cfg, keep = small
    embed, layers, scales, lm_q, lm_s, fnorm, cos, sin = keep
    lib, S = mq._lib.load(), d["max_seq_len"]
    kc = torch.zeros((cfg.num_layers, 8, S, 128), dtype=torch.bfloat16, device=dev)
    vc = torch.zeros_like(kc)
    scr = _reference_scratch(dev, cfg.hidden_size, cfg.intermediate_size)
    stream = ctypes.c_void_p(mq._lib.stream_handle(dev))

    def launch(tok, out_tok, pos, ptrs):
        lib.launch_a10_int8_decode(tok, out_tok.data_ptr(), embed.data_ptr(), dec.d_layer_weights.data_ptr(),
                                   fnorm.data_ptr(), lm_q.data_ptr(), lm_s.data_ptr(), cos.data_ptr(), sin.data_ptr(),
                                   kc.data_ptr(), vc.data_ptr(), *ptrs, cfg.num_layers, pos, pos + 1, S,
                                   dec.attn_scale, dec.d_layer_scales.data_ptr(), stream)

    with _reference_dims(mq, cfg):
        toks = _reference_drive(mq, dev, d, prompt, 32, launch, scr)
    assert toks == d["tokens"], (toks, d["tokens"])
    # the debug buffers of the last step against the oracle run over the same tokens
    ref = _ref_for(small)
    ref.reset()
    for t in (list(prompt) + toks)[: len(prompt) + 31]:
        ref.step_logits(int(t))
    last = ref.last
    for name, key in (("q", "g_q"), ("k", "g_k"), ("v", "g_v"), ("attn_out", "g_attn_out"),
                      ("residual", "g_residual"), ("activations", "g_activations"),
                      ("mlp_intermediate", "g_mlp_intermediate"), ("normalized", "g_normalized")):
        a, b = scr[key].cpu().double(), last[name].double()
        e = float(torch.linalg.norm(a - b) / torch.linalg.norm(b))
        assert e < 1e-3, (name, e)
    h = scr["hidden_buffer"].cpu().float().double()
    assert float(torch.linalg.norm(h - last["hidden"]) / torch.linalg.norm(last["hidden"])) < 1e-3
    # per-workgroup maxima: the largest is the step's token
    bv, bi = scr["block_max_vals"][:256].cpu(), scr["block_max_idxs"][:256].cpu()
    assert int(bi[int(torch.argmax(bv))]) == toks[-1]


def test_reference_bf16_launcher(mq, dev):
    """launch_a10_decode (a10_decode_kernel.cu:761-780) driven through ctypes for 8 prompt and 32
    greedy steps, scratch buffers as a10_decode.py allocates them: the bf16 fixture's tokens."""
    print("building qwen3_0.6b_bf16", flush=True)
    dec, d, prompt, cfg, keep = _build(mq, dev, "qwen3_0.6b_bf16")
    embed, layers, fnorm, lm, cos, sin = keep
    lib, S = mq._lib.load(), d["max_seq_len"]
    kc = torch.zeros((cfg.num_layers, 8, S, 128), dtype=torch.bfloat16, device=dev)
    vc = torch.zeros_like(kc)
    scr = _reference_scratch(dev, cfg.hidden_size, cfg.intermediate_size)
    stream = ctypes.c_void_p(mq._lib.stream_handle(dev))

    def launch(tok, out_tok, pos, ptrs):
        lib.launch_a10_decode(tok, out_tok.data_ptr(), embed.data_ptr(), dec.d_layer_weights.data_ptr(),
                              fnorm.data_ptr(), lm.data_ptr(), cos.data_ptr(), sin.data_ptr(), kc.data_ptr(),
                              vc.data_ptr(), *ptrs, cfg.num_layers, pos, pos + 1, S, dec.attn_scale, stream)

    toks = _reference_drive(mq, dev, d, prompt, 32, launch, scr)
    assert toks == d["tokens"], (toks, d["tokens"])
    del dec, keep, kc, vc
    torch.cuda.empty_cache()


def test_reference_launcher_recovers_after_failed_step(mq, dev, small):
    """A step of launch_a10_int8_decode whose waits expire stores token -1; the next call
    reports that failure through mq_last_error(), re-initialises the library-owned workspace
    and launches, so the sequence continues (the failed position is fed again)."""
    dec, d, prompt, cfg, keep = small
    embed, layers, scales, lm_q, lm_s, fnorm, cos, sin = keep
    lib, S = mq._lib.load(), d["max_seq_len"]
    kc = torch.zeros((cfg.num_layers, 8, S, 128), dtype=torch.bfloat16, device=dev)
    vc = torch.zeros_like(kc)
    stream = ctypes.c_void_p(mq._lib.stream_handle(dev))
    out_tok = torch.zeros(1, dtype=torch.int32, device=dev)

    def step(tok, pos):
        lib.launch_a10_int8_decode(tok, out_tok.data_ptr(), embed.data_ptr(), dec.d_layer_weights.data_ptr(),
                                   fnorm.data_ptr(), lm_q.data_ptr(), lm_s.data_ptr(), cos.data_ptr(), sin.data_ptr(),
                                   kc.data_ptr(), vc.data_ptr(), *([None] * 11), cfg.num_layers, pos, pos + 1, S,
                                   dec.attn_scale, dec.d_layer_scales.data_ptr(), stream)
        msg = mq._lib.last_error()
        return int(out_tok.item()), msg

    with _reference_dims(mq, cfg):
        _recover_after_failed_step(lib, step, prompt, d)


def _recover_after_failed_step(lib, step, prompt, d):
    for pos in range(3):
        _, msg = step(int(prompt[pos]), pos)
        assert msg == "", msg
    lib.mq_reference_set_spin_limit(1)
    try:
        tok, _ = step(int(prompt[3]), 3)
    finally:
        lib.mq_reference_set_spin_limit(0)
    assert tok == -1
    tok, msg = step(int(prompt[3]), 3)          # the failed position again
    assert "previous step failed" in msg, msg
    for pos in range(4, len(prompt)):
        tok, msg = step(int(prompt[pos]), pos)
        assert msg == "", msg
    toks, pos = [tok], len(prompt)
    while len(toks) < 8:
        tok, msg = step(tok, pos)
        assert msg == "", msg
        toks.append(tok)
        pos += 1
    assert toks == d["tokens"][:8], (toks, d["tokens"][:8])


@pytest.mark.parametrize("int8", [True, False])
def test_a10decoder_generate(mq, dev, int8):
    """A10Decoder (a10_decode.py:35-393) with seeded random weights: generate() prefills one
    decode_step per prompt token and takes the last prefill output as the first generated token
    (verify_correctness_a10.py:323-339), giving the config-1 / config-3 fixtures' 32 tokens."""
    d = _fixture("qwen3_0.6b_int8" if int8 else "qwen3_0.6b_bf16")
    print(f"A10Decoder int8={int8}", flush=True)
    dec = mq.A10Decoder(seed=d["seed"], int8=int8, max_seq_len=d["max_seq_len"], device=dev)
    ids, tok_s, times = dec.generate(d["prompt"], 32)
    assert ids[:8] == d["prompt"]
    assert ids[8:] == d["tokens"], (ids[8:], d["tokens"])
    assert tok_s > 0 and len(times) == 31
    del dec
    torch.cuda.empty_cache()


def test_forced_kernel_out_of_range_is_refused(mq, dev, small):
    """A kernel forced by set_decode_variant that cannot run a step refuses it with MQError
    (nothing launched, position unchanged) instead of running another kernel: the
    async-wave kernel past its 10240 positions."""
    dec0, d, prompt, cfg, keep = small
    embed, layers, scales, lm_q, lm_s, fnorm, _, _ = keep
    S = 10250
    cos, sin = mq.precompute_rope_freqs(cfg.head_dim, S, cfg.rope_theta, device=dev)
    dec = mq.A10Int8MegakernelDecoder(embed, layers, scales, lm_q, lm_s, fnorm, cos, sin, cfg.num_layers, S)
    dec.prefill_random_kv(10240, seed=1)
    mq.set_decode_variant("async")
    try:
        with pytest.raises(mq._lib.MQError, match="async-wave"):
            dec.decode_step(int(prompt[0]))
    finally:
        mq.set_decode_variant("auto")
    assert dec.position() == 10240
    assert 0 <= dec.decode_step(int(prompt[0])) < cfg.vocab_size          # the automatic choice runs it
    del dec
    torch.cuda.empty_cache()
