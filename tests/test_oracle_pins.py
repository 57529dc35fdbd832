"""Pins the CPU oracle against things other than itself (runs on CPU).

* quantizer: the torch restatement vs the independent C restatement
  (oracle/c/oracle.c), invariants of round-to-nearest-even quantization, the
  committed fixture, and hand-derived tie cases;
* RoPE tables: float64 closed form, structure (split-half duplication,
  row 0), the committed rows;
* decode step: with the rounding points switched off, the oracle must
  reproduce HF transformers' Qwen3 forward pass in float64 (architecture:
  norm placement, QK-norm, RoPE convention, GQA head mapping, SwiGLU,
  residuals, tied LM head, attention scale); with them on, the documented
  rounding points (bf16 hidden, bf16 KV) must hold;
* the committed greedy-token fixtures must be reproduced.
"""
from __future__ import annotations

import ctypes
import json
import math

import numpy as np
import pytest
import torch

from oracle import quant as oquant
from oracle import rope as orope
from oracle.ref_cpu import Dims, RefDecoder, greedy_generate

from .conftest import GOLDEN, ROOT


@pytest.fixture(scope="module")
def coracle():
    path = ROOT / "oracle" / "lib" / "liboracle.so"
    if not path.exists():
        import subprocess
        subprocess.run(["make", "-s", "-C", str(ROOT / "oracle")], check=True)
    return ctypes.CDLL(str(path))


def c_quantize(lib, w):
    M, K = w.shape
    bits = w.contiguous().view(torch.int16).numpy().view(np.uint16).copy()
    q = np.empty((M, K), np.int8)
    s = np.empty(M, np.float32)
    lib.oracle_quantize_bf16(bits.ctypes.data_as(ctypes.c_void_p), ctypes.c_int64(M), ctypes.c_int64(K),
                             q.ctypes.data_as(ctypes.c_void_p), s.ctypes.data_as(ctypes.c_void_p))
    return q, s


# ---------------------------------------------------------------- quantizer
def test_quantizer_matches_c_restatement(coracle):
    g = torch.Generator().manual_seed(11)
    w = (torch.randn(512, 1024, generator=g) * 0.02).to(torch.bfloat16)
    w[3] = 0
    w[7, 100] = 5.0
    q, s = oquant.quantize_per_channel(w)
    qc, sc = c_quantize(coracle, w)
    assert np.array_equal(q.numpy(), qc)
    assert np.array_equal(s.numpy(), sc)


def test_quantizer_invariants():
    g = torch.Generator().manual_seed(12)
    w = (torch.randn(256, 333, generator=g) * 0.02).to(torch.bfloat16)
    q, s = oquant.quantize_per_channel(w)
    wf = w.float()
    amax = wf.abs().amax(1)
    # the scale is the bf16 rounding of amax/127 (so it is bf16-representable) ...
    assert torch.equal(s, s.to(torch.bfloat16).float())
    assert torch.all((s - amax / 127).abs() <= (amax / 127) * 2.0 ** -8)
    # ... every code is within half a step of w/s (round to nearest), and the
    # row maximum lands on +-127 (or +-126/128 clamped, when the bf16 scale rounded)
    err = (q.double() * s.double()[:, None] - wf.double()).abs()
    clamped = (wf / s[:, None]).abs() > 127.5
    assert torch.all(err[~clamped] <= s.double()[:, None].expand_as(err)[~clamped] / 2 + 1e-12)
    top = q.gather(1, wf.abs().argmax(1, keepdim=True)).abs().squeeze(1)
    assert torch.all((top >= 126) & (top <= 127))


def test_quantizer_ties_and_edges():
    d = np.load(GOLDEN / "quant_cases.npz")
    w = torch.from_numpy(d["w_bits"].view(np.int16)).view(torch.bfloat16)
    q, s = oquant.quantize_per_channel(w)
    assert np.array_equal(q.numpy(), d["q"]) and np.array_equal(s.numpy(), d["scale"])
    # row 0 is all zeros: scale clamps to 1e-12 (as fp32) and every code is 0
    assert s[0] == torch.tensor(1e-12, dtype=torch.float32) and torch.all(q[0] == 0)
    # a single negative element maps to -127
    assert q[1, 5] == -127 and int((q[1] != 0).sum()) == 1
    # rows 7..9 hold w = c * 2^e with c in {127, .5, 1.5, 2.5, -.5, -1.5, 126.5, -127}: ties go to even
    expect = torch.tensor([127, 0, 2, 2, 0, -2, 126, -127] * 8, dtype=torch.int8)
    for r in (7, 8, 9):
        assert torch.equal(q[r], expect), (r, q[r][:8])
    # generic: wherever w/s is exactly a half-integer the code is the even neighbour
    ratio = w.double() / s.double()[:, None]
    half = (ratio - ratio.floor()) == 0.5
    assert int(half.sum()) >= 24
    lo = ratio.floor()
    even = torch.where(torch.remainder(lo, 2) == 0, lo, lo + 1).clamp(-128, 127)
    assert torch.equal(q.double()[half], even[half])


# ---------------------------------------------------------------- rope
def test_rope_split_half_closed_form():
    S, D, theta = 8192, 128, 1e6
    c, s = orope.split_half_tables(S, D, theta)
    assert torch.equal(c[:, :64], c[:, 64:]) and torch.equal(s[:, :64], s[:, 64:])
    assert torch.all(c[0] == 1) and torch.all(s[0] == 0)
    p = torch.arange(S, dtype=torch.float64)[:, None]
    f = theta ** (-torch.arange(0, D, 2, dtype=torch.float64) / D)
    ang = p * f[None, :]
    # bf16 rounding (2^-9 relative) plus the fp32 phase error of p * inv_freq (~ p * 2^-24)
    tol = 2.0 ** -8 + ang * 2.0 ** -22 + 1e-7
    assert torch.all((c[:, :64].double() - torch.cos(ang)).abs() <= tol)
    assert torch.all((s[:, :64].double() - torch.sin(ang)).abs() <= tol)


def test_rope_legacy_closed_form():
    c, s = orope.pair_duplicated_tables(64, 128, 1e4)
    assert torch.equal(c[:, 0::2], c[:, 1::2]) and torch.equal(s[:, 0::2], s[:, 1::2])
    ang = torch.arange(64, dtype=torch.float64)[:, None] / (1e4 ** (torch.arange(0, 128, 2) / 128.0))[None, :]
    assert torch.all((c[:, 0::2].double() - torch.cos(ang)).abs() <= 2.0 ** -8)


def test_rope_golden_rows(mq):
    d = np.load(GOLDEN / "rope_rows.npz")
    c, s = orope.split_half_tables(8192, 128, 1e6)
    bits = lambda t: t.view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(bits(c[d["pos"]]), d["cos"]) and np.array_equal(bits(s[d["pos"]]), d["sin"])
    # the library's own table builder produces the same bits
    pc, ps = mq.precompute_rope_freqs(128, 8192, 1e6)
    assert torch.equal(pc, c) and torch.equal(ps, s)
    lc, ls = orope.pair_duplicated_tables(2048, 128, 1e4)
    assert np.array_equal(bits(lc[d["legacy_pos"]]), d["legacy_cos"])
    mc, ms = mq.make_rope(2048, 128)
    assert torch.equal(mc, lc) and torch.equal(ms, ls)


# ---------------------------------------------------------------- decode step vs HF Qwen3
def _tiny_hf_model(seed=0):
    transformers = pytest.importorskip("transformers")
    cfg = transformers.Qwen3Config(vocab_size=97, hidden_size=64, intermediate_size=96, num_hidden_layers=2,
                                   num_attention_heads=4, num_key_value_heads=2, head_dim=16, rms_norm_eps=1e-6,
                                   rope_theta=1e6, tie_word_embeddings=True, max_position_embeddings=64,
                                   attention_bias=False, attn_implementation="eager")
    torch.manual_seed(seed)
    model = transformers.Qwen3ForCausalLM(cfg).to(torch.float64).eval()
    g = torch.Generator().manual_seed(seed + 1)
    with torch.no_grad():
        for name, p in model.named_parameters():
            if "norm" in name:
                p.copy_(1.0 + 0.2 * torch.randn(p.shape, generator=g, dtype=torch.float64))
            else:
                p.copy_(0.3 * torch.randn(p.shape, generator=g, dtype=torch.float64))
    return model


def _hf_layers(sd, L):
    layers = []
    for i in range(L):
        p = f"model.layers.{i}"
        layers += [sd[f"{p}.input_layernorm.weight"], sd[f"{p}.self_attn.q_proj.weight"],
                   sd[f"{p}.self_attn.k_proj.weight"], sd[f"{p}.self_attn.v_proj.weight"],
                   sd[f"{p}.self_attn.q_norm.weight"], sd[f"{p}.self_attn.k_norm.weight"],
                   sd[f"{p}.self_attn.o_proj.weight"], sd[f"{p}.post_attention_layernorm.weight"],
                   sd[f"{p}.mlp.gate_proj.weight"], sd[f"{p}.mlp.up_proj.weight"], sd[f"{p}.mlp.down_proj.weight"]]
    return layers


def _max_gap_vs_hf(mutate=None):
    """Largest |oracle - HF| logit gap over an 8-token sequence, relative to max |logit|."""
    model = _tiny_hf_model()
    sd = model.state_dict()
    L, D, S = 2, 16, 16
    layers = _hf_layers(sd, L)
    if mutate is not None:
        layers = mutate(list(layers))
    inv = 1e6 ** (-torch.arange(0, D, 2, dtype=torch.float64) / D)
    ang = torch.arange(S, dtype=torch.float64)[:, None] * inv[None, :]
    cos, sin = torch.cat([ang.cos(), ang.cos()], 1), torch.cat([ang.sin(), ang.sin()], 1)
    dims = Dims(hidden_size=64, intermediate_size=96, num_q_heads=4, num_kv_heads=2, head_dim=D, vocab_size=97)
    ref = RefDecoder(dims, sd["model.embed_tokens.weight"], layers, None, sd["model.norm.weight"],
                     sd["lm_head.weight"], None, cos, sin, L, S, dtype=torch.float64, rounding=False)
    ref.attn_scale = 1.0 / math.sqrt(D)
    ids = [5, 17, 3, 96, 0, 42, 42, 7]
    with torch.no_grad():
        hf_logits = model(torch.tensor([ids])).logits[0]
    gap = 0.0
    for t, tok in enumerate(ids):
        ours = ref.step_logits(tok)
        gap = max(gap, float((ours - hf_logits[t]).abs().max() / hf_logits[t].abs().max()))
    return gap


def test_oracle_architecture_matches_hf_qwen3():
    # HF computes RMSNorm in fp32 even for a float64 model, so agreement is ~1e-7, not 1e-15
    assert _max_gap_vs_hf() < 1e-5


@pytest.mark.parametrize("swap", [(4, 5), (0, 7), (8, 9)], ids=["q_norm<->k_norm", "in_ln<->post_ln", "gate<->up"])
def test_hf_pin_detects_wiring_mistakes(swap):
    """A plausible wiring mistake planted in the oracle's inputs breaks the HF comparison."""
    def mutate(layers):
        for l in range(2):
            a, b = 11 * l + swap[0], 11 * l + swap[1]
            layers[a], layers[b] = layers[b], layers[a]
        return layers
    assert _max_gap_vs_hf(mutate) > 1e-3


def test_oracle_rounding_points():
    """With rounding on, the layer output is bf16-representable and the cache holds bf16(k'), bf16(v)."""
    d = json.loads((GOLDEN / "tokens_small_int8.json").read_text())
    from tests.golden.make_golden import oracle_for
    dec, prompt, cfg, _ = oracle_for("small_int8")
    dec.step_logits(int(prompt[0]))
    h = dec.last["hidden"]
    assert torch.equal(h, h.to(torch.bfloat16).to(torch.float64))
    assert torch.equal(dec.k_cache[-1, :, 0].double().reshape(-1), dec.last["k"].to(torch.float32).to(torch.bfloat16).double())
    assert torch.equal(dec.v_cache[-1, :, 0].double().reshape(-1), dec.last["v"].to(torch.float32).to(torch.bfloat16).double())
    assert d["case"] == "small_int8"


# ---------------------------------------------------------------- fixtures
def _check_tokens(name, dtype=torch.float64):
    from tests.golden.make_golden import oracle_for
    d = json.loads((GOLDEN / f"tokens_{name}.json").read_text())
    dec, prompt, cfg, digest = oracle_for(name, dtype=dtype)
    assert digest == d["weights_sha256"], "random-init weight generator drifted"
    assert prompt.tolist() == d["prompt"]
    toks, margins = greedy_generate(dec, prompt.tolist(), len(d["tokens"]))
    assert toks == d["tokens"]
    return margins


def test_small_fixture_reproduced():
    _check_tokens("small_int8")


def test_small_fixture_fp32_port_agrees():
    # the plain fp32 port (the CPU baseline) yields the same tokens as the float64 oracle
    _check_tokens("small_int8", dtype=torch.float32)


def test_full_int8_fixture_reproduced():
    margins = _check_tokens("qwen3_0.6b_int8")
    assert min(margins) > 1e-3


# ---- sampling restatement (oracle.ref_cpu.gumbel_noise / sampled_choice) ----------------

def test_splitmix64_known_answers():
    """splitmix64_mix(k * golden) is the k-th output of SplitMix64 started from state 0; the
    first three are the published values of the generator's reference implementation."""
    from oracle.ref_cpu import _GOLDEN, splitmix64_mix
    want = [0xE220A8397B1DCDAF, 0x6E789E6AA1B965F4, 0x06C45D188009454F]
    assert [splitmix64_mix((k * _GOLDEN) % 2 ** 64) for k in (1, 2, 3)] == want
    import numpy as np
    keys = np.array([(k * _GOLDEN) % 2 ** 64 for k in (1, 2, 3)], dtype=np.uint64)
    assert [int(v) for v in splitmix64_mix(keys)] == want       # the numpy path wraps the same way


def test_gumbel_noise_matches_integer_restatement():
    """The vectorised noise against a big-integer restatement, u exactly in (0, 1)."""
    import math
    import numpy as np
    from oracle.ref_cpu import _GOLDEN, gumbel_noise, splitmix64_mix
    rng = np.random.default_rng(5)
    for _ in range(20):
        seed = int(rng.integers(0, 2 ** 63)) * 2 + int(rng.integers(0, 2))
        pos = int(rng.integers(0, 40000))
        rows = rng.integers(0, 151936, size=16)
        got = gumbel_noise(seed, pos, rows)
        for r, gv in zip(rows.tolist(), got.tolist()):
            z = splitmix64_mix(seed ^ ((((pos << 32) | r) * _GOLDEN) % 2 ** 64))
            u = ((z >> 41) + 0.5) * 2.0 ** -23
            assert 0.0 < u < 1.0
            assert math.isclose(gv, -math.log(-math.log(u)), rel_tol=1e-14)   # numpy's log vs libm's: an ulp


def test_gumbel_max_samples_softmax():
    """argmax(logits / T + g) over independent noise (one position per draw) follows
    softmax(logits / T): frequencies within 5 standard errors over 40,000 draws."""
    import numpy as np
    from oracle.ref_cpu import sampled_choice
    logits = np.array([1.0, 0.5, -0.3, 2.0, 1.7])
    T = 0.7
    p = np.exp(logits / T - np.max(logits / T))
    p /= p.sum()
    n = 40000
    counts = np.zeros(len(logits))
    for pos in range(n):
        tok, _ = sampled_choice(logits, T, seed=12345, pos=pos)
        counts[tok] += 1
    se = np.sqrt(p * (1 - p) / n)
    assert np.all(np.abs(counts / n - p) < 5 * se), (counts / n, p)


def test_gumbel_max_detects_wrong_temperature():
    """The frequency check above fails for a sampler at the wrong temperature (T^2)."""
    import numpy as np
    from oracle.ref_cpu import sampled_choice
    logits = np.array([1.0, 0.5, -0.3, 2.0, 1.7])
    T = 0.7
    p = np.exp(logits / T - np.max(logits / T))
    p /= p.sum()
    n = 20000
    counts = np.zeros(len(logits))
    for pos in range(n):
        tok, _ = sampled_choice(logits, T * T, seed=7, pos=pos)
        counts[tok] += 1
    se = np.sqrt(p * (1 - p) / n)
    assert not np.all(np.abs(counts / n - p) < 5 * se)


# ---- other weight formats (oracle/formats.py) -----------------------------------------
def test_fp8_decode_known_answers():
    """OCP E4M3FN values of landmark codes (exponent bias 7, subnormals m * 2^-9, 0x7F NaN)."""
    import math
    from oracle.formats import fp8_decode_table
    t = fp8_decode_table()
    want = {0x00: 0.0, 0x01: 2.0 ** -9, 0x07: 7 * 2.0 ** -9, 0x08: 2.0 ** -6, 0x38: 1.0, 0x3F: 1.875,
            0x40: 2.0, 0x7E: 448.0, 0xB8: -1.0, 0xFE: -448.0, 0x80: 0.0}
    for c, v in want.items():
        assert t[c] == v, (hex(c), t[c], v)
    assert math.copysign(1.0, t[0x80]) == -1.0
    assert np.isnan(t[0x7F]) and np.isnan(t[0xFF])
    assert np.sum(np.isnan(t)) == 2
    finite = t[:0x7F]
    assert np.all(np.diff(finite) > 0)                       # codes 0..0x7E increase strictly


def _fp8_brute(x: float) -> int:
    """Nearest finite code by exhaustive search; ties to the even code; saturation at 448."""
    from oracle.formats import fp8_decode_table
    t = fp8_decode_table()[:0x7F]
    a = abs(x)
    sign = 0x80 if np.signbit(np.float32(x)) else 0
    if a >= 448.0:
        return sign | 0x7E
    d = np.abs(t - a)
    best = np.flatnonzero(d == d.min())
    c = int(best[0]) if len(best) == 1 else int([b for b in best if b % 2 == 0][0])
    return sign | c


def test_fp8_encode_brute_force():
    from oracle.formats import fp8_decode_table, fp8_encode
    t = fp8_decode_table()[:0x7F]
    rng = np.random.default_rng(3)
    xs = list(rng.choice([-1.0, 1.0], 3000) * 2.0 ** rng.uniform(-13, 10, 3000))
    xs += [float((t[i] + t[i + 1]) / 2) for i in range(0x7E)]          # every midpoint: ties
    xs += [float(-(t[i] + t[i + 1]) / 2) for i in range(0x7E)]
    xs += [0.0, -0.0, 447.9, 448.0, 455.0, 464.0, 470.0, 480.0, 1e9, 2.0 ** -10, 2.0 ** -11, 3 * 2.0 ** -11]
    xs32 = np.array(xs, dtype=np.float32)
    got = fp8_encode(xs32)
    for x, g in zip(xs32, got):
        assert int(g) == _fp8_brute(float(x)), (float(x), hex(int(g)), hex(_fp8_brute(float(x))))


def test_fp8_quantizer_round_trip():
    """Every element's dequantized value is the nearest representable one: within half a step."""
    from oracle.formats import dequant_fp8, quantize_fp8_rows
    g = torch.Generator().manual_seed(11)
    w = (torch.randn(37, 96, generator=g) * 0.02).to(torch.bfloat16)
    w[3] = 0
    q, s = quantize_fp8_rows(w)
    d = dequant_fp8(q, s)
    wf = w.double().numpy()
    assert np.all(d[3] == 0) and s[3].item() == np.float32(1e-12)
    rel = np.abs(d - wf) / np.maximum(np.abs(wf), 1e-30)
    big = np.abs(wf) >= s.numpy()[:, None] * 2.0 ** -6                 # normal range of the codes
    assert np.all(rel[big] <= 2.0 ** -4 + 1e-7)
    assert np.all(np.abs(q.numpy().astype(np.int64) & 0x7F) <= 0x7E)
    amax_code = (q.numpy()[np.arange(37) != 3] & 0x7F).max(axis=1)
    assert np.all(amax_code == 0x7E)                                   # each row's largest maps to 448


def test_int4_quantizer_matches_torch_expression():
    """The numpy restatement against the INT8 quantizer's torch expression with 7 and a group axis."""
    from oracle.formats import quantize_int4_groups, unpack_int4
    g = torch.Generator().manual_seed(12)
    M, K, G = 19, 512, 128
    w = (torch.randn(M, K, generator=g) * 0.02).to(torch.bfloat16)
    w[1] = 0
    w[2, :128] = 0.5                                                   # a group of equal values
    w[4, 5] = -3.0
    packed, s = quantize_int4_groups(w)
    wg = w.view(M, K // G, G)
    amax = wg.abs().amax(dim=-1)                                       # bf16
    s_t = (amax / 7.0).to(torch.float32).clamp(min=1e-12)              # bf16 division, widened
    q_t = (wg.to(torch.float32) / s_t[..., None]).round().clamp(-8, 7).to(torch.int64).view(M, K)
    assert torch.equal(torch.from_numpy(s.numpy()), s_t)
    assert np.array_equal(unpack_int4(packed), q_t.numpy())


def test_int4_packing_known_answer():
    """Low nibble = even element, two's complement: [1, -1, 7, -8, 0, 3] -> 0xF1, 0x87, 0x30."""
    from oracle.formats import unpack_int4
    packed = torch.tensor([[0xF1, 0x87, 0x30]], dtype=torch.uint8)
    assert unpack_int4(packed).tolist() == [[1, -1, 7, -8, 0, 3]]
    from oracle.formats import quantize_int4_groups
    w = torch.zeros(1, 128, dtype=torch.bfloat16)
    w[0, :6] = torch.tensor([1.0, -1.0, 7.0, -7.0, 0.0, 3.0])
    p, s = quantize_int4_groups(w)
    assert s.tolist() == [[1.0]]
    assert p[0, :3].tolist() == [0xF1, 0x97, 0x30]                     # -7 -> 0x9
