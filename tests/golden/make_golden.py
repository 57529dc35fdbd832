"""Regenerate the golden fixtures in this directory from the CPU oracle.

    python tests/golden/make_golden.py [--only NAME]

Fixtures (all small; weights are regenerated from their seed, never stored):

* quant_cases.npz    — bf16 weight matrices with edge cases (zero row, single
                       element, negative maxima, exact .5 ties, tiny values) and
                       their int8 codes and fp32 scales. The Python and C
                       quantizer restatements must agree on them before they
                       are written.
* rope_rows.npz      — bf16 bits of the theta=1e6 split-half cos/sin tables at
                       positions 0, 1, 7, 2047, 8191 and of the legacy
                       theta=1e4 pair-duplicated table at 0, 1, 7, 2047.
* tokens_<case>.json — prompt, 32 greedy tokens, per-step top-2 logit margins
                       and the sha256 of the generated weights, from the
                       float64 oracle, for each decode case in CASES (the
                       _fp8 case: FP8 E4M3 weights from oracle/formats.py,
                       decoded to their exact values for the oracle; the _int4
                       case: INT4-g128 layer projections dequantized exactly,
                       the LM head INT8 per row).
"""
from __future__ import annotations

import argparse
import ctypes
import json
import sys
import time
from pathlib import Path

import numpy as np
import torch

HERE = Path(__file__).resolve().parent
ROOT = HERE.parents[1]
sys.path.insert(0, str(ROOT))

import __graft_entry__  # noqa: E402
from oracle import formats as oformats  # noqa: E402
from oracle import quant as oquant  # noqa: E402
from oracle import rope as orope  # noqa: E402
from oracle.ref_cpu import Dims, RefDecoder, greedy_generate  # noqa: E402

mq = __graft_entry__.load_package()

# name -> (config overrides, seed, int8, norm_jitter, max_seq_len, tokens)
CASES = {
    "small_int8": (dict(num_layers=2, vocab_size=4096), 1, True, 0.1, 64, 32),
    "qwen3_0.6b_fp8": (dict(), 0, True, 0.0, 64, 32),
    "qwen3_0.6b_int4": (dict(), 0, True, 0.0, 64, 32),
    "qwen3_0.6b_int8": (dict(), 0, True, 0.0, 64, 32),
    "qwen3_0.6b_bf16": (dict(), 0, False, 0.0, 64, 32),
}


def quant_matrices(seed: int = 7):
    g = torch.Generator().manual_seed(seed)
    K = 64
    rows = []
    rows.append(torch.zeros(K))                                               # zero row -> scale floor
    r = torch.zeros(K); r[5] = -0.75; rows.append(r)                          # single negative element
    rows.append(torch.randn(K, generator=g) * 0.02)                           # typical
    rows.append(-torch.rand(K, generator=g) * 3.0)                            # all negative
    rows.append(torch.randn(K, generator=g) * 1e-30)                          # tiny magnitudes
    rows.append(torch.randn(K, generator=g) * 1e4)                            # large magnitudes
    r = torch.randn(K, generator=g) * 0.02; r[0] = 1.0; rows.append(r)        # one outlier
    w = torch.stack(rows).to(torch.bfloat16)
    # rows engineered so that several w/scale land exactly on .5 (ties to even)
    tie_rows = []
    for e in (-7, -5, -9):
        # amax = 127 * 2^e makes the scale exactly 2^e, so every c * 2^e below is exact in bf16
        q = torch.tensor([127.0, 0.5, 1.5, 2.5, -0.5, -1.5, 126.5, -127.0] * (K // 8))
        tie_rows.append((q * 2.0 ** e).to(torch.bfloat16))
    w = torch.cat([w, torch.stack(tie_rows), (torch.randn(16, K, generator=g) * 0.02).to(torch.bfloat16)])
    return w


def c_quantize(w: torch.Tensor):
    lib = ctypes.CDLL(str(ROOT / "oracle" / "lib" / "liboracle.so"))
    M, K = w.shape
    bits = w.contiguous().view(torch.int16).numpy().view(np.uint16).copy()
    q = np.empty((M, K), np.int8)
    s = np.empty(M, np.float32)
    lib.oracle_quantize_bf16(bits.ctypes.data_as(ctypes.c_void_p), ctypes.c_int64(M), ctypes.c_int64(K),
                             q.ctypes.data_as(ctypes.c_void_p), s.ctypes.data_as(ctypes.c_void_p))
    return q, s


def make_quant():
    w = quant_matrices()
    q, s = oquant.quantize_per_channel(w)
    qc, sc = c_quantize(w)
    assert np.array_equal(q.numpy(), qc) and np.array_equal(s.numpy(), sc), "quantizer restatements disagree"
    np.savez_compressed(HERE / "quant_cases.npz", w_bits=w.view(torch.int16).numpy().view(np.uint16),
                        q=q.numpy(), scale=s.numpy())


def make_rope():
    c, s = orope.split_half_tables(8192, 128, 1e6)
    pos = np.array([0, 1, 7, 2047, 8191])
    lc, ls = orope.pair_duplicated_tables(2048, 128, 1e4)
    lpos = np.array([0, 1, 7, 2047])
    bits = lambda t: t.view(torch.int16).numpy().view(np.uint16)
    np.savez_compressed(HERE / "rope_rows.npz", pos=pos, cos=bits(c[pos]), sin=bits(s[pos]), legacy_pos=lpos,
                        legacy_cos=bits(lc[lpos]), legacy_sin=bits(ls[lpos]))


# one-byte weight format of a case whose int8 flag is set (default int8)
FORMAT = {"qwen3_0.6b_fp8": "fp8", "qwen3_0.6b_int4": "int4"}


def _quantize(w: torch.Tensor, fmt: str):
    """(weights as the oracle multiplies them, fp32 row scales)."""
    if fmt == "fp8":
        q, s = oformats.quantize_fp8_rows(w)
        return torch.from_numpy(oformats.fp8_decode_table()[q.numpy().astype(np.int64)]), s
    if fmt == "int4":
        # the dequantized values (nibble x group scale, exact in fp64), row scales of 1
        q, s = oformats.quantize_int4_groups(w)
        return torch.from_numpy(oformats.dequant_int4(q, s)), torch.ones(w.shape[0], dtype=torch.float32)
    return oquant.quantize_per_channel(w)


def oracle_for(name: str, dtype=torch.float64):
    """Builds (RefDecoder, prompt, cfg, digest) for a fixture case on the CPU (quantizing with the oracle)."""
    over, seed, int8, jitter, S, _ = CASES[name]
    fmt = FORMAT.get(name, "int8")
    cfg = mq.QWEN3_0_6B.with_(name=name, **over)
    state, prompt = mq.random_init_state(cfg, seed=seed, norm_jitter=jitter)
    digest = mq.state_digest(state)
    cos, sin = orope.split_half_tables(S, cfg.head_dim, cfg.rope_theta)
    dims = Dims(hidden_size=cfg.hidden_size, intermediate_size=cfg.intermediate_size, vocab_size=cfg.vocab_size)
    layers, scales = [], []
    for i in range(cfg.num_layers):
        p = f"model.layers.{i}"

        def proj(n):
            w = state[f"{p}.{n}.weight"]
            if not int8:
                return w
            qq, ss = _quantize(w, fmt)
            scales.append(ss)
            return qq
        layers.append(state[f"{p}.input_layernorm.weight"])
        layers += [proj("self_attn.q_proj"), proj("self_attn.k_proj"), proj("self_attn.v_proj")]
        layers += [state[f"{p}.self_attn.q_norm.weight"], state[f"{p}.self_attn.k_norm.weight"]]
        layers.append(proj("self_attn.o_proj"))
        layers.append(state[f"{p}.post_attention_layernorm.weight"])
        layers += [proj("mlp.gate_proj"), proj("mlp.up_proj"), proj("mlp.down_proj")]
    if int8:
        # INT4 models keep the LM head INT8 per row
        lm, lms = _quantize(state["lm_head.weight"], "int8" if fmt == "int4" else fmt)
    else:
        lm, lms = state["lm_head.weight"], None
    dec = RefDecoder(dims, state["model.embed_tokens.weight"], layers, scales if int8 else None,
                     state["model.norm.weight"], lm, lms, cos, sin, cfg.num_layers, S, dtype=dtype)
    return dec, prompt, cfg, digest


def make_tokens(name: str):
    t0 = time.time()
    dec, prompt, cfg, digest = oracle_for(name)
    n = CASES[name][5]
    toks, margins = greedy_generate(dec, prompt.tolist(), n)
    rec = {"case": name, "config": cfg.__dict__, "seed": CASES[name][1], "int8": CASES[name][2],
           "weight_format": FORMAT.get(name, "int8") if CASES[name][2] else "bf16",
           "norm_jitter": CASES[name][3], "max_seq_len": CASES[name][4], "prompt": prompt.tolist(),
           "tokens": toks, "top2_margins": margins, "weights_sha256": digest,
           "oracle": "oracle.ref_cpu.RefDecoder float64, rounding points of a10_int8_decode_kernel.cu"}
    (HERE / f"tokens_{name}.json").write_text(json.dumps(rec, indent=1) + "\n")
    print(f"{name}: {toks[:8]}... min margin {min(margins):.4g} ({time.time() - t0:.1f}s)")


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--only", default=None)
    args = ap.parse_args()
    torch.set_num_threads(max(1, torch.get_num_threads()))
    if args.only in (None, "quant"):
        make_quant()
    if args.only in (None, "rope"):
        make_rope()
    for name in CASES:
        if args.only in (None, name):
            make_tokens(name)


if __name__ == "__main__":
    main()
