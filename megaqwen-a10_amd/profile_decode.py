"""Decode driver for profiler runs (``rocprofv3 --kernel-trace`` / ``--pmc``).

Builds the config-1 model (Qwen3-0.6B shape, random-init seed 0, per-row INT8),
prefills the 8-token prompt one decode_step per token and runs ``--steps``
greedy steps through ``A10Int8MegakernelDecoder.decode_step``. With
``--copy-mib N`` it first runs four uint8 adds over an N MiB buffer (each reads
and writes exactly N MiB), the calibration for FETCH_SIZE / WRITE_SIZE. With
``--generate`` it then runs the same prompt and steps again as one launch
(``generate``: prefill and greedy steps handed on on the device).

    python megaqwen-a10_amd/profile_decode.py [--steps 32] [--variant auto|flat|xcd|async] [--copy-mib 256]
                                              [--generate]
"""
from __future__ import annotations

import argparse
import sys
from pathlib import Path

ROOT = Path(__file__).resolve().parents[1]
sys.path.insert(0, str(ROOT))


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--steps", type=int, default=32)
    ap.add_argument("--variant", default="auto", choices=["auto", "flat", "xcd", "async"])
    ap.add_argument("--copy-mib", type=int, default=0)
    ap.add_argument("--generate", action="store_true")
    args = ap.parse_args()

    import torch
    import __graft_entry__

    mq = __graft_entry__.load_package()
    dev = torch.device("cuda:0")
    if args.copy_mib:
        a = torch.zeros(args.copy_mib * 2 ** 20, dtype=torch.uint8, device=dev)
        b = torch.empty_like(a)
        for _ in range(4):
            torch.add(a, 1, out=b)
        torch.cuda.synchronize()
        del a, b
    cfg = mq.QWEN3_0_6B
    state, prompt = mq.random_init_state(cfg, seed=0)
    S = len(prompt) + args.steps + 8
    cos, sin = mq.precompute_rope_freqs(cfg.head_dim, S, cfg.rope_theta, device=dev)
    qstate = mq.quantize_state(state, cfg, dev)
    del state
    embed, layers, scales, lm_q, lm_s, fnorm = mq.pack_int8(qstate, cfg)
    dec = mq.A10Int8MegakernelDecoder(embed, layers, scales, lm_q, lm_s, fnorm, cos, sin, cfg.num_layers, S)
    mq.set_decode_variant(args.variant)
    tok = None
    for t in prompt.tolist():
        tok = dec.decode_step(int(t))
    for _ in range(args.steps):
        tok = dec.decode_step(tok)
    torch.cuda.synchronize()
    print(f"decoded {len(prompt) + args.steps} steps with the {mq.decode_variant()} kernel, last token {tok}",
          flush=True)
    if args.generate:
        dec.reset()
        toks = dec.generate(prompt.tolist(), args.steps + 1)
        torch.cuda.synchronize()
        print(f"generate: {len(prompt) + args.steps} steps, last token {toks[-1]} "
              f"({'same' if toks[-1] == tok else 'DIFFERENT'})", flush=True)
    # release device memory before interpreter shutdown (profilers finalise at exit)
    del dec, embed, layers, scales, lm_q, lm_s, fnorm, cos, sin, qstate
    torch.cuda.synchronize()
    torch.cuda.empty_cache()
    return 0


if __name__ == "__main__":
    # return normally on success: interpreter shutdown then runs the same way as
    # at the end of a plain script (the exit path profilers finalise on)
    status = main()
    if status:
        sys.exit(status)
