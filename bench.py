"""Benchmark: INT8 batch-1 greedy decode of the Qwen3-0.6B shape on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu] [--workload NAME]

Default workload: random-init Qwen3-0.6B-architecture
weights (seed 0, N(0, 0.02) -> bf16 -> per-row INT8), an 8-token random prompt
prefilled one decode_step per token (untimed), then K greedy decode steps
timed through the drop-in API (``A10Int8MegakernelDecoder.decode_step``: one
kernel launch and one token read-back per step, as bench_int8.py:355-362).
``value`` = K / wall time of those K steps, inputs already resident in HBM.

The JSON line also carries:
* ``roofline`` — algorithmic bytes per decode launch (all weights once + the
  KV rows read and written) over the kernel's average duration, measured with
  HIP events on the launch stream inside the timed region, against 8 TB/s;
* ``cpu_baseline`` — the float32 CPU port of the same decode (oracle.ref_cpu,
  ``(q.float() @ x) * scale``) timed on this host for the 32-token workload;
* ``parity`` — the timed tokens against the committed oracle fixture.

Other workloads (parity-case shapes, one JSON line each): ``matvec``
``formats`` (the config-2 shapes in INT8, INT4 per group and
FP8 E4M3, steady state), ``positions`` (config 3 positions, bf16 weights),
``longctx`` (config 4: KV pre-filled to 1024 / 4096 / 8192, ``--steps 64``),
``batched`` (config 5: Qwen3-1.7B shape, B = 1 / 4 / 8 / 16, ``--steps 128``; one
sequence per batch size teacher-force checked against the float64 oracle for
``--check-steps`` tokens, reported as ``per_batch[B].parity``), ``prefill`` (the
prompt-batched prefill of 8 / 64 / 512 / 2040 tokens against one decode step per
token, ``--prompt-lens``), and
``traffic``: a uint8 add over a 256 MiB buffer (reads and writes exactly
256 MiB, the calibration for the FETCH_SIZE / WRITE_SIZE counters) followed
by 8 decode steps, for ``rocprofv3 --pmc`` runs.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

HBM_PEAK_GBS = 8000.0
INT8_PEAK_TOPS = 5000.0          # dense int8 MFMA, MI355X
PROMPT_LEN = 8
# Memory traffic per decode launch of each kernel, measured with rocprofv3 --pmc FETCH_SIZE and
# WRITE_SIZE runs of megaqwen-a10_amd/profile_decode.py, each scaled by the counter's reading for a
# 256 MiB copy (the commands and numbers are in profiles/decode_*_kernel_int8_qwen3-0.6b_traffic.txt).
MEASURED_TRAFFIC = {"mq::decode_async_kernel<false, false, false>": 641_659_290,
                    "mq::decode_xcd_kernel<1024, 3072, mq::Int8W, false>": 639_234_240}


def parse():
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=None,
                    help="timed steps (default: 32; the BASELINE counts for longctx, 64, and batched, 128)")
    ap.add_argument("--warmup", type=int, default=8)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--cpu-steps", type=int, default=112,
                    help="greedy steps of the CPU baseline sample (about 10 s on 16 host threads)")
    ap.add_argument("--workload", default="decode",
                    choices=["decode", "matvec", "formats", "positions", "longctx", "batched", "prefill", "traffic"])
    ap.add_argument("--prompt-lens", default="8,64,512,2040", help="prefill: prompt lengths")
    ap.add_argument("--weight-format", default="int8", choices=["int8", "int4"],
                    help="decode: INT8 per row (config 1), or INT4 per group of 128 with the LM head INT8")
    ap.add_argument("--depths", default="1024,4096,8192", help="longctx: KV depths")
    ap.add_argument("--batches", default="1,4,8,16", help="batched: batch sizes")
    ap.add_argument("--variant", default="auto", choices=["auto", "xcd", "async"],
                    help="longctx: decode kernel (auto: the library's choice per step)")
    ap.add_argument("--split-min", type=int, default=0,
                    help="longctx: attention split threshold (0 = library default, -1 = never)")
    ap.add_argument("--seed", type=int, default=0)
    ap.add_argument("--check-steps", type=int, default=8,
                    help="batched: generated tokens of one sequence per batch size teacher-force checked "
                         "against the float64 CPU oracle (0 = no check)")
    ap.add_argument("--no-kernel-events", action="store_true",
                    help="do not attach timing events to the decode launches (for runs under rocprofv3 "
                         "--kernel-trace, which supplies the kernel durations itself); roofline.achieved then "
                         "uses the wall time per step")
    args = ap.parse_args()
    if args.steps is None:
        args.steps = {"longctx": 64, "batched": 128}.get(args.workload, 32)
    return args


def cpu_baseline(keep, cfg, prompt, steps):
    """Time the fp32 CPU port of the reference decode on this host (bounded sample)."""
    import torch
    from oracle.ref_cpu import Dims, RefDecoder

    embed, layers, scales, lm_q, lm_s, fnorm, cos, sin = keep
    c = lambda t: t.cpu()
    threads = torch.get_num_threads()
    ref = RefDecoder(Dims(), c(embed), [c(t) for t in layers], [c(t) for t in scales], c(fnorm), c(lm_q), c(lm_s),
                     c(cos), c(sin), cfg.num_layers, cos.shape[0], dtype=torch.float32)
    ref.reset()
    tok = None
    for t in prompt:
        tok = ref.decode_step(int(t))
    t0 = time.perf_counter()
    toks = []
    for _ in range(steps):
        tok = ref.decode_step(tok)
        toks.append(tok)
    dt = time.perf_counter() - t0
    del ref
    return {"value": round(steps / dt, 3), "unit": "tok/s", "cores": threads, "kind": "port",
            "sample": f"{steps} greedy decode steps after the {PROMPT_LEN}-token prefill, Qwen3-0.6B shape "
                      f"INT8 weights, fp32 torch CPU port (oracle.ref_cpu, (q.float() @ x) * scale), "
                      f"{threads} torch threads on {os.cpu_count()} host CPUs",
            "seconds": round(dt, 3), "tokens": toks}


def _events(torch, n):
    """n start/end pairs of timing events, created before any timed region."""
    ev = ([torch.cuda.Event(enable_timing=True) for _ in range(n)],
          [torch.cuda.Event(enable_timing=True) for _ in range(n)])
    for e in ev[0] + ev[1]:
        e.record()
    torch.cuda.synchronize()
    return ev


def _timed_pass(torch, dec, first, steps, wait, events=None, step=None):
    """`steps` greedy steps from `first` through launch_step + wait (or `step`, e.g. the
    decoder's decode_step): (tokens, wall s, kernel ms).

    With `events` every dispatch records its own start/end pair (hipExtLaunchKernel on the
    launch stream), which costs about 20 us of host time per launch. So the pass that sets
    a workload's tok/s runs without them, and a second pass over the same steps (same
    positions, same tokens) measures the kernel."""
    toks, tok = [], first
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for i in range(steps):
        if events is not None:
            dec.set_timing_events(events[0][i], events[1][i])
        if step is not None:
            tok = step(tok)
        else:
            dec.launch_step(tok)
            tok = wait()
        toks.append(tok)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    kern_ms = None
    if events is not None:
        dec.set_timing_events(None, None)
        kern_ms = [a.elapsed_time(b) for a, b in zip(*events)]
    return toks, wall, kern_ms


KERNEL_TIMING = ("a second pass over the same steps (same positions and tokens), each dispatch recording "
                 "its own start/end HIP events (hipExtLaunchKernel, launch stream); the pass that sets tok/s "
                 "runs without them, since they add about 20 us of host time per launch")


def run_decode(args, mq, torch):
    dev = torch.device("cuda:0")
    cfg = mq.QWEN3_0_6B
    state, prompt = mq.random_init_state(cfg, seed=args.seed)
    S = PROMPT_LEN + max(args.steps, args.warmup, 0 if args.no_cpu else args.cpu_steps) + 8
    cos, sin = mq.precompute_rope_freqs(cfg.head_dim, S, cfg.rope_theta, device=dev)
    w4 = args.weight_format == "int4"
    qstate = mq.quantize_state(state, cfg, dev, weight_format=args.weight_format)
    del state
    embed, layers, scales, lm_q, lm_s, fnorm = mq.pack_int8(qstate, cfg)
    keep = (embed, layers, scales, lm_q, lm_s, fnorm, cos, sin)
    cls = mq.A10Int4MegakernelDecoder if w4 else mq.A10Int8MegakernelDecoder
    dec = cls(embed, layers, scales, lm_q, lm_s, fnorm, cos, sin, cfg.num_layers, S)
    prompt = prompt.tolist()

    def prefill():
        dec.reset()
        tok = None
        for t in prompt:
            tok = dec.decode_step(int(t))
        return tok

    tok = prefill()
    for _ in range(args.warmup):
        tok = dec.decode_step(tok)
    events = None if args.no_kernel_events else _events(torch, args.steps)

    # timed region: K greedy steps through the drop-in API (decode_step, as bench_int8.py:217-218)
    first = prefill()
    toks, wall, _ = _timed_pass(torch, dec, first, args.steps, None, step=dec.decode_step)
    repeat_identical = None
    if args.no_kernel_events:
        kern_ms = [wall * 1e3 / args.steps] * args.steps
    else:
        first2 = prefill()
        toks2, _, kern_ms = _timed_pass(torch, dec, first2, args.steps, dec.wait_token, events)
        repeat_identical = first2 == first and toks2 == toks
    if min(toks) < 0:
        status = dec._lib.mq_decode_check(dec.workspace.data_ptr(), None)
        raise RuntimeError(f"decode step {toks.index(min(toks))} of the timed region failed: "
                           f"status {status}: {mq._lib.last_error()}")
    variant = "async" if w4 else mq.decode_variant(cfg.hidden_size, cfg.intermediate_size, int8=True)
    kernel = {"async": f"mq::decode_async_kernel<false, false, {'true' if w4 else 'false'}>",
              "xcd": "mq::decode_xcd_kernel<1024, 3072, mq::Int8W, false>",
              "flat": "mq::decode_kernel<1024, 3072, mq::Int8W, false>"}[variant]
    arithmetic = ("matrix products as exact sums of int8 digits of a 55-bit fixed-point activation on the int8 "
                  "matrix cores, recombined in fp64; other layer stages fp64; values rounded to fp32/bf16 where "
                  "the reference stores them; LM head fp32") if variant == "async" else (
                  "layer stages fp64 (rounded to fp32/bf16 where the reference stores), LM head fp32")

    # algorithmic bytes of each timed launch: positions PROMPT_LEN .. PROMPT_LEN+K-1
    step_bytes = cfg.int4_step_bytes if w4 else cfg.int8_step_bytes
    bytes_total = sum(step_bytes(cache_len=PROMPT_LEN + i + 1) for i in range(args.steps))
    kern_s = sum(kern_ms) / 1e3
    achieved = bytes_total / kern_s / 1e9

    device_loop = None
    if variant == "async":
        # the same K steps as ONE launch (mq_int8_decode_generate): each step's token goes to
        # the next on the device, so no host round trip per token; wall time of the call.
        # None from the one-launch path: the steps reach past the kernel's position range.
        first3 = prefill()
        warm = dec._generate_one_launch([first3], 1)
        if warm is not None:
            prefill()
            torch.cuda.synchronize()
            t0 = time.perf_counter()
            toks3 = dec._generate_one_launch([first3], args.steps)
            wall3 = time.perf_counter() - t0
            if toks3 is not None:
                device_loop = {"tok_s": round(args.steps / wall3, 1),
                               "ms_per_step": round(wall3 / args.steps * 1e3, 4),
                               "entry_point": f"mq_{args.weight_format}_decode_generate: one launch for all K steps",
                               "tokens_match_per_step_launches": first3 == first and toks3 == toks}

    parity = None
    fx = ROOT / "tests" / "golden" / f"tokens_qwen3_0.6b_{args.weight_format}.json"
    if fx.exists() and args.seed == 0:
        want = json.loads(fx.read_text())["tokens"]
        n = min(len(want) - 1, args.steps)
        parity = {"fixture": fx.name, "checked": n + 1,
                  "match": [first] + toks[:n] == want[:n + 1]}

    value = args.steps / wall
    out = {
        "metric": ("INT4-g128 decode tok/s (LM head INT8), Qwen3-0.6B shape bs=1; achieved HBM GB/s vs peak" if w4
                   else "INT8 decode tok/s, Qwen3-0.6B shape bs=1; achieved HBM GB/s vs peak"),
        "value": round(value, 2),
        "unit": "tok/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(wall / args.steps * 1e3, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f64",
        "data": "synthetic",
        "config": {"workload": "config 1: INT8 greedy decode, Qwen3-0.6B architecture random-init (seed 0), "
                               "bs=1, 8-token random prompt prefilled untimed, K greedy steps timed",
                   "weights": ("int4 per group of 128 (scale=bf16(absmax/7)), LM head int8 per row; "
                               "embed/norms/RoPE/KV bf16") if w4 else
                              "int8 per-output-channel (scale=bf16(absmax/127)); embed/norms/RoPE/KV bf16",
                   "arithmetic": arithmetic, "kernel_variant": variant,
                   "layers": cfg.num_layers, "hidden": cfg.hidden_size, "vocab": cfg.vocab_size,
                   "batch": 1, "prompt_len": PROMPT_LEN, "parallelism": "single GPU"},
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": MEASURED_TRAFFIC.get(kernel),
                     "kernel": kernel,
                     "kernel_avg_us": round(sum(kern_ms) / len(kern_ms) * 1e3, 2),
                     "timing": "wall per step" if args.no_kernel_events else KERNEL_TIMING,
                     "kernel_pass_tokens_identical": repeat_identical,
                     "bytes_per_launch_avg": int(bytes_total / args.steps)},
        "device_tok_s": round(args.steps / kern_s, 1),
        "device_loop": device_loop,
        "parity": parity,
    }
    if w4:
        out["config"]["workload"] = out["config"]["workload"].replace("config 1: INT8", "INT4-g128")
    if not args.no_cpu and not w4:
        cb = cpu_baseline(keep, cfg, prompt, args.cpu_steps)
        cpu_toks = cb.pop("tokens")
        gpu_ref = [first] + toks
        n = min(len(cpu_toks), len(gpu_ref) - 1)
        cb["tokens_match_gpu"] = cpu_toks[:n] == gpu_ref[1:n + 1]
        if not cb["tokens_match_gpu"]:
            i = next(j for j in range(n) if cpu_toks[j] != gpu_ref[1 + j])
            cb["first_divergent_step"] = i + 1
            cb["note"] = ("the fp32 CPU port diverges from the GPU/float64-oracle tokens where the top-2 "
                          "logit margin is small; the GPU tokens are checked against the float64 oracle")
        out["cpu_baseline"] = cb
        out["speedup_vs_cpu"] = round(value / cb["value"], 1)
    return out


def run_matvec(args, mq, torch):
    """per-shape INT8 matvec GB/s, rotating weight copies past the 256 MB MALL."""
    dev = torch.device("cuda:0")
    shapes = {"qkv": (4096, 1024), "o": (1024, 2048), "gate_up": (6144, 1024), "down": (1024, 3072),
              "lm_head": (151936, 1024)}
    res = {}
    g = torch.Generator().manual_seed(args.seed)
    for name, (M, K) in shapes.items():
        w = (torch.randn(M, K, generator=g) * 0.02).to(torch.bfloat16).to(dev)
        q, s = mq.quantize_per_channel(w)
        del w
        nbytes = M * K + 8 * M + 4 * K
        copies = max(1, -(-512 * 2 ** 20 // (M * K)))
        wcopies = q.unsqueeze(0).expand(copies, M, K).contiguous()     # one contiguous [copies, M, K]
        qs = [wcopies[i] for i in range(copies)]
        x = torch.randn(K, generator=g).to(dev)
        y = torch.empty(M, device=dev)
        for i in range(20):
            mq.int8_gemv(x, qs[i % copies], s, out=y)
        reps = 1000
        ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        ev0.record()
        for i in range(reps):
            mq.int8_gemv(x, qs[i % copies], s, out=y)
        ev1.record()
        torch.cuda.synchronize()
        us = ev0.elapsed_time(ev1) / reps * 1e3
        # the same launches captured once in a HIP graph and replayed: no host cost per launch,
        # so small shapes show the kernel rather than the Python/ctypes launch rate
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            for i in range(reps):
                mq.int8_gemv(x, qs[i % copies], s, out=y)
        want = mq.int8_gemv(x, qs[(reps - 1) % copies], s)
        graph_ok = True
        for _ in range(2):                       # replays checked against the eager result
            graph.replay()
            torch.cuda.synchronize()
            graph_ok = graph_ok and torch.equal(y, want)
        torch.cuda.synchronize()
        ev0.record()
        graph.replay()
        ev1.record()
        torch.cuda.synchronize()
        graph_ok = graph_ok and torch.equal(y, want)
        us_g = ev0.elapsed_time(ev1) / reps * 1e3
        del graph
        # steady state: one launch streams n_rep matvecs over the rotating copies (about 2 GB)
        n_rep = max(copies, -(-2 * 2 ** 30 // (M * K)))
        ys = torch.empty((copies, M), device=dev)
        mq.int8_gemv_repeat(x, wcopies, s, n_rep, out=ys)
        torch.cuda.synchronize()
        steady_ok = torch.equal(ys[(reps - 1) % copies], want) or bool(
            torch.allclose(ys[(reps - 1) % copies], want, rtol=1e-5, atol=1e-6))
        ev0.record()
        mq.int8_gemv_repeat(x, wcopies, s, n_rep, out=ys)
        ev1.record()
        torch.cuda.synchronize()
        us_s = ev0.elapsed_time(ev1) / n_rep * 1e3
        res[name] = {"shape": [M, K], "us": round(us_g, 3), "GBs": round(nbytes / us_g / 1e3, 1),
                     "frac": round(nbytes / us_g / 1e3 / HBM_PEAK_GBS, 4), "graph_replay_matches_eager": graph_ok,
                     "steady_us": round(us_s, 4), "steady_GBs": round(nbytes / us_s / 1e3, 1),
                     "steady_frac": round(nbytes / us_s / 1e3 / HBM_PEAK_GBS, 4), "steady_reps": n_rep,
                     "steady_matches_single_call": steady_ok,
                     "eager_us": round(us, 3), "eager_GBs": round(nbytes / us / 1e3, 1), "copies": copies}
        print(f"{name}: {res[name]}", file=sys.stderr, flush=True)
        del qs, q, s, wcopies, ys
        torch.cuda.empty_cache()
    lm = res["lm_head"]
    return {"metric": "INT8 matvec GB/s (BASELINE config 2)", "value": lm["GBs"], "unit": "GB/s", "n_gpus": 1,
            "steps": 1000, "warmup": 20, "ms_per_step": round(lm["us"] / 1e3, 5), "higher_is_better": True,
            "scaling": "weak", "vs_baseline": None, "dtype": "fp32", "data": "synthetic",
            "config": {"workload": "config 2: isolated INT8 matvec, 1000 launches per shape replayed from a HIP "
                                   "graph (eager_* fields: the same 1000 launches from Python; steady_* fields: one "
                                   "launch of mq_int8_gemv_repeat streaming about 2 GB of matvecs, time / reps), "
                                   "weight copies rotated to exceed the 256 MB MALL", "shapes": res,
                       "steady_frac_min_small_shapes": min(res[k]["steady_frac"] for k in ("qkv", "o", "gate_up", "down"))}}


def run_formats(args, mq, torch):
    """Other weight formats: INT8 per row, INT4 per group of 128, FP8 E4M3 per row, at the config-2
    shapes: steady-state time per matvec (one launch over rotating copies past the 256 MB MALL),
    bytes read, and each format's error against the bf16 weights' product."""
    dev = torch.device("cuda:0")
    shapes = {"qkv": (4096, 1024), "o": (1024, 2048), "gate_up": (6144, 1024), "down": (1024, 3072),
              "lm_head": (151936, 1024)}
    g = torch.Generator().manual_seed(args.seed)
    res = {}
    ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    for name, (M, K) in shapes.items():
        w = (torch.randn(M, K, generator=g) * 0.02).to(torch.bfloat16).to(dev)
        x = torch.randn(K, generator=g).to(dev)
        exact = (w.double() @ x.double())
        per = {}
        for fmt in ("int8", "int4", "fp8"):
            if fmt == "int8":
                q, s = mq.quantize_per_channel(w)
                rep = lambda xc, wc, n: mq.int8_gemv_repeat(xc, wc, s, n)
            elif fmt == "int4":
                q, s = mq.quantize_int4(w)
                rep = lambda xc, wc, n: mq.int4_gemv_repeat(xc, wc, s, n)
            else:
                q, s = mq.quantize_fp8(w)
                rep = lambda xc, wc, n: mq.fp8_gemv_repeat(xc, wc, s, n)
            wbytes = q.numel() * q.element_size()
            nbytes = wbytes + s.numel() * 4 + 4 * K + 4 * M
            copies = max(1, -(-512 * 2 ** 20 // wbytes))
            wc = q.unsqueeze(0).expand(copies, *q.shape).contiguous()
            n_rep = max(copies, -(-2 * 2 ** 30 // wbytes))
            y = rep(x, wc, n_rep)
            torch.cuda.synchronize()
            err = float(torch.linalg.norm(y[0].double() - exact) / torch.linalg.norm(exact))
            ev0.record()
            rep(x, wc, n_rep)
            ev1.record()
            torch.cuda.synchronize()
            us = ev0.elapsed_time(ev1) / n_rep * 1e3
            per[fmt] = {"us": round(us, 4), "bytes": nbytes, "GBs": round(nbytes / us / 1e3, 1),
                        "frac": round(nbytes / us / 1e3 / HBM_PEAK_GBS, 4), "rel_err_vs_bf16": float(f"{err:.3e}"),
                        "reps": n_rep, "copies": copies}
            del wc, q, s, y
            torch.cuda.empty_cache()
        res[name] = per
        print(f"{name}: {per}", file=sys.stderr, flush=True)
        del w
    L = mq.QWEN3_0_6B.num_layers
    step = {f: round(L * sum(res[k][f]["us"] for k in ("qkv", "o", "gate_up", "down")) + res["lm_head"][f]["us"], 2)
            for f in ("int8", "int4", "fp8")}

    # the whole config-1 decode step with FP8 weights, beside INT8 on the same (XCD-aware) kernel
    cfg = mq.QWEN3_0_6B
    state, prompt = mq.random_init_state(cfg, seed=args.seed)
    S = PROMPT_LEN + args.steps + 8
    cos, sin = mq.precompute_rope_freqs(cfg.head_dim, S, cfg.rope_theta, device=dev)
    decode = {}
    events = _events(torch, args.steps)
    for fmt in ("int8", "fp8"):
        qstate = mq.quantize_state(state, cfg, dev, weight_format=fmt)
        packed = mq.pack_int8(qstate, cfg)
        del qstate
        cls = mq.A10Fp8MegakernelDecoder if fmt == "fp8" else mq.A10Int8MegakernelDecoder
        dec = cls(*packed, cos, sin, cfg.num_layers, S)
        mq.set_decode_variant("xcd")
        try:
            def prefill():
                dec.reset()
                tok = None
                for t in prompt.tolist():
                    tok = dec.decode_step(int(t))
                return tok
            first = prefill()
            toks, wall, _ = _timed_pass(torch, dec, first, args.steps, dec.wait_token)
            first2 = prefill()
            toks2, _, kern_ms = _timed_pass(torch, dec, first2, args.steps, dec.wait_token, events)
        finally:
            mq.set_decode_variant("auto")
        decode[fmt] = {"tok_s": round(args.steps / wall, 1), "kernel_avg_us": round(sum(kern_ms) / args.steps * 1e3, 2),
                       "kernel_pass_tokens_identical": toks2 == toks and first2 == first}
        if fmt == "fp8":
            fx = ROOT / "tests" / "golden" / "tokens_qwen3_0.6b_fp8.json"
            if fx.exists() and args.seed == 0:
                want = json.loads(fx.read_text())["tokens"]
                n = min(len(want) - 1, args.steps)
                decode[fmt]["fixture_match"] = [first] + toks[:n] == want[:n + 1]
        print(f"decode {fmt}: {decode[fmt]}", file=sys.stderr, flush=True)
        del dec, packed
        torch.cuda.empty_cache()
    return {"metric": "matvec-only decode step time at the Qwen3-0.6B shapes, INT4 per-group weights "
                      "(steady state; INT8 and FP8 E4M3 beside it)",
            "value": step["int4"], "unit": "us", "n_gpus": 1, "steps": 1, "warmup": 1,
            "ms_per_step": round(step["int4"] / 1e3, 5), "higher_is_better": False, "scaling": "weak",
            "vs_baseline": None, "dtype": "int4 / fp8 / int8 weights, fp32 activations; fp32 sums (int8, fp8), exact products and fp64 sums (int4)", "data": "synthetic",
            "config": {"workload": "other weight formats: N(0, 0.02) bf16 weights per config-2 shape quantized to INT8 "
                                   "per row, INT4 per group of 128, FP8 E4M3 per row; one launch of the format's "
                                   "steady-state matvec over rotating copies (about 2 GB), time / reps; error = rel. "
                                   "L2 of the format's product against the bf16 weights' float64 product",
                       "step_us_28_layers_plus_lm_head": step, "shapes": res,
                       "decode_config1_xcd_kernel": decode}}


def run_positions(args, mq, torch):
    """bf16 weights, tok/s at positions 1, 25, 50, 100, 200.

    Three rates per position n: greedy decoding after the 8-token seed-0 prompt (prefilled
    untimed), n / wall of the first n greedy steps (BASELINE's definition; best of 3); the
    reference's own definition n / wall(reset + n steps of token 0) (bench_and_plot_int8.py:78-85,
    best of 3); and the marginal rate of 8 steps starting at that position (wall with one token
    read-back per step, and each step's kernel time from HIP events). The greedy run's first 32
    tokens are compared with the bf16 float64-oracle fixture."""
    dev = torch.device("cuda:0")
    cfg = mq.QWEN3_0_6B
    state, prompt = mq.random_init_state(cfg, seed=args.seed)
    prompt = prompt.tolist()
    positions = (1, 25, 50, 100, 200)
    marg = 8
    S = PROMPT_LEN + max(positions) + marg + 8
    cos, sin = mq.precompute_rope_freqs(cfg.head_dim, S, cfg.rope_theta, device=dev)
    embed, layers, fnorm, lm = mq.pack_bf16(state, cfg, dev)
    del state
    dec = mq.A10MegakernelDecoder(embed, layers, fnorm, lm, cos, sin, cfg.num_layers, S)
    for _ in range(5):
        dec.decode_step(0)
    # greedy decoding after the prompt: cumulative wall time at each of the positions
    greedy, tokens = {}, None
    for _ in range(3):
        dec.reset()
        tok = None
        for t in prompt:
            tok = dec.decode_step(int(t))
        got, stamps = [tok], {}
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for n in range(1, max(positions) + 1):
            tok = dec.decode_step(tok)
            got.append(tok)
            if n in positions:
                stamps[n] = time.perf_counter() - t0
        for n, dt in stamps.items():
            greedy[str(n)] = max(greedy.get(str(n), 0.0), round(n / dt, 1))
        tokens = got
    res = {}
    for n in positions:
        best = None
        for _ in range(3):
            torch.cuda.synchronize()
            t0 = time.perf_counter()
            dec.reset()
            for _ in range(n):
                dec.decode_step(0)
            torch.cuda.synchronize()
            dt = time.perf_counter() - t0
            best = dt if best is None else min(best, dt)
        res[str(n)] = round(n / best, 1)
    # marginal rate: steps at positions p .. p + 7 (cache_len p + 1 ..), token 0 as above
    events = _events(torch, marg)
    marginal = {}
    for p0 in positions:
        dec.reset()
        for _ in range(p0):
            dec.decode_step(0)
        pos_state = dec.position()
        _, wall, _ = _timed_pass(torch, dec, 0, marg, dec.wait_token)
        dec.reset()
        for _ in range(p0):
            dec.decode_step(0)
        _, _, kern_ms = _timed_pass(torch, dec, 0, marg, dec.wait_token, events)
        kern_s = sum(kern_ms) / 1e3
        nbytes = sum(cfg.bf16_step_bytes(cache_len=pos_state + i + 1) for i in range(marg))
        marginal[str(p0)] = {"tok_s": round(marg / wall, 1), "kernel_avg_us": round(kern_s / marg * 1e6, 2),
                             "hbm_frac": round(nbytes / kern_s / 1e9 / HBM_PEAK_GBS, 4)}
    # the same greedy decoding as ONE launch (the XCD-aware kernel's multi-step form): the
    # prompt and 200 generated steps, wall time of the call
    dev_loop = {}
    for _ in range(3):
        dec.reset()
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        got1 = dec.generate(prompt, max(positions) + 1, device_loop=True, batched_prefill=False)
        dt = time.perf_counter() - t0
        steps1 = len(prompt) + max(positions)
        if not dev_loop or steps1 / dt > dev_loop["tok_s"]:
            dev_loop = {"tok_s": round(steps1 / dt, 1), "ms_per_step": round(dt * 1e3 / steps1, 4),
                        "steps": steps1, "tokens_match_per_step_launches": got1 == tokens,
                        "entry_point": "mq_bf16_decode_generate: one launch for the prompt and all generated steps"}
    parity = None
    fx = ROOT / "tests" / "golden" / "tokens_qwen3_0.6b_bf16.json"
    if fx.exists() and args.seed == 0:
        want = json.loads(fx.read_text())["tokens"]
        parity = {"fixture": fx.name, "checked": len(want), "match": tokens[:len(want)] == want}
    return {"metric": "BF16 decode tok/s at positions (BASELINE config 3)", "value": greedy["200"], "unit": "tok/s",
            "n_gpus": 1, "steps": 200, "warmup": 5, "ms_per_step": round(1e3 / greedy["200"], 4),
            "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "f64", "data": "synthetic",
            "config": {"workload": "config 3: bf16 weights, greedy decoding after the 8-token seed-0 prompt, "
                                   "n / wall of the first n greedy steps (value: n = 200)",
                       "kernel": "mq::decode_xcd_kernel<1024, 3072, mq::Bf16W, false>",
                       "tok_s_greedy_after_prompt": greedy,
                       "tok_s_at_position": res,
                       "reference_definition": "n / wall(reset + n decode_step(0)) (bench_and_plot_int8.py:78-85)",
                       "marginal_at_position": marginal,
                       "marginal_method": f"{marg} steps from the position; tok/s from wall with one read-back per step; "
                                          + KERNEL_TIMING},
            "device_loop": dev_loop,
            "parity": parity}


def run_longctx(args, mq, torch):
    """INT8 Qwen3-0.6B shape with the KV cache pre-filled by seeded N(0,1) bf16
    rows to each depth, then 64 timed greedy steps per depth (kernel time from HIP events)."""
    dev = torch.device("cuda:0")
    cfg = mq.QWEN3_0_6B
    depths = [int(d) for d in args.depths.split(",")]
    steps = args.steps
    state, prompt = mq.random_init_state(cfg, seed=args.seed)
    S = max(depths) + max(steps, args.warmup) + 8
    cos, sin = mq.precompute_rope_freqs(cfg.head_dim, S, cfg.rope_theta, device=dev)
    qstate = mq.quantize_state(state, cfg, dev)
    del state
    embed, layers, scales, lm_q, lm_s, fnorm = mq.pack_int8(qstate, cfg)
    dec = mq.A10Int8MegakernelDecoder(embed, layers, scales, lm_q, lm_s, fnorm, cos, sin, cfg.num_layers, S)
    dec.set_attn_split(args.split_min)
    mq.set_decode_variant(args.variant)
    first = int(prompt[-1])
    events = _events(torch, steps)
    per_depth = {}
    for depth in depths:
        dec.prefill_random_kv(depth, seed=args.seed)
        tok = first
        for _ in range(args.warmup):
            tok = dec.decode_step(tok)
        dec.prefill_random_kv(depth, seed=args.seed)
        toks, wall, _ = _timed_pass(torch, dec, first, steps, dec.wait_token)
        if min(toks) < 0:
            raise RuntimeError(f"a timed decode step at depth {depth} failed: {mq._lib.last_error()}")
        dec.prefill_random_kv(depth, seed=args.seed)
        toks2, _, kern_ms = _timed_pass(torch, dec, first, steps, dec.wait_token, events)
        bytes_total = sum(cfg.int8_step_bytes(cache_len=depth + i + 1) for i in range(steps))
        achieved = bytes_total / (sum(kern_ms) / 1e3) / 1e9
        roof_tok_s = steps / (bytes_total / (HBM_PEAK_GBS * 1e9))
        per_depth[str(depth)] = {
            "tok_s": round(steps / wall, 1), "kernel_avg_us": round(sum(kern_ms) / steps * 1e3, 2),
            "device_tok_s": round(steps / (sum(kern_ms) / 1e3), 1), "achieved_GBs": round(achieved, 1),
            "frac": round(achieved / HBM_PEAK_GBS, 4), "roofline_tok_s": round(roof_tok_s, 1),
            "bytes_per_launch_avg": int(bytes_total / steps), "kernel_pass_tokens_identical": toks2 == toks,
            "kernel": mq.decode_variant(cfg.hidden_size, cfg.intermediate_size, int8=True, cache_len=depth + 1)}
        print(f"depth {depth}: {per_depth[str(depth)]}", file=sys.stderr, flush=True)
    top = per_depth[str(max(depths))]
    mq.set_decode_variant("auto")
    variant = args.variant
    return {"metric": f"INT8 decode tok/s at KV depth {max(depths)}, Qwen3-0.6B shape bs=1 (BASELINE config 4)",
            "value": top["tok_s"], "unit": "tok/s", "n_gpus": 1, "steps": steps, "warmup": args.warmup,
            "ms_per_step": round(1e3 / top["tok_s"], 4), "higher_is_better": True, "scaling": "weak",
            "vs_baseline": None, "dtype": "f64", "data": "synthetic",
            "config": {"workload": "config 4: KV cache pre-filled with seeded N(0,1) bf16 rows to each depth, "
                                   "then K greedy steps timed per depth",
                       "depths": depths, "variant": variant,
                       "attn_split_min": args.split_min or "library default", "per_depth": per_depth},
            "roofline": {"bound": "hbm", "achieved": top["achieved_GBs"], "peak": HBM_PEAK_GBS, "unit": "GB/s",
                         "frac": top["frac"], "traffic": None, "kernel_avg_us": top["kernel_avg_us"],
                         "timing": KERNEL_TIMING}}


def _prefill_ops(cfg, P):
    """int8 digit-plane products the prefill's matrix cores execute for P positions: every
    product over the padded position count (multiples of 32), 8 digit planes per position,
    the last layer's QKV only."""
    H, I, Q, KV, L = cfg.hidden_size, cfg.intermediate_size, cfg.q_size, cfg.kv_size, cfg.num_layers
    Pp = (P + 31) // 32 * 32
    qkv = (Q + 2 * KV) * H
    rest = H * Q + 2 * I * H + H * I
    return 2 * 8 * Pp * (L * qkv + (L - 1) * rest)


PREFILL_PHASES = ("input_digits", "qkv", "attention", "attn_digits", "o", "post_attn_digits", "gate_up",
                  "swiglu_digits", "down")


def _prefill_phases(dec, ids, torch):
    """Phase timeline of the prefill's last chunk (the kernel's optional trace, 100 MHz clock):
    per phase, the time from the grid barrier before it (the last workgroup out) to the last
    workgroup done, and the barrier after it (last workgroup done to last workgroup out);
    microseconds averaged over layers 1 .. L-2 and 3 prefills."""
    import numpy as np
    L = dec.num_layers
    ncu = torch.cuda.get_device_properties(dec.device).multi_processor_count
    buf = torch.zeros(L * 18 * ncu, dtype=torch.int64, device=dec.device)
    split = len(ids) - (len(ids) - 1) % dec.PREFILL_CHUNK - 1         # all chunks but the last untraced
    recs = []
    for _ in range(3):
        dec.reset()
        if split:
            dec.prefill(ids[:split])
        dec.set_prefill_trace(buf)
        buf.zero_()
        dec.prefill(ids[split:])
        dec.set_prefill_trace(None)
        torch.cuda.synchronize()
        recs.append(buf.view(L, 18, ncu).cpu().numpy().astype(np.float64) / 100.0)
    T = np.stack(recs)[:, :L - 1]
    out = {}
    for k, name in enumerate(PREFILL_PHASES):
        done, passed = T[:, 1:, 2 * k, :], T[:, 1:, 2 * k + 1, :]
        start = T[:, :-1, 17, :] if k == 0 else T[:, 1:, 2 * k - 1, :]
        work = (done.max(axis=2) - start.max(axis=2)).mean()
        barrier = (passed.max(axis=2) - done.max(axis=2)).mean()
        out[name] = [round(float(work), 1), round(float(barrier), 1)]
    out["layer"] = round(float((T[:, 1:, 17, :].max(axis=2) - T[:, :-1, 17, :].max(axis=2)).mean()), 1)
    return out


def run_prefill(args, mq, torch):
    """Prompt-batched prefill: the K/V cache rows of a P-token prompt of the config-1
    model written by A10Int8MegakernelDecoder.prefill (each layer's weights once for all P positions),
    against the reference's way, P decode steps. HIP events around each prefill on its stream."""
    dev = torch.device("cuda:0")
    cfg = mq.QWEN3_0_6B
    lens = [int(v) for v in args.prompt_lens.split(",")]
    S = max(lens) + 8
    state, _ = mq.random_init_state(cfg, seed=args.seed)
    cos, sin = mq.precompute_rope_freqs(cfg.head_dim, S, cfg.rope_theta, device=dev)
    qstate = mq.quantize_state(state, cfg, dev)
    del state
    embed, layers, scales, lm_q, lm_s, fnorm = mq.pack_int8(qstate, cfg)
    dec = mq.A10Int8MegakernelDecoder(embed, layers, scales, lm_q, lm_s, fnorm, cos, sin, cfg.num_layers, S)
    g = torch.Generator().manual_seed(args.seed + 1)
    t0e, t1e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    per_len = {}
    for P in lens:
        ids = torch.randint(0, cfg.vocab_size, (P,), generator=g).tolist()
        reps = max(3, min(20, 4096 // P))
        dec.reset()
        dec.prefill(ids)                                   # warm-up (workspace, code objects)
        torch.cuda.synchronize()
        ms = []
        for _ in range(reps):
            dec.reset()
            torch.cuda.synchronize()
            t0 = time.perf_counter()
            t0e.record()
            dec.prefill(ids)
            host = time.perf_counter() - t0
            t1e.record()
            torch.cuda.synchronize()
            wall = time.perf_counter() - t0
            ms.append((t0e.elapsed_time(t1e), wall * 1e3, host * 1e3))
        k_batched, v_batched = dec.k_cache[:, :, :P].clone(), dec.v_cache[:, :, :P].clone()
        dev_ms = sum(m[0] for m in ms) / reps
        wall_ms = sum(m[1] for m in ms) / reps
        host_ms = sum(m[2] for m in ms) / reps
        # the reference's way: one decode step per prompt token
        dec.reset()
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for t in ids:
            dec.decode_step(int(t))
        steps_ms = (time.perf_counter() - t0) * 1e3
        same = float(((dec.k_cache[:, :, :P] == k_batched).double().mean() +
                      (dec.v_cache[:, :, :P] == v_batched).double().mean()) / 2)
        ops = _prefill_ops(cfg, P)
        w_bytes = cfg.int8_step_bytes() - cfg.vocab_size * (cfg.hidden_size + 4)     # layer weights, no LM head
        per_len[str(P)] = {
            "tok_s": round(P / (wall_ms / 1e3), 1), "device_ms": round(dev_ms, 3), "wall_ms": round(wall_ms, 3),
            "host_call_ms": round(host_ms, 3),
            "per_token_steps_ms": round(steps_ms, 2), "per_token_steps_tok_s": round(P / (steps_ms / 1e3), 1),
            "speedup_vs_per_token_steps": round(steps_ms / wall_ms, 1),
            "mfma_digit_tops": round(ops / (dev_ms / 1e3) / 1e12, 1),
            "mfma_frac": round(ops / (dev_ms / 1e3) / 1e12 / INT8_PEAK_TOPS, 4),
            "weight_GBs": round(w_bytes / (dev_ms / 1e3) / 1e9, 1),
            "kv_rows_identical_to_per_token_steps": round(same, 6), "reps": reps,
            "last_chunk_phase_us_work_barrier": _prefill_phases(dec, ids, torch)}
        print(f"prefill P={P}: {per_len[str(P)]}", file=sys.stderr, flush=True)
    head = str(512 if 512 in lens else max(lens))
    top = per_len[head]
    return {"metric": f"INT8 prompt prefill tok/s, Qwen3-0.6B shape bs=1, prompt of {head} tokens (SURVEY f1)",
            "value": top["tok_s"], "unit": "tok/s", "n_gpus": 1, "steps": top["reps"], "warmup": 1,
            "ms_per_step": top["wall_ms"], "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
            "dtype": "int8 digit products (exact), fp64 attention and norms", "data": "synthetic",
            "config": {"workload": "prompt-batched prefill of P random tokens into an empty KV cache of the config-1 "
                                   "model (random-init seed 0), K/V rows of all 28 layers; a step = one prefill",
                       "prompt_lens": lens, "per_len": per_len},
            "roofline": {"bound": "mfma", "achieved": top["mfma_digit_tops"], "peak": INT8_PEAK_TOPS,
                         "unit": "TOP/s", "frac": top["mfma_frac"], "traffic": None,
                         "timing": "int8 digit-plane products executed (8 planes per position, positions padded to "
                                   "32) over the whole prefill's device time (HIP events around it: norms, "
                                   "attention and launch gaps included)"}}


def run_batched(args, mq, torch):
    """batched INT8 decode of the Qwen3-1.7B shape, B independent seeded
    8-token prompts, then K greedy steps timed per batch size (kernel time from HIP events)."""
    dev = torch.device("cuda:0")
    cfg = mq.QWEN3_1_7B
    batches = [int(b) for b in args.batches.split(",")]
    steps = args.steps
    state, _ = mq.random_init_state(cfg, seed=args.seed)
    S = PROMPT_LEN + steps + max(args.warmup, 1) + 8
    cos, sin = mq.precompute_rope_freqs(cfg.head_dim, S, cfg.rope_theta, device=dev)
    qstate = mq.quantize_state(state, cfg, dev)
    del state
    packed = mq.pack_int8(qstate, cfg)
    del qstate
    g = torch.Generator().manual_seed(args.seed + 100)
    prompts_all = torch.randint(0, cfg.vocab_size, (max(batches), PROMPT_LEN), generator=g).tolist()
    weight_bytes = cfg.int8_step_bytes(cache_len=0) - cfg.num_layers * 2 * cfg.num_kv_heads * cfg.head_dim * 2
    # useful int8 multiply-adds per sequence and step: every projection and the LM head once
    H, I, V, L = cfg.hidden_size, cfg.intermediate_size, cfg.vocab_size, cfg.num_layers
    macs = L * (H * (cfg.q_size + 2 * cfg.kv_size) + cfg.q_size * H + 3 * H * I) + V * H
    events = _events(torch, steps)
    oracle = None
    if args.check_steps > 0:
        from oracle.ref_cpu import Dims, RefDecoder
        embed, layers, scales, lm_q, lm_s, fnorm = packed
        c = lambda t: t.cpu()
        oracle = RefDecoder(Dims(hidden_size=H, intermediate_size=I, vocab_size=V), c(embed), [c(t) for t in layers],
                            [c(t) for t in scales], c(fnorm), c(lm_q), c(lm_s), c(cos), c(sin), L, S)
    per_batch = {}
    for B in batches:
        prompts = prompts_all[:B]
        dec = mq.A10Int8BatchDecoder(*packed, cos, sin, L, S, B)

        def prefill():
            dec.reset()
            out = None
            for i in range(PROMPT_LEN):
                out = dec.decode_step([p[i] for p in prompts])
            return out

        out = prefill()
        for _ in range(args.warmup):
            out = dec.decode_step(out)
        first = prefill()
        toks, wall, _ = _timed_pass(torch, dec, first, steps, dec.wait_tokens)
        out = toks[-1]
        first2 = prefill()
        toks2, _, kern_ms = _timed_pass(torch, dec, first2, steps, dec.wait_tokens, events)
        if min(out) < 0:
            raise RuntimeError(f"a timed batched step (B={B}) failed: {mq._lib.last_error()}")
        kern_s = sum(kern_ms) / 1e3
        kv_bytes = sum(B * L * 2 * cfg.num_kv_heads * cfg.head_dim * 2 * (PROMPT_LEN + i + 1) for i in range(steps))
        achieved = (steps * weight_bytes + kv_bytes) / kern_s / 1e9
        mfma_tops = 2.0 * macs * B * steps / kern_s / 1e12
        per_batch[str(B)] = {
            "tok_s": round(B * steps / wall, 1), "kernel_avg_us": round(kern_s / steps * 1e6, 2),
            "device_tok_s": round(B * steps / kern_s, 1), "achieved_GBs": round(achieved, 1),
            "hbm_frac": round(achieved / HBM_PEAK_GBS, 4),
            "roofline_tok_s": round(B * HBM_PEAK_GBS * 1e9 / (weight_bytes + kv_bytes / steps / 1.0), 1),
            "useful_int8_TOPs": round(mfma_tops, 2), "mfma_util": round(mfma_tops / INT8_PEAK_TOPS, 5),
            "kernel_pass_tokens_identical": first2 == first and toks2 == toks}
        if oracle is not None:
            s_ = B - 1                           # a different prompt slot for every batch size
            gen = [first[s_]] + [t[s_] for t in toks]
            per_batch[str(B)]["parity"] = _teacher_force(oracle, prompts[s_], gen[:args.check_steps], s_)
        print(f"batch {B}: {per_batch[str(B)]}", file=sys.stderr, flush=True)
        del dec
        torch.cuda.empty_cache()
    top = per_batch[str(max(batches))]
    return {"metric": f"batched INT8 decode aggregate tok/s, Qwen3-1.7B shape, batch {max(batches)} (BASELINE config 5)",
            "value": top["tok_s"], "unit": "tok/s", "n_gpus": 1, "steps": steps, "warmup": args.warmup,
            "ms_per_step": round(1e3 * max(batches) / top["tok_s"], 4), "higher_is_better": True, "scaling": "weak",
            "vs_baseline": None, "dtype": "int8 x 4-digit int8 (int32 sums), fp64 recombination", "data": "synthetic",
            "config": {"workload": "config 5: Qwen3-1.7B architecture random-init (seed 0), independent seeded 8-token "
                                   "prompts per sequence prefilled untimed, K greedy steps timed per batch size",
                       "batches": batches, "per_batch": per_batch,
                       "parity_all_match": None if oracle is None else all(
                           v["parity"]["match"] for v in per_batch.values()),
                       "weight_bytes_per_step": weight_bytes, "useful_int8_macs_per_token": macs},
            "roofline": {"bound": "hbm", "achieved": top["achieved_GBs"], "peak": HBM_PEAK_GBS, "unit": "GB/s",
                         "frac": top["hbm_frac"], "traffic": None, "kernel_avg_us": top["kernel_avg_us"],
                         "mfma_util": top["mfma_util"],
                         "timing": KERNEL_TIMING}}


def _teacher_force(oracle, prompt, gen, seq, min_margin=1e-3):
    """Feed `prompt` and then the GPU's own tokens `gen` to the float64 oracle; each GPU token
    must be the oracle's argmax wherever the oracle's top-2 margin exceeds `min_margin`
    (fp32 logit rounding is far below it)."""
    import torch
    from oracle.ref_cpu import top2_margin

    oracle.reset()
    logits = None
    for t in prompt:
        logits = oracle.step_logits(int(t))
    checked = mismatched = skipped = 0
    for i, tok in enumerate(gen):
        if top2_margin(logits) > min_margin:
            checked += 1
            mismatched += int(tok != int(torch.argmax(logits)))
        else:
            skipped += 1
        if i + 1 < len(gen):
            logits = oracle.step_logits(int(tok))
    return {"sequence": seq, "tokens": len(gen), "checked": checked, "skipped_small_margin": skipped,
            "match": checked > 0 and mismatched == 0,
            "oracle": "oracle.ref_cpu float64, prompt then the GPU's tokens teacher-forced"}


def run_traffic(args, mq, torch):
    """Counter calibration plus decode steps for rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE runs."""
    dev = torch.device("cuda:0")
    nbytes = 256 * 2 ** 20
    a = torch.zeros(nbytes, dtype=torch.uint8, device=dev)
    b = torch.empty_like(a)
    for _ in range(4):
        torch.add(a, 1, out=b)              # reads nbytes, writes nbytes
    torch.cuda.synchronize()
    del a, b
    cfg = mq.QWEN3_0_6B
    state, prompt = mq.random_init_state(cfg, seed=args.seed)
    S = PROMPT_LEN + 16
    cos, sin = mq.precompute_rope_freqs(cfg.head_dim, S, cfg.rope_theta, device=dev)
    qstate = mq.quantize_state(state, cfg, dev)
    del state
    embed, layers, scales, lm_q, lm_s, fnorm = mq.pack_int8(qstate, cfg)
    dec = mq.A10Int8MegakernelDecoder(embed, layers, scales, lm_q, lm_s, fnorm, cos, sin, cfg.num_layers, S)
    tok = None
    for t in prompt.tolist():
        tok = dec.decode_step(int(t))
    for _ in range(8):
        tok = dec.decode_step(tok)
    torch.cuda.synchronize()
    return {"metric": "counter calibration run", "value": 0, "unit": "none", "n_gpus": 1, "steps": 8, "warmup": 0,
            "ms_per_step": 0, "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "f64",
            "data": "synthetic",
            "config": {"workload": "traffic: 4 x uint8 add over 256 MiB (256 MiB read + 256 MiB written each), "
                                   "then 8-token prefill + 8 decode steps of config 1",
                       "copy_bytes": nbytes, "decode_steps": 16, "variant": mq.decode_variant()}}


def main():
    args = parse()
    if args.gpus != 1:
        print(f"bench.py runs on one GPU only (asked for --gpus {args.gpus}): the batch-1 decode step runs on a "
              "single device", file=sys.stderr)
        return 2
    import torch
    import __graft_entry__
    mq = __graft_entry__.load_package()
    if not torch.cuda.is_available():
        print("no HIP device visible", file=sys.stderr)
        return 1
    fn = {"decode": run_decode, "matvec": run_matvec, "formats": run_formats, "positions": run_positions,
          "longctx": run_longctx,
          "batched": run_batched, "prefill": run_prefill, "traffic": run_traffic}[args.workload]
    out = fn(args, mq, torch)
    print(json.dumps(out), flush=True)
    return 0


if __name__ == "__main__":
    # return normally on success (the interpreter-shutdown path profilers finalise on)
    status = main()
    if status:
        sys.exit(status)
