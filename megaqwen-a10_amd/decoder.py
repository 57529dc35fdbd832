"""Drop-in decoder classes for the batch-1 decode path.

* ``A10Int8MegakernelDecoder`` — the INT8 class of bench_int8.py:119-255
  (same constructor arguments, ``decode_step`` / ``reset`` / ``position``).
* ``A10MegakernelDecoder`` — the bf16 class of a10_decode.py:87-261, with the
  debug getters of run_benchmark.py:174-183.
* ``A10Decoder`` — the Python wrapper of a10_decode.py:35-393 (``.decoder``,
  ``reset``, ``generate``), which here loads weights from a safetensors
  checkpoint directory or builds seeded random-init weights.

Each step is ONE launch of the persistent gfx950 kernel (csrc/decode.hip)
through the C ABI; the returned token is read back like the reference's
``output_token_.item<int>()`` (bench_int8.py:218). Arguments are validated on
the host before anything is launched (the reference launches unchecked):
wrong dtypes/shapes/devices/counts raise ``TypeError``/``ValueError``, a token
id outside the vocabulary or a full KV cache raise ``ValueError``.
"""
from __future__ import annotations

import ctypes
import math
import time
from pathlib import Path

import torch

from . import _lib
from .config import QWEN3_0_6B, ModelConfig
from .rope import precompute_rope_freqs
from .weights import pack_bf16, pack_int8, quantize_state, random_init_state

TOKEN_PENDING = -2          # written into a pinned token word before a launch; kernels store >= -1
WAIT_US = 2_000_000         # host spin on the token before falling back to a stream synchronisation
TOKEN_SLOTS = 256           # pinned token words, one per step in flight (launch_step without wait_token)

LM_PARTIALS = 256   # per-workgroup LM-head maxima written to block_max_vals/idxs

VARIANTS = {"auto": 0, "flat": 1, "xcd": 2, "async": 3}


def set_decode_variant(name: str) -> None:
    """Select the decode kernel for all following steps in this process:
    ``"auto"`` (default: the async-wave kernel for INT8 Qwen3-0.6B-shape steps
    up to 6144 cached positions (10240 when forced), else the XCD-aware kernel when the workgroups of
    each residue class g mod 8 share one XCD, checked once per device),
    ``"flat"`` (single-level exchanges), ``"xcd"`` or ``"async"``."""
    lib = _lib.load()
    _lib.check(lib.mq_decode_set_variant(VARIANTS[name]), "mq_decode_set_variant")


def set_cooperative_launch(enable: bool) -> None:
    """Launch the persistent kernels cooperatively from now on (``True``): the runtime then
    starts a step only when all of its workgroups can be resident at once, at about 10 us
    per launch; ``False`` (default) launches plainly (mq_decode_set_cooperative)."""
    _lib.check(_lib.load().mq_decode_set_cooperative(int(bool(enable))), "mq_decode_set_cooperative")


def decode_variant(hidden_size: int = 1024, intermediate_size: int = 3072, int8: bool = True,
                   cache_len: int | None = None) -> str:
    """The kernel a step with these dims would use now (attending over ``cache_len`` cached
    positions, the first step's 1 when omitted)."""
    lib = _lib.load()
    dims = _lib.ModelDims(hidden_size, intermediate_size, 16, 8, 128, 151936)
    if cache_len is None:
        v = lib.mq_decode_variant(ctypes.byref(dims), int(int8))
    else:
        v = lib.mq_decode_variant_at(ctypes.byref(dims), int(int8), int(cache_len))
    if v < 0:
        _lib.check(-v, "mq_decode_variant")
    return {1: "flat", 2: "xcd", 3: "async"}[v]


def _check_tensor(t, name, dtype, shape=None, device=None):
    if not isinstance(t, torch.Tensor):
        raise TypeError(f"{name}: expected a torch.Tensor, got {type(t).__name__}")
    if t.dtype != dtype:
        raise TypeError(f"{name}: expected dtype {dtype}, got {t.dtype}")
    if not t.is_cuda:
        raise ValueError(f"{name}: must live on a HIP device")
    if device is not None and t.device != device:
        raise ValueError(f"{name}: on {t.device}, expected {device}")
    if shape is not None and tuple(t.shape) != tuple(shape):
        raise ValueError(f"{name}: expected shape {tuple(shape)}, got {tuple(t.shape)}")
    if not t.is_contiguous():
        raise ValueError(f"{name}: must be contiguous")


def _device_array(structs, device) -> torch.Tensor:
    raw = bytes(structs)
    host = torch.frombuffer(bytearray(raw), dtype=torch.uint8)
    return host.to(device)


class _DecoderBase:
    """Owns the KV cache, the reference's scratch buffers, the workspace and the step state."""

    _int8: bool = True         # one-byte weights with per-row scales
    _fp8: bool = False         # ... that are FP8 E4M3 codes rather than int8
    _int4: bool = False        # layer projections INT4 per group of 128 (LM head INT8 per row)

    def _setup(self, embed, layer_tensors, final_norm, lm_head, cos_table, sin_table, num_layers,
               max_seq_len, layer_scales=None, lm_head_scale=None):
        self._hold_weights(embed, layer_tensors, final_norm, lm_head, cos_table, sin_table, num_layers,
                           max_seq_len, layer_scales, lm_head_scale)
        self._alloc_state()

    def _hold_weights(self, embed, layer_tensors, final_norm, lm_head, cos_table, sin_table, num_layers,
                      max_seq_len, layer_scales=None, lm_head_scale=None):
        """Validate the reference's constructor arguments and keep them (with the device
        LayerWeights / ScalePointers arrays) alive on the decoder."""
        if not isinstance(num_layers, int) or num_layers < 1:
            raise ValueError(f"num_layers must be a positive int, got {num_layers!r}")
        if not isinstance(max_seq_len, int) or max_seq_len < 1:
            raise ValueError(f"max_seq_len must be a positive int, got {max_seq_len!r}")
        _check_tensor(embed, "embed_weight", torch.bfloat16)
        if embed.dim() != 2:
            raise ValueError("embed_weight must be [vocab, hidden]")
        dev = embed.device
        V, H = embed.shape
        if len(layer_tensors) != 11 * num_layers:
            raise ValueError(f"layer_weights_flat: expected {11 * num_layers} tensors (11 per layer), "
                             f"got {len(layer_tensors)}")
        wdt = torch.uint8 if (self._fp8 or self._int4) else torch.int8 if self._int8 else torch.bfloat16
        I = layer_tensors[8].shape[0]
        D = 128
        Q, KV = 16 * D, 8 * D
        # INT4: packed rows of in / 2 bytes, one scale per group of 128 inputs
        w_ = (lambda o, i: (o, i // 2)) if self._int4 else (lambda o, i: (o, i))
        s_ = (lambda o, i: (o, i // 128)) if self._int4 else (lambda o, i: (o,))
        shapes = [(H,), w_(Q, H), w_(KV, H), w_(KV, H), (D,), (D,), w_(H, Q), (H,), w_(I, H), w_(I, H), w_(H, I)]
        dtypes = [torch.bfloat16, wdt, wdt, wdt, torch.bfloat16, torch.bfloat16, wdt, torch.bfloat16,
                  wdt, wdt, wdt]
        for i, t in enumerate(layer_tensors):
            _check_tensor(t, f"layer_weights_flat[{i}]", dtypes[i % 11], shapes[i % 11], dev)
        if self._int8:
            if layer_scales is None or len(layer_scales) != 7 * num_layers:
                raise ValueError(f"layer_scales_all: expected {7 * num_layers} tensors (7 per layer)")
            sshapes = [s_(Q, H), s_(KV, H), s_(KV, H), s_(H, Q), s_(I, H), s_(I, H), s_(H, I)]
            for i, t in enumerate(layer_scales):
                _check_tensor(t, f"layer_scales_all[{i}]", torch.float32, sshapes[i % 7], dev)
            _check_tensor(lm_head_scale, "lm_head_scale", torch.float32, (V,), dev)
        _check_tensor(lm_head, "lm_head", torch.int8 if self._int4 else wdt, (V, H), dev)
        _check_tensor(final_norm, "final_norm_weight", torch.bfloat16, (H,), dev)
        _check_tensor(cos_table, "cos_table", torch.bfloat16, None, dev)
        _check_tensor(sin_table, "sin_table", torch.bfloat16, None, dev)
        if cos_table.dim() != 2 or cos_table.shape[1] != D or cos_table.shape[0] < max_seq_len:
            raise ValueError(f"cos_table must be [>= max_seq_len, {D}], got {tuple(cos_table.shape)}")
        if tuple(sin_table.shape) != tuple(cos_table.shape):
            raise ValueError("sin_table must match cos_table")

        self.device = dev
        self.num_layers = num_layers
        self.max_seq_len = max_seq_len
        self.dims = (H, I, V)
        self._pos = 0
        self.attn_scale = 1.0 / math.sqrt(float(D))
        # hold every tensor the kernel reads (the reference's INT8 class drops the scale list)
        self.embed_weight = embed
        self.layer_tensors = list(layer_tensors)
        self.layer_scales = list(layer_scales) if layer_scales is not None else None
        self.final_norm_weight = final_norm
        self.lm_head_weight = lm_head
        self.lm_head_scale = lm_head_scale
        self.cos_table, self.sin_table = cos_table, sin_table

        lw = (_lib.LayerWeights * num_layers)()
        for l in range(num_layers):
            for f, t in zip(_lib.LAYER_FIELDS, layer_tensors[11 * l: 11 * l + 11]):
                setattr(lw[l], f, t.data_ptr())
        self.d_layer_weights = _device_array(lw, dev)
        self.d_layer_scales = None
        if self._int8:
            sp = (_lib.ScalePointers * num_layers)()
            for l in range(num_layers):
                for f, t in zip(_lib.SCALE_FIELDS, layer_scales[7 * l: 7 * l + 7]):
                    setattr(sp[l], f, t.data_ptr())
            self.d_layer_scales = _device_array(sp, dev)

    def _alloc_state(self):
        dev, num_layers, max_seq_len = self.device, self.num_layers, self.max_seq_len
        H, I, V = self.dims
        D = 128
        Q, KV = 16 * D, 8 * D
        embed, final_norm, lm_head, lm_head_scale = (self.embed_weight, self.final_norm_weight, self.lm_head_weight,
                                                     self.lm_head_scale)
        cos_table, sin_table = self.cos_table, self.sin_table
        f32 = dict(dtype=torch.float32, device=dev)
        self.k_cache = torch.zeros((num_layers, 8, max_seq_len, D), dtype=torch.bfloat16, device=dev)
        self.v_cache = torch.zeros_like(self.k_cache)
        self.hidden_buffer = torch.zeros(H, dtype=torch.bfloat16, device=dev)
        self.g_activations = torch.zeros(H, **f32)
        self.g_residual = torch.zeros(H, **f32)
        self.g_q = torch.zeros(Q, **f32)
        self.g_k = torch.zeros(KV, **f32)
        self.g_v = torch.zeros(KV, **f32)
        self.g_attn_out = torch.zeros(Q, **f32)
        self.g_mlp_intermediate = torch.zeros(I, **f32)
        self.g_normalized = torch.zeros(H, **f32)
        self.block_max_vals = torch.zeros(LM_PARTIALS, **f32)
        self.block_max_idxs = torch.zeros(LM_PARTIALS, dtype=torch.int32, device=dev)
        # the kernel writes the token straight into pinned host memory: the host spins on
        # it (no device-to-host copy, no stream-synchronisation wake-up). Each step in
        # flight has its own word, so a step launched behind another (a prefill that does
        # not read its tokens) cannot have its word overwritten by the earlier one's store.
        self.output_token = torch.full((TOKEN_SLOTS,), TOKEN_PENDING, dtype=torch.int32, pin_memory=True)
        self._tok_host = self.output_token.numpy()
        self._next_slot = 0
        self._inflight = []          # (slot, position) of every launched step not yet collected

        self._lib = _lib.load()
        self._dims = _lib.ModelDims(H, I, 16, 8, D, V)
        ws_bytes = self._lib.mq_decode_workspace_bytes(ctypes.byref(self._dims))
        if ws_bytes == 0:
            raise ValueError(f"unsupported model dims H={H} I={I}: {_lib.last_error()}")
        self.workspace = torch.empty(ws_bytes, dtype=torch.uint8, device=dev)
        self._stream = None
        self._init_workspace()

        a = _lib.DecodeArgs()
        a.output_token_id = self.output_token.data_ptr()      # slot 0; launch_step picks the slot
        a.embed_weight = embed.data_ptr()
        a.layer_weights = self.d_layer_weights.data_ptr()
        a.scales = self.d_layer_scales.data_ptr() if self._int8 else None
        a.final_norm_weight = final_norm.data_ptr()
        a.lm_head_weight = lm_head.data_ptr()
        a.lm_head_scale = lm_head_scale.data_ptr() if self._int8 else None
        a.cos_table, a.sin_table = cos_table.data_ptr(), sin_table.data_ptr()
        a.k_cache, a.v_cache = self.k_cache.data_ptr(), self.v_cache.data_ptr()
        a.num_layers = num_layers
        a.max_seq_len = max_seq_len
        a.attn_scale = self.attn_scale
        a.dims = ctypes.addressof(self._dims)
        a.workspace = self.workspace.data_ptr()
        a.workspace_bytes = ws_bytes
        a.spin_limit = 0
        self._args = a
        self._args_ref = ctypes.byref(a)
        self._tok_base = self.output_token.data_ptr()
        self._step_fn = (self._lib.mq_fp8_decode_step if self._fp8 else
                         self._lib.mq_int4_decode_step if self._int4 else
                         self._lib.mq_int8_decode_step if self._int8 else self._lib.mq_bf16_decode_step)
        self._debug = False

    def _init_workspace(self):
        with torch.cuda.device(self.device):
            _lib.check(self._lib.mq_workspace_init(self.workspace.data_ptr(), self.workspace.numel(),
                                                   _lib.stream_handle()), "mq_workspace_init")

    # -- reference surface ---------------------------------------------------------------
    def launch_step(self, input_token_id: int) -> None:
        """Enqueue one decode step on the current stream without waiting for the token.
        Several steps may be launched before ``wait_token`` (for example a prefill whose
        tokens are not needed); ``wait_token`` then returns the last one's token."""
        # (kept lean: this is on every step's host path, between one kernel and the next)
        if not isinstance(input_token_id, int) or not 0 <= input_token_id < self.dims[2]:
            raise ValueError(f"input_token_id {input_token_id!r} outside [0, {self.dims[2]})")
        pos = self._pos
        if pos >= self.max_seq_len:
            raise ValueError(f"KV cache full: position {pos} == max_seq_len {self.max_seq_len}")
        slot = self._next_slot
        if len(self._inflight) >= TOKEN_SLOTS:
            # every token word is held by a step in flight (slots are handed out in turn):
            # let them finish before this one is reused
            torch.cuda.current_stream(self.device).synchronize()
        a = self._args
        a.input_token_id = input_token_id
        a.position = pos
        a.cache_len = pos + 1
        a.output_token_id = self._tok_base + 4 * slot
        self._tok_host[slot] = TOKEN_PENDING
        st = self._step_fn(self._args_ref, _lib.stream_handle(self.device))
        if st:
            _lib.check(st, "decode step")
        self._inflight.append((slot, self._pos))
        self._next_slot = (slot + 1) % TOKEN_SLOTS
        self._pos += 1

    def wait_token(self) -> int:
        """Wait for the last enqueued step and return its token. Spins on the pinned word the
        kernel stores last; falls back to a stream synchronisation (which reports errors) if
        no token arrives within WAIT_US or the step reports a failure (-1).

        A failed step (its in-kernel wait expired, MQTimeoutError) leaves the decoder at that
        step's position with a re-initialised workspace: the steps from there on are undone,
        and decoding continues by feeding the same token again (the cache rows the failed
        steps wrote are rewritten when those positions are recomputed)."""
        if not self._inflight:
            raise RuntimeError("no decode step in flight (call launch_step first)")
        slot = self._inflight[-1][0]
        if self._lib.mq_wait_host_token(self._tok_base + 4 * slot, TOKEN_PENDING, WAIT_US) != _lib.MQ_OK:
            torch.cuda.current_stream(self.device).synchronize()
        tok = int(self._tok_host[slot])
        if tok < 0:
            torch.cuda.current_stream(self.device).synchronize()
            # a failed step makes every later step on the workspace fail too: resume at the first
            failed = [pos for sl, pos in self._inflight if int(self._tok_host[sl]) < 0]
            self._pos = failed[0] if failed else self._inflight[-1][1]
            self._inflight.clear()
            status = self._lib.mq_decode_check(self.workspace.data_ptr(),
                                               ctypes.c_void_p(_lib.stream_handle(self.device)))
            self._init_workspace()
            _lib.check(status if status != _lib.MQ_OK else _lib.MQ_ERR_TIMEOUT, "decode step")
        self._inflight.clear()
        return tok

    def decode_step(self, input_token_id: int) -> int:
        self.launch_step(input_token_id)
        return self.wait_token()

    def reset(self) -> None:
        if self._inflight:
            # steps still in flight store into their token words: let them land first
            torch.cuda.current_stream(self.device).synchronize()
            self._inflight.clear()
        self._pos = 0
        self.k_cache.zero_()
        self.v_cache.zero_()

    def position(self) -> int:
        return self._pos

    def set_timing_events(self, start=None, stop=None) -> None:
        """Have every following step record ``start``/``stop`` (torch.cuda.Event with
        timing) at the kernel's own start and end; ``None`` turns it off."""
        if start is None or stop is None:
            self._args.timing_start = None
            self._args.timing_stop = None
            return
        for e in (start, stop):
            if e.cuda_event == 0:
                e.record()          # torch creates the HIP event lazily
        self._args.timing_start = start.cuda_event
        self._args.timing_stop = stop.cuda_event

    _DEBUG_FIELDS = ("hidden_buffer", "g_activations", "g_residual", "g_q", "g_k", "g_v", "g_attn_out",
                     "g_mlp_intermediate", "g_normalized", "block_max_vals", "block_max_idxs")

    def enable_debug(self, on: bool = True) -> None:
        """Fill the per-stage buffers behind the debug getters on every following step
        (run_benchmark.py:174-183 semantics: the last layer's values). Off by default:
        the kernel then carries no debug outputs."""
        self._debug = bool(on)
        for f in self._DEBUG_FIELDS:
            setattr(self._args, f, getattr(self, f).data_ptr() if on else None)

    def set_trace(self, buf) -> None:
        """Record a per-stage timeline of every following step into ``buf`` (int64 tensor of
        ``(num_layers + 1) * 10 * 256`` entries on the decoder's device); ``None`` stops it."""
        if buf is None:
            self._args.trace = None
            return
        need = (self.num_layers + 1) * 10 * 256
        if buf.dtype != torch.int64 or buf.numel() < need or buf.device != self.device or not buf.is_contiguous():
            raise ValueError(f"trace buffer must be a contiguous int64 tensor of >= {need} entries on {self.device}")
        self._trace_buf = buf
        self._args.trace = buf.data_ptr()

    def set_spin_limit(self, polls: int) -> None:
        """Bound on every in-kernel wait (0 = library default)."""
        self._args.spin_limit = int(polls)

    def set_sampling(self, temperature: float = 0.0, seed: int = 0) -> None:
        """Token choice of every following step: ``temperature`` 0 (default) is the greedy
        argmax; above 0 the token is drawn from softmax(logits / temperature) by the
        Gumbel-max rule with noise keyed by (seed, position, vocabulary row), so a given
        seed gives the same tokens whether steps run one per launch or in one launch
        (``generate``). The reference accepts a temperature and ignores it
        (a10_decode.py:358)."""
        t = float(temperature)
        if not (t >= 0.0) or t == float("inf"):
            raise ValueError(f"temperature must be a finite value >= 0, got {temperature!r}")
        if not isinstance(seed, int) or not 0 <= seed < 2 ** 64:
            raise ValueError(f"seed must be an int in [0, 2**64), got {seed!r}")
        self._args.temperature = t
        self._args.seed = seed

    def generate(self, prompt_ids, n_tokens: int, device_loop: bool = True, batched_prefill: bool = True) -> list:
        """Feed ``prompt_ids`` from the current position and return ``n_tokens`` generated
        tokens, the first being the last prompt step's output (verify_correctness_a10.py:
        323-339). The tokens follow ``set_sampling``. With ``batched_prefill`` (INT8,
        hidden 1024) and a prompt of more than ``PREFILL_MIN`` tokens, every prompt token but
        the last goes through ``prefill`` (each layer's weights read once for the whole
        prompt); the last prompt token and every generated step are decode steps. With
        ``device_loop`` those steps run in ONE launch and hand their tokens on on the device
        (mq_int8/bf16/fp8_decode_generate: the async-wave kernel within its range, else the
        XCD-aware kernel's multi-step form); with ``device_loop=False``, or where neither
        kernel runs (the single-level fallback), one launch per step. All give the same
        tokens. A failed launch leaves the decoder at the position where its decode steps
        started."""
        ids = [int(t) for t in prompt_ids]
        V = self.dims[2]
        if not ids:
            raise ValueError("empty prompt")
        if any(not 0 <= t < V for t in ids):
            raise ValueError(f"prompt token outside [0, {V})")
        if not isinstance(n_tokens, int) or n_tokens < 1:
            raise ValueError(f"n_tokens must be a positive int, got {n_tokens!r}")
        if self._pos + len(ids) + n_tokens - 1 > self.max_seq_len:
            raise ValueError(f"position {self._pos} + {len(ids) + n_tokens - 1} steps exceed max_seq_len "
                             f"{self.max_seq_len}")
        if batched_prefill and len(ids) - 1 >= self.PREFILL_MIN and self.prefill_supported():
            self.prefill(ids[:-1])
            ids = ids[-1:]
        if device_loop:
            out = self._generate_one_launch(ids, n_tokens)
            if out is not None:
                return out
        tok = None
        for t in ids:
            tok = self.decode_step(t)
        out = [tok]
        while len(out) < n_tokens:
            tok = self.decode_step(tok)
            out.append(tok)
        return out

    PREFILL_CHUNK = 512      # positions per prefill chunk (workspace ~51 KB per position)
    # shortest prompt prefix generate() sends through prefill(): a prefill of a few positions
    # takes about 4 ms (one pass over the weights per product phase), as long as 12 decode steps
    # in one launch, so shorter prompts run as decode steps
    PREFILL_MIN = 16

    def prefill_supported(self) -> bool:
        """Whether ``prefill`` runs for this decoder (INT8 weights, hidden 1024)."""
        return self._int8 and not self._fp8 and not self._int4 and self.dims[:2] == (1024, 3072)

    def prefill(self, token_ids, check: bool = True) -> None:
        """Write the K/V cache rows of ``token_ids`` at the next positions, as that many
        decode steps would (a10_decode.py:367-368), with each layer's weights read once
        for the whole prompt (mq_int8_prefill: products of all positions on the int8
        matrix cores, causal attention in fp64). No token is produced: the decode step of
        the following token gives the next output. Runs in chunks of ``PREFILL_CHUNK``
        positions, one launch each. With ``check`` (default) the call waits for the prefill
        and raises MQTimeoutError if its grid-wide waits expired; otherwise it returns once
        the launches are queued on the current stream."""
        ids = [int(t) for t in token_ids]
        if not ids:
            return
        if not self.prefill_supported():
            raise ValueError("prefill runs for INT8 weights of hidden 1024 / intermediate 3072 only")
        V = self.dims[2]
        if any(not 0 <= t < V for t in ids):
            raise ValueError(f"token outside [0, {V})")
        if self._pos + len(ids) > self.max_seq_len:
            raise ValueError(f"positions {self._pos} + {len(ids)} exceed max_seq_len {self.max_seq_len}")
        stream = _lib.stream_handle(self.device)
        if self._inflight:
            # steps in flight store into their token words when they end: let them land first
            torch.cuda.current_stream(self.device).synchronize()
            self._inflight.clear()
        cap = min(self.PREFILL_CHUNK, (len(ids) + 63) // 64 * 64)
        if getattr(self, "_pf_cap", 0) < cap:
            nbytes = self._lib.mq_prefill_workspace_bytes(ctypes.byref(self._dims), cap)
            if nbytes == 0:
                raise ValueError(f"prefill: {_lib.last_error()}")
            self._pf_ws = torch.empty(nbytes, dtype=torch.uint8, device=self.device)
            self._pf_cap = cap
        if getattr(self, "_pf_tokens", None) is None:
            # pinned token list, reused: the library copies each chunk's tokens from it on the stream
            self._pf_tokens = torch.empty(self.max_seq_len, dtype=torch.int32, pin_memory=True)
            self._pf_done = torch.cuda.Event()
        else:
            self._pf_done.synchronize()          # the previous prefill's token copies have run
        self._pf_tokens.numpy()[:len(ids)] = ids
        a = self._args
        a.position = self._pos
        a.cache_len = self._pos + 1
        step_trace, a.trace = a.trace, getattr(self, "_pf_trace_ptr", None)   # the prefill's own timeline
        try:
            st = self._lib.mq_int8_prefill(ctypes.byref(a), ctypes.c_void_p(self._pf_tokens.data_ptr()), len(ids),
                                           ctypes.c_void_p(self._pf_ws.data_ptr()), self._pf_ws.numel(),
                                           ctypes.c_void_p(stream))
        finally:
            a.trace = step_trace
        self._pf_done.record(torch.cuda.current_stream(self.device))
        _lib.check(st, "mq_int8_prefill")
        if check:
            # waits for the prefill; a grid barrier that expired (compute units held by other
            # work) leaves the position unchanged
            _lib.check(self._lib.mq_prefill_check(ctypes.c_void_p(self._pf_ws.data_ptr()), self._pf_ws.numel(),
                                                  ctypes.c_void_p(stream)), "prefill")
        self._pos += len(ids)

    def set_prefill_trace(self, buf) -> None:
        """Record the phase timeline of the following prefills' last chunk into ``buf`` (int64,
        at least ``num_layers * 18 * n_cu`` entries on the decoder's device, n_cu = the device's
        compute units, entry ``(l * 18 + 2 k + e) * n_cu + g``: workgroup g done with phase k of
        layer l, e = 1 past the grid barrier after it); ``None`` stops it."""
        if buf is None:
            self._pf_trace_ptr = None
            return
        need = self.num_layers * 18 * torch.cuda.get_device_properties(self.device).multi_processor_count
        if buf.dtype != torch.int64 or buf.numel() < need or buf.device != self.device or not buf.is_contiguous():
            raise ValueError(f"prefill trace buffer must be a contiguous int64 tensor of >= {need} entries on {self.device}")
        self._pf_trace_buf = buf
        self._pf_trace_ptr = buf.data_ptr()

    def _generate_one_launch(self, ids, n_tokens):
        """mq_int8/int4/bf16/fp8_decode_generate; None when no multi-step kernel covers the request."""
        if self._inflight:
            torch.cuda.current_stream(self.device).synchronize()
            self._inflight.clear()
        # pinned output words, kept between calls (allocating pinned memory costs about a
        # decode step's time); each call ends synchronised, so the buffer is free here
        if getattr(self, "_gen_out", None) is None or self._gen_out.numel() < n_tokens:
            self._gen_out = torch.empty(max(n_tokens, 256), dtype=torch.int32, pin_memory=True)
        out = self._gen_out[:n_tokens]
        out.fill_(TOKEN_PENDING)
        prompt = (ctypes.c_int * len(ids))(*ids)
        a = self._args
        a.input_token_id = ids[0]
        a.position = self._pos
        a.cache_len = self._pos + 1
        a.output_token_id = self.output_token.data_ptr()
        self._tok_host[0] = TOKEN_PENDING
        g = _lib.GenerateArgs(ctypes.cast(prompt, ctypes.c_void_p), len(ids), n_tokens, out.data_ptr())
        fn = (self._lib.mq_fp8_decode_generate if self._fp8 else
              self._lib.mq_int4_decode_generate if self._int4 else
              self._lib.mq_int8_decode_generate if self._int8 else self._lib.mq_bf16_decode_generate)
        st = fn(ctypes.byref(a), ctypes.byref(g), ctypes.c_void_p(_lib.stream_handle(self.device)))
        if st == _lib.MQ_ERR_UNSUPPORTED:
            return None
        _lib.check(st, "decode generate")
        torch.cuda.current_stream(self.device).synchronize()
        toks = out.tolist()
        if min(toks) < 0:
            status = self._lib.mq_decode_check(self.workspace.data_ptr(),
                                               ctypes.c_void_p(_lib.stream_handle(self.device)))
            self._init_workspace()
            _lib.check(status if status != _lib.MQ_OK else _lib.MQ_ERR_TIMEOUT, "decode generate")
        self._pos += len(ids) + n_tokens - 1
        return toks

    def set_attn_split(self, min_len: int) -> None:
        """Context length from which the XCD-aware kernel splits each KV head's attention
        over its 32 workgroups (0 = library default, negative = never; the unsplit
        path attends over at most 1024 positions)."""
        self._args.attn_split_min = int(min_len)

    def prefill_random_kv(self, depth: int, seed: int = 0) -> None:
        """Long-context set-up (the reference has no counterpart):
        K and V cache rows of positions [0, depth) of every layer and KV head become
        seeded N(0, 1) values rounded to bf16, later rows zero, and the next step
        decodes at position ``depth``. The rows come from a generator on the
        decoder's device seeded with ``seed``, one layer at a time."""
        if not isinstance(depth, int) or not 0 <= depth < self.max_seq_len:
            raise ValueError(f"depth {depth!r} outside [0, {self.max_seq_len})")
        g = torch.Generator(device=self.device)
        g.manual_seed(int(seed))
        shape = (self.k_cache.shape[1], depth, self.k_cache.shape[3])
        with torch.cuda.device(self.device):
            for cache in (self.k_cache, self.v_cache):
                cache.zero_()
                for l in range(self.num_layers):
                    cache[l, :, :depth].copy_(torch.randn(shape, generator=g, device=self.device,
                                                          dtype=torch.float32))
        self._pos = depth

    # debug getters (run_benchmark.py:174-183): the last layer's values after a step,
    # filled while enable_debug() is on
    def get_hidden(self): return self.hidden_buffer
    def get_activations(self): return self.g_activations
    def get_residual(self): return self.g_residual
    def get_q(self): return self.g_q
    def get_k(self): return self.g_k
    def get_v(self): return self.g_v
    def get_attn_out(self): return self.g_attn_out
    def get_mlp_int(self): return self.g_mlp_intermediate
    def get_normalized(self): return self.g_normalized


class A10Int8MegakernelDecoder(_DecoderBase):
    """bench_int8.py:121-130 constructor: (embed_weight, layer_weights_flat,
    layer_scales_all, lm_head_int8, lm_head_scale, final_norm_weight,
    cos_table, sin_table, num_layers, max_seq_len)."""

    _int8 = True

    def __init__(self, embed_weight, layer_weights_flat, layer_scales_all, lm_head_int8, lm_head_scale,
                 final_norm_weight, cos_table, sin_table, num_layers, max_seq_len):
        self._setup(embed_weight, layer_weights_flat, final_norm_weight, lm_head_int8, cos_table, sin_table,
                    num_layers, max_seq_len, layer_scales=layer_scales_all, lm_head_scale=lm_head_scale)


class A10Fp8MegakernelDecoder(_DecoderBase):
    """FP8 E4M3 weights (no counterpart in the reference, which has INT8 and BF16):
    the constructor of A10Int8MegakernelDecoder with every linear and the LM head
    given as FP8 codes (uint8 [out, in], from ``quantize_fp8``) and their per-row
    fp32 scales, in the same packing order. Hidden 1024 / intermediate 3072; one
    launch of the XCD-aware kernel per step (mq_fp8_decode_step)."""

    _int8 = True
    _fp8 = True

    def __init__(self, embed_weight, layer_weights_flat, layer_scales_all, lm_head_fp8, lm_head_scale,
                 final_norm_weight, cos_table, sin_table, num_layers, max_seq_len):
        self._setup(embed_weight, layer_weights_flat, final_norm_weight, lm_head_fp8, cos_table, sin_table,
                    num_layers, max_seq_len, layer_scales=layer_scales_all, lm_head_scale=lm_head_scale)


class A10Int4MegakernelDecoder(_DecoderBase):
    """INT4 weights per group of 128 inputs (no counterpart in the reference, which has
    INT8 and BF16): the constructor of A10Int8MegakernelDecoder with the seven layer
    projections given as packed nibbles (uint8 [out, in / 2], from ``quantize_int4``) and
    their fp32 group scales ([out, in / 128]) in the same packing order, and the LM head
    INT8 per row (``quantize_state(..., weight_format="int4")`` + ``pack_int8``). Hidden
    1024 / intermediate 3072 up to 10240 positions, on the async-wave kernel
    (mq_int4_decode_step; one launch for a whole generation with
    mq_int4_decode_generate). No batched prefill (prompts run as decode steps)."""

    _int8 = True
    _int4 = True

    def __init__(self, embed_weight, layer_weights_flat, layer_scales_all, lm_head_int8, lm_head_scale,
                 final_norm_weight, cos_table, sin_table, num_layers, max_seq_len):
        self._setup(embed_weight, layer_weights_flat, final_norm_weight, lm_head_int8, cos_table, sin_table,
                    num_layers, max_seq_len, layer_scales=layer_scales_all, lm_head_scale=lm_head_scale)


class A10MegakernelDecoder(_DecoderBase):
    """a10_decode.py:89-98 constructor: (embed_weight, layer_weights_flat,
    final_norm_weight, lm_head_weight, cos_table, sin_table, num_layers, max_seq_len)."""

    _int8 = False

    def __init__(self, embed_weight, layer_weights_flat, final_norm_weight, lm_head_weight, cos_table,
                 sin_table, num_layers, max_seq_len):
        self._setup(embed_weight, layer_weights_flat, final_norm_weight, lm_head_weight, cos_table, sin_table,
                    num_layers, max_seq_len)


class A10Int8BatchDecoder(_DecoderBase):
    """Batched INT8 decode (the reference has no batched path):
    ``batch`` independent sequences share one pass over the weights per step, each
    with its own KV cache and position. Constructor arguments are those of
    A10Int8MegakernelDecoder plus ``batch`` (1..16); Qwen3-1.7B layer shapes only.

    ``decode_step(tokens)`` feeds one token per sequence and returns the next
    greedy token of each. The matrix products run on the int8 matrix cores with
    28-bit activations (four int8 digits) and the RMSNorm scale applied after the
    product, so results agree with the single-sequence path within bf16 rounding
    of intermediate values rather than bitwise."""

    def __init__(self, embed_weight, layer_weights_flat, layer_scales_all, lm_head_int8, lm_head_scale,
                 final_norm_weight, cos_table, sin_table, num_layers, max_seq_len, batch):
        if not isinstance(batch, int) or not 1 <= batch <= _lib.MAX_BATCH:
            raise ValueError(f"batch must be an int in [1, {_lib.MAX_BATCH}], got {batch!r}")
        self._hold_weights(embed_weight, layer_weights_flat, final_norm_weight, lm_head_int8, cos_table, sin_table,
                           num_layers, max_seq_len, layer_scales_all, lm_head_scale)
        H, I, V = self.dims
        if (H, I) != (2048, 6144):
            raise ValueError(f"the batched kernel is compiled for hidden 2048 / intermediate 6144, got {H} / {I}")
        if max_seq_len > 1024:
            raise ValueError(f"max_seq_len {max_seq_len} > 1024: the batched path attends within one workgroup")
        dev = self.device
        self.batch = batch
        D = 128
        self.k_cache = torch.zeros((batch, num_layers, 8, max_seq_len, D), dtype=torch.bfloat16, device=dev)
        self.v_cache = torch.zeros_like(self.k_cache)
        self.output_tokens = torch.zeros(batch, dtype=torch.int32, pin_memory=True)   # written by the kernel
        self.hidden_buffer = torch.zeros((batch, H), dtype=torch.bfloat16, device=dev)
        f32 = dict(dtype=torch.float32, device=dev)
        self.qkv_buffer = torch.zeros((batch, 8, 512), **f32)
        self.attn_buffer = torch.zeros((batch, 16 * D), **f32)
        self.act_buffer = torch.zeros((batch, H), **f32)
        self.mlp_buffer = torch.zeros((batch, I), **f32)
        self._lib = _lib.load()
        self._dims = _lib.ModelDims(H, I, 16, 8, D, V)
        ws_bytes = self._lib.mq_batch_workspace_bytes(ctypes.byref(self._dims))
        if ws_bytes == 0:
            raise ValueError(f"unsupported model dims H={H} I={I}: {_lib.last_error()}")
        self.workspace = torch.empty(ws_bytes, dtype=torch.uint8, device=dev)
        self._init_workspace()
        a = _lib.BatchArgs()
        a.batch = batch
        a.output_token_ids = self.output_tokens.data_ptr()
        a.embed_weight = self.embed_weight.data_ptr()
        a.layer_weights = self.d_layer_weights.data_ptr()
        a.scales = self.d_layer_scales.data_ptr()
        a.final_norm_weight = self.final_norm_weight.data_ptr()
        a.lm_head_weight = self.lm_head_weight.data_ptr()
        a.lm_head_scale = self.lm_head_scale.data_ptr()
        a.cos_table, a.sin_table = self.cos_table.data_ptr(), self.sin_table.data_ptr()
        a.k_cache, a.v_cache = self.k_cache.data_ptr(), self.v_cache.data_ptr()
        a.num_layers = num_layers
        a.max_seq_len = max_seq_len
        a.attn_scale = self.attn_scale
        a.dims = ctypes.addressof(self._dims)
        a.workspace = self.workspace.data_ptr()
        a.workspace_bytes = ws_bytes
        self._args = a
        self._positions = [0] * batch
        self._inflight = None        # positions before the launched, not yet collected step

    def launch_step(self, tokens) -> None:
        """Enqueue one step (one token per sequence) on the current stream. A step still
        in flight is collected first (its tokens are dropped): the token words are reused."""
        if self._inflight is not None:
            self.wait_tokens()
        tokens = [int(t) for t in tokens]
        if len(tokens) != self.batch:
            raise ValueError(f"expected {self.batch} tokens, got {len(tokens)}")
        V = self.dims[2]
        for b, t in enumerate(tokens):
            if not 0 <= t < V:
                raise ValueError(f"sequence {b}: token {t} outside [0, {V})")
            if self._positions[b] >= self.max_seq_len:
                raise ValueError(f"sequence {b}: KV cache full at position {self._positions[b]}")
        a = self._args
        for b in range(self.batch):
            a.input_token_ids[b] = tokens[b]
            a.positions[b] = self._positions[b]
        # a step that returns before its token stores (an early exit of the kernel) leaves the
        # sentinel in place, which wait_tokens reports as a failure
        self.output_tokens.fill_(TOKEN_PENDING)
        st = self._lib.mq_int8_decode_batch_step(ctypes.byref(a), ctypes.c_void_p(_lib.stream_handle(self.device)))
        _lib.check(st, "batched decode step")
        self._inflight = list(self._positions)
        self._positions = [p + 1 for p in self._positions]

    def wait_tokens(self) -> list:
        """Wait for the last enqueued step and return its tokens. A failed step (MQTimeoutError)
        is undone: positions go back to the step's own and the workspace is re-initialised, so
        the same tokens can be fed again."""
        if self._inflight is None:
            raise RuntimeError("no batched step in flight (call launch_step first)")
        torch.cuda.current_stream(self.device).synchronize()
        out = self.output_tokens.tolist()
        before, self._inflight = self._inflight, None
        if min(out) < 0:
            self._positions = before
            status = self._lib.mq_decode_check(self.workspace.data_ptr(),
                                               ctypes.c_void_p(_lib.stream_handle(self.device)))
            self._init_workspace()
            _lib.check(status if status != _lib.MQ_OK else _lib.MQ_ERR_TIMEOUT, "batched decode step")
        return out

    def decode_step(self, tokens) -> list:
        self.launch_step(tokens)
        return self.wait_tokens()

    def reset(self) -> None:
        if self._inflight is not None:
            torch.cuda.current_stream(self.device).synchronize()
            self._inflight = None
        self._positions = [0] * self.batch
        self.k_cache.zero_()
        self.v_cache.zero_()

    def positions(self) -> list:
        return list(self._positions)

    def position(self) -> int:
        return self._positions[0]

    def set_timing_events(self, start=None, stop=None) -> None:
        if start is None or stop is None:
            self._args.timing_start = None
            self._args.timing_stop = None
            return
        for e in (start, stop):
            if e.cuda_event == 0:
                e.record()
        self._args.timing_start = start.cuda_event
        self._args.timing_stop = stop.cuda_event

    def set_spin_limit(self, polls: int) -> None:
        self._args.spin_limit = int(polls)

    def enable_debug(self, on: bool = True) -> None:
        """Write each sequence's last-layer values on every following step: ``get_hidden()``
        (bf16 [batch, H]), ``get_qkv()`` ([batch, 8, 512]: per KV head the two query heads,
        key and value before QK-norm), ``get_attn_out()``, ``get_activations()`` (the
        post-attention residual) and ``get_mlp_int()``."""
        a = self._args
        for f, t in (("hidden_out", self.hidden_buffer), ("qkv_out", self.qkv_buffer),
                     ("attn_out", self.attn_buffer), ("act_out", self.act_buffer), ("mlp_out", self.mlp_buffer)):
            setattr(a, f, t.data_ptr() if on else None)

    def set_trace(self, buf) -> None:
        """Record a per-stage timeline of every following step into ``buf`` (int64, at least
        ``(num_layers + 1) * 10 * 256`` entries on the decoder's device); ``None`` stops it."""
        if buf is None:
            self._args.trace = None
            return
        need = (self.num_layers + 1) * 10 * 256
        if buf.dtype != torch.int64 or buf.numel() < need or buf.device != self.device or not buf.is_contiguous():
            raise ValueError(f"trace buffer must be a contiguous int64 tensor of >= {need} entries on {self.device}")
        self._trace_buf = buf
        self._args.trace = buf.data_ptr()

    def get_hidden(self): return self.hidden_buffer
    def get_qkv(self): return self.qkv_buffer
    def get_attn_out(self): return self.attn_buffer
    def get_activations(self): return self.act_buffer
    def get_mlp_int(self): return self.mlp_buffer


def load_checkpoint_state(model_path, cfg: ModelConfig) -> dict:
    """bf16 state dict from a local HF safetensors checkpoint directory (no network),
    as the reference's ``_load_model`` takes it from the HF model (a10_decode.py:281-325):
    every tensor of every ``*.safetensors`` file (shards merged) in bf16; ``lm_head.weight``
    the embedding when the checkpoint ties it (absent key); a missing ``q_norm`` /
    ``k_norm`` gain becomes ones (a10_decode.py:304-309). A missing projection, layer
    norm, embedding or final norm raises ``KeyError`` naming the key."""
    from safetensors.torch import load_file
    path = Path(model_path)
    files = sorted(path.glob("*.safetensors"))
    if not files:
        raise FileNotFoundError(f"no *.safetensors under {path}")
    state = {}
    for f in files:
        state.update({k: v.to(torch.bfloat16) for k, v in load_file(str(f)).items()})
    if "lm_head.weight" not in state and "model.embed_tokens.weight" in state:
        state["lm_head.weight"] = state["model.embed_tokens.weight"]
    for i in range(cfg.num_layers):
        p = f"model.layers.{i}.self_attn"
        state.setdefault(f"{p}.q_norm.weight", torch.ones(cfg.head_dim, dtype=torch.bfloat16))
        state.setdefault(f"{p}.k_norm.weight", torch.ones(cfg.head_dim, dtype=torch.bfloat16))
    need = ["model.embed_tokens.weight", "model.norm.weight", "lm_head.weight"]
    for i in range(cfg.num_layers):
        p = f"model.layers.{i}"
        need += [f"{p}.input_layernorm.weight", f"{p}.post_attention_layernorm.weight"]
        need += [f"{p}.{proj}.weight" for proj in ("self_attn.q_proj", "self_attn.k_proj", "self_attn.v_proj",
                                                    "self_attn.o_proj", "mlp.gate_proj", "mlp.up_proj",
                                                    "mlp.down_proj")]
    for k in need:
        if k not in state:
            raise KeyError(f"checkpoint {path} has no tensor {k!r}")
    return state


def config_from_checkpoint(model_path, default: ModelConfig) -> ModelConfig:
    """The model shape of a checkpoint directory: HF ``config.json`` fields (layers, hidden
    and intermediate sizes, heads, head_dim, vocabulary, RMSNorm eps, RoPE theta) over
    ``default``; ``default`` itself when the directory has no ``config.json`` (the
    reference hard-codes Qwen3-0.6B, a10_decode.py:22-31)."""
    import json
    f = Path(model_path) / "config.json"
    if not f.exists():
        return default
    c = json.loads(f.read_text())
    keys = {"num_hidden_layers": "num_layers", "hidden_size": "hidden_size",
            "intermediate_size": "intermediate_size", "num_attention_heads": "num_q_heads",
            "num_key_value_heads": "num_kv_heads", "head_dim": "head_dim", "vocab_size": "vocab_size",
            "rms_norm_eps": "rms_eps", "rope_theta": "rope_theta", "tie_word_embeddings": "tie_word_embeddings"}
    kw = {ours: c[theirs] for theirs, ours in keys.items() if theirs in c}
    return default.with_(name=c.get("_name_or_path", Path(model_path).name) or default.name, **kw)


def load_tokenizer(model_path):
    """The checkpoint's tokenizer (``AutoTokenizer``, local files only), or None when the
    directory holds none that transformers can load."""
    try:
        from transformers import AutoTokenizer
        return AutoTokenizer.from_pretrained(str(model_path), local_files_only=True)
    except Exception:
        return None


class A10Decoder:
    """a10_decode.py:35-393. ``A10Decoder(model_path, max_seq_len)`` loads a
    local checkpoint directory (safetensors weights, its ``config.json`` shape when
    present, its tokenizer when transformers can load one); ``A10Decoder(seed=0)``
    (or a missing ``model_path``) builds seeded random-init weights of ``config``.
    ``int8=True`` quantizes every linear and the LM head (bench_int8.py:27-55) and
    drives ``A10Int8MegakernelDecoder``; otherwise the bf16 ``A10MegakernelDecoder``."""

    def __init__(self, model_path=None, max_seq_len: int = 2048, *, seed: int | None = None,
                 config: ModelConfig = QWEN3_0_6B, int8: bool = False, device="cuda"):
        self.max_seq_len = max_seq_len
        self.device = torch.device(device)
        self.tokenizer = None
        if model_path is not None and Path(model_path).exists():
            config = config_from_checkpoint(model_path, config)
            state = load_checkpoint_state(model_path, config)
            self.tokenizer = load_tokenizer(model_path)
        else:
            if model_path is not None and seed is None:
                raise FileNotFoundError(f"checkpoint {model_path} not found (pass seed= for random weights)")
            state, _ = random_init_state(config, seed=0 if seed is None else seed)
        if (config.num_q_heads, config.num_kv_heads, config.head_dim, config.rms_eps) != (16, 8, 128, 1e-6):
            raise ValueError(f"the decode kernels are compiled for 16 query / 8 KV heads of 128 and RMSNorm eps "
                             f"1e-6, got {config.num_q_heads} / {config.num_kv_heads} heads of {config.head_dim}, "
                             f"eps {config.rms_eps}")
        self.config = config
        self.cos_table, self.sin_table = precompute_rope_freqs(config.head_dim, max_seq_len, config.rope_theta,
                                                               device=self.device)
        if int8:
            qstate = quantize_state(state, config, self.device)
            embed, layers, scales, lm_q, lm_s, fnorm = pack_int8(qstate, config)
            self._keep = (embed, layers, scales, lm_q, lm_s, fnorm)
            self.decoder = A10Int8MegakernelDecoder(embed, layers, scales, lm_q, lm_s, fnorm, self.cos_table,
                                                    self.sin_table, config.num_layers, max_seq_len)
        else:
            embed, layers, fnorm, lm = pack_bf16(state, config, self.device)
            self._keep = (embed, layers, fnorm, lm)
            self.decoder = A10MegakernelDecoder(embed, layers, fnorm, lm, self.cos_table, self.sin_table,
                                                config.num_layers, max_seq_len)

    def reset(self):
        self.decoder.reset()

    def generate(self, prompt, max_new_tokens: int = 128, temperature: float = 0.0, seed: int = 0,
                 device_loop: bool = True, batched_prefill: bool = True):
        """Generation from a string (needs a tokenizer) or a list of ids. The prompt is
        prefilled as by one decode step per token (INT8: all but its last token in one
        prompt-batched pass, ``batched_prefill``) and the last prompt token's decode step
        gives the first generated token (verify_correctness_a10.py:323-339; a10_decode.py:375
        re-feeds the last prompt token instead, which decodes it twice). ``temperature`` 0 is greedy; above 0 tokens
        are sampled from softmax(logits / temperature) with ``seed`` (the reference accepts
        a temperature and ignores it, a10_decode.py:358). Within the INT8 async-wave
        kernel's range every step runs in one launch (``device_loop``), else one launch per
        step; the tokens are the same. Generation stops after an EOS token when the
        tokenizer has one. Returns ``(text_or_ids, tok_per_s, per_token_ms)``: the prompt and
        generated tokens decoded as text without special tokens (a10_decode.py:387) for a
        string prompt, as ids for an id list; with one launch, per_token_ms holds the
        launch's average time per step."""
        if isinstance(prompt, str):
            if self.tokenizer is None:
                raise ValueError("a string prompt needs a checkpoint with a tokenizer; pass token ids")
            ids = self.tokenizer.encode(prompt)
        else:
            ids = [int(t) for t in prompt]
        if not ids:
            raise ValueError("empty prompt")
        if not isinstance(max_new_tokens, int) or max_new_tokens < 1:
            raise ValueError(f"max_new_tokens must be a positive int, got {max_new_tokens!r}")
        self.reset()
        self.decoder.set_sampling(temperature, seed)
        eos = getattr(self.tokenizer, "eos_token_id", None)
        torch.cuda.synchronize(self.device)
        t0 = time.perf_counter()
        toks = self.decoder.generate(ids, max_new_tokens, device_loop=device_loop, batched_prefill=batched_prefill)
        torch.cuda.synchronize(self.device)
        ms = (time.perf_counter() - t0) * 1e3
        if eos is not None and eos in toks:
            toks = toks[:toks.index(eos) + 1]
        steps = len(ids) + max_new_tokens - 1
        times = [ms / steps] * (len(toks) - 1)          # the steps after the first generated token
        tok_s = 1e3 * steps / ms if ms > 0 else 0.0
        generated = list(ids) + toks
        out = self.tokenizer.decode(generated, skip_special_tokens=True) if isinstance(prompt, str) else generated
        return out, tok_s, times
