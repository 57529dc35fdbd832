"""Free-function decode surface of the reference's chat program (a10_chat.py:84-189).

The reference compiles a module with three functions and keeps the model in
module state (one model per process):

* ``init_ldg_layer_weights(input_layernorm_weights, q_proj_weights, ...,
  down_proj_weights)`` (a10_chat.py:84-116): eleven lists of per-layer bf16
  tensors, turned into the device ``LayerWeights[L]`` array;
* ``init_ldg_embed_weight(embed_weight)`` (a10_chat.py:118-120);
* ``decode_a10(input_token_id, final_norm_weight, lm_head_weight, cos_table,
  sin_table, k_cache, v_cache, hidden_buffer, g_activations, g_residual, g_q,
  g_k, g_v, g_attn_out, g_mlp_intermediate, g_normalized, block_max_vals,
  block_max_idxs, num_layers, position, cache_len, max_seq_len) -> int``
  (a10_chat.py:122-182): one bf16 decode step on the caller's KV cache and
  scratch, on the current stream, waited for; returns the greedy token.

This module is that surface over the gfx950 library: ``decode_a10`` runs the
BF16 step entry point (``mq_bf16_decode_step``) with attn_scale 1/sqrt(128)
as the reference does. Differences, all on the side of failing loudly: the
reference keeps only raw pointers to the layer tensors and the embedding (the
caller must keep them alive); this module holds references to them. The
reference checks nothing; here a call before the init functions, tensors of
the wrong dtype, shape or device, a token outside the vocabulary or a position
outside the cache raise ``RuntimeError``/``TypeError``/``ValueError`` before
anything is launched, and a failed step raises ``MQError``. The library also
needs a workspace of its own for its exchanges, which the first ``decode_a10``
allocates on the weights' device.
"""
from __future__ import annotations

import ctypes
import math

import torch

from . import _lib
from .decoder import LM_PARTIALS, _check_tensor, _device_array

_FIELDS = ("input_layernorm_weights", "q_proj_weights", "k_proj_weights", "v_proj_weights", "q_norm_weights",
           "k_norm_weights", "o_proj_weights", "post_attn_layernorm_weights", "gate_proj_weights",
           "up_proj_weights", "down_proj_weights")


class _State:
    layers = None           # per-layer tuples of the 11 tensors, in LayerWeights order
    d_layer_weights = None  # device LayerWeights[L]
    embed = None
    device = None
    hidden = None
    inter = None
    workspace = None        # the library's exchange workspace, sized at the first step


_state = _State()


def init_ldg_layer_weights(input_layernorm_weights, q_proj_weights, k_proj_weights, v_proj_weights,
                           q_norm_weights, k_norm_weights, o_proj_weights, post_attn_layernorm_weights,
                           gate_proj_weights, up_proj_weights, down_proj_weights) -> None:
    """Build the device LayerWeights array from eleven per-layer lists of bf16
    tensors (a10_chat.py:84-116); replaces the model of an earlier call."""
    lists = (input_layernorm_weights, q_proj_weights, k_proj_weights, v_proj_weights, q_norm_weights,
             k_norm_weights, o_proj_weights, post_attn_layernorm_weights, gate_proj_weights, up_proj_weights,
             down_proj_weights)
    L = len(lists[0])
    if L < 1:
        raise ValueError("init_ldg_layer_weights: no layers")
    for name, lst in zip(_FIELDS, lists):
        if len(lst) != L:
            raise ValueError(f"init_ldg_layer_weights: {name} has {len(lst)} tensors, "
                             f"{_FIELDS[0]} has {L}")
    t0 = lists[0][0]
    _check_tensor(t0, "input_layernorm_weights[0]", torch.bfloat16)
    dev = t0.device
    H = t0.shape[0]
    I = lists[8][0].shape[0] if lists[8][0].dim() == 2 else -1
    D = 128
    Q, KV = 16 * D, 8 * D
    shapes = [(H,), (Q, H), (KV, H), (KV, H), (D,), (D,), (H, Q), (H,), (I, H), (I, H), (H, I)]
    for f, (name, lst) in enumerate(zip(_FIELDS, lists)):
        for l, t in enumerate(lst):
            _check_tensor(t, f"{name}[{l}]", torch.bfloat16, shapes[f], dev)

    lw = (_lib.LayerWeights * L)()
    layers = []
    for l in range(L):
        row = tuple(lst[l] for lst in lists)
        for field, t in zip(_lib.LAYER_FIELDS, row):
            setattr(lw[l], field, t.data_ptr())
        layers.append(row)
    _state.layers = layers
    _state.d_layer_weights = _device_array(lw, dev)
    _state.device = dev
    _state.hidden, _state.inter = H, I
    _state.workspace = None
    if _state.embed is not None and _state.embed.device != dev:
        _state.embed = None


def init_ldg_embed_weight(embed_weight) -> None:
    """Set the embedding table, bf16 [vocab, hidden] (a10_chat.py:118-120)."""
    _check_tensor(embed_weight, "embed_weight", torch.bfloat16)
    if embed_weight.dim() != 2:
        raise ValueError("embed_weight must be [vocab, hidden]")
    _state.embed = embed_weight


def decode_a10(input_token_id, final_norm_weight, lm_head_weight, cos_table, sin_table, k_cache, v_cache,
               hidden_buffer, g_activations, g_residual, g_q, g_k, g_v, g_attn_out, g_mlp_intermediate,
               g_normalized, block_max_vals, block_max_idxs, num_layers, position, cache_len,
               max_seq_len) -> int:
    """One bf16 decode step of the initialised model at ``position`` over the
    caller's KV cache ([num_layers, 8, max_seq_len, 128] bf16 each); waits for it
    and returns the greedy token (a10_chat.py:122-182)."""
    if _state.layers is None or _state.embed is None:
        raise RuntimeError("decode_a10: call init_ldg_layer_weights and init_ldg_embed_weight first")
    dev, H, I = _state.device, _state.hidden, _state.inter
    if _state.embed.device != dev or _state.embed.shape[1] != H:
        raise ValueError(f"embed_weight {tuple(_state.embed.shape)} on {_state.embed.device} does not match "
                         f"the layers (hidden {H}, {dev})")
    V = _state.embed.shape[0]
    if not isinstance(num_layers, int) or not 1 <= num_layers <= len(_state.layers):
        raise ValueError(f"num_layers {num_layers!r} outside [1, {len(_state.layers)}]")
    if not isinstance(max_seq_len, int) or max_seq_len < 1:
        raise ValueError(f"max_seq_len must be a positive int, got {max_seq_len!r}")
    if not isinstance(position, int) or not 0 <= position < max_seq_len:
        raise ValueError(f"position {position!r} outside [0, {max_seq_len})")
    if cache_len != position + 1:
        raise ValueError(f"cache_len must be position + 1 = {position + 1}, got {cache_len!r}")
    if not isinstance(input_token_id, int) or not 0 <= input_token_id < V:
        raise ValueError(f"input_token_id {input_token_id!r} outside [0, {V})")
    D = 128
    _check_tensor(final_norm_weight, "final_norm_weight", torch.bfloat16, (H,), dev)
    _check_tensor(lm_head_weight, "lm_head_weight", torch.bfloat16, (V, H), dev)
    for name, t in (("cos_table", cos_table), ("sin_table", sin_table)):
        _check_tensor(t, name, torch.bfloat16, None, dev)
        if t.dim() != 2 or t.shape[1] != D or t.shape[0] < max_seq_len:
            raise ValueError(f"{name} must be [>= max_seq_len, {D}], got {tuple(t.shape)}")
    for name, t in (("k_cache", k_cache), ("v_cache", v_cache)):
        _check_tensor(t, name, torch.bfloat16, (num_layers, 8, max_seq_len, D), dev)
    f32 = torch.float32
    scratch = (("hidden_buffer", hidden_buffer, torch.bfloat16, H), ("g_activations", g_activations, f32, H),
               ("g_residual", g_residual, f32, H), ("g_q", g_q, f32, 16 * D), ("g_k", g_k, f32, 8 * D),
               ("g_v", g_v, f32, 8 * D), ("g_attn_out", g_attn_out, f32, 16 * D),
               ("g_mlp_intermediate", g_mlp_intermediate, f32, I), ("g_normalized", g_normalized, f32, H),
               ("block_max_vals", block_max_vals, f32, LM_PARTIALS),
               ("block_max_idxs", block_max_idxs, torch.int32, LM_PARTIALS))
    for name, t, dt, n in scratch:
        _check_tensor(t, name, dt, None, dev)
        if t.numel() < n:
            raise ValueError(f"{name}: needs at least {n} elements, has {t.numel()}")

    lib = _lib.load()
    dims = _lib.ModelDims(H, I, 16, 8, D, V)
    need = lib.mq_decode_workspace_bytes(ctypes.byref(dims))
    if need == 0:
        raise ValueError(f"unsupported model dims H={H} I={I} V={V}: {_lib.last_error()}")
    if _state.workspace is None or _state.workspace.numel() < need:
        _state.workspace = torch.empty(need, dtype=torch.uint8, device=dev)
        with torch.cuda.device(dev):
            _lib.check(lib.mq_workspace_init(_state.workspace.data_ptr(), need, _lib.stream_handle()),
                       "mq_workspace_init")
    out = torch.full((1,), -2, dtype=torch.int32, device=dev)
    a = _lib.DecodeArgs()
    a.input_token_id = input_token_id
    a.output_token_id = out.data_ptr()
    a.embed_weight = _state.embed.data_ptr()
    a.layer_weights = _state.d_layer_weights.data_ptr()
    a.final_norm_weight = final_norm_weight.data_ptr()
    a.lm_head_weight = lm_head_weight.data_ptr()
    a.cos_table, a.sin_table = cos_table.data_ptr(), sin_table.data_ptr()
    a.k_cache, a.v_cache = k_cache.data_ptr(), v_cache.data_ptr()
    for name, t, _, _ in scratch:
        setattr(a, name, t.data_ptr())
    a.num_layers = num_layers
    a.position = position
    a.cache_len = cache_len
    a.max_seq_len = max_seq_len
    a.attn_scale = 1.0 / math.sqrt(float(D))
    a.dims = ctypes.addressof(dims)
    a.workspace = _state.workspace.data_ptr()
    a.workspace_bytes = _state.workspace.numel()
    with torch.cuda.device(dev):
        stream = ctypes.c_void_p(_lib.stream_handle())
        _lib.check(lib.mq_bf16_decode_step(ctypes.byref(a), stream), "decode_a10")
        torch.cuda.current_stream().synchronize()
        tok = int(out.item())
        if tok < 0:
            status = lib.mq_decode_check(_state.workspace.data_ptr(), stream)
            _lib.check(lib.mq_workspace_init(_state.workspace.data_ptr(), _state.workspace.numel(), stream),
                       "mq_workspace_init")
            _lib.check(status if status != _lib.MQ_OK else _lib.MQ_ERR_TIMEOUT, "decode_a10")
    return tok
