"""ctypes binding of ``lib/libmegaqwen_a10.so`` (the C ABI in include/megaqwen_a10.h).

torch is imported first so that the library resolves ``libamdhip64.so.7`` to
the HIP runtime torch already loaded (one runtime per process, so device
pointers and streams from torch are valid in the library). There is no CPU
fallback: if the library is missing, every entry point raises.
"""
from __future__ import annotations

import ctypes
from ctypes import POINTER, Structure, c_float, c_int, c_int64, c_size_t, c_uint, c_void_p
from pathlib import Path

import torch  # noqa: F401  (must be loaded before the HIP library)

LIB_PATH = Path(__file__).resolve().parent / "lib" / "libmegaqwen_a10.so"

MQ_OK = 0
MQ_ERR_INVALID_ARGUMENT = 1
MQ_ERR_UNSUPPORTED = 2
MQ_ERR_HIP = 3
MQ_ERR_TIMEOUT = 4
MQ_ERR_OUT_OF_MEMORY = 5

LAYER_FIELDS = (
    "input_layernorm_weight", "q_proj_weight", "k_proj_weight", "v_proj_weight",
    "q_norm_weight", "k_norm_weight", "o_proj_weight", "post_attn_layernorm_weight",
    "gate_proj_weight", "up_proj_weight", "down_proj_weight",
)
SCALE_FIELDS = ("q_scale", "k_scale", "v_scale", "o_scale", "gate_scale", "up_scale", "down_scale")


class LayerWeights(Structure):
    """config.cuh:45-57 — 11 device pointers per layer."""
    _fields_ = [(n, c_void_p) for n in LAYER_FIELDS]


class ScalePointers(Structure):
    """config.cuh:59-67 — 7 fp32 scale vectors per layer."""
    _fields_ = [(n, c_void_p) for n in SCALE_FIELDS]


class ModelDims(Structure):
    _fields_ = [("hidden_size", c_int), ("intermediate_size", c_int), ("num_q_heads", c_int),
                ("num_kv_heads", c_int), ("head_dim", c_int), ("vocab_size", c_int)]


class DecodeArgs(Structure):
    _fields_ = [
        ("input_token_id", c_int), ("output_token_id", c_void_p),
        ("embed_weight", c_void_p), ("layer_weights", c_void_p), ("scales", c_void_p),
        ("final_norm_weight", c_void_p), ("lm_head_weight", c_void_p), ("lm_head_scale", c_void_p),
        ("cos_table", c_void_p), ("sin_table", c_void_p), ("k_cache", c_void_p), ("v_cache", c_void_p),
        ("hidden_buffer", c_void_p), ("g_activations", c_void_p), ("g_residual", c_void_p),
        ("g_q", c_void_p), ("g_k", c_void_p), ("g_v", c_void_p), ("g_attn_out", c_void_p),
        ("g_mlp_intermediate", c_void_p), ("g_normalized", c_void_p),
        ("block_max_vals", c_void_p), ("block_max_idxs", c_void_p),
        ("num_layers", c_int), ("position", c_int), ("cache_len", c_int), ("max_seq_len", c_int),
        ("attn_scale", c_float), ("dims", c_void_p), ("workspace", c_void_p),
        ("workspace_bytes", c_size_t), ("spin_limit", c_uint),
        ("timing_start", c_void_p), ("timing_stop", c_void_p), ("trace", c_void_p),
        ("attn_split_min", c_int),
        ("temperature", c_float), ("seed", ctypes.c_ulonglong),
    ]


class GenerateArgs(Structure):
    """mq_generate_args: several decode steps in one launch."""
    _fields_ = [("prompt_tokens", c_void_p), ("n_forced", c_int), ("n_generate", c_int), ("output_tokens", c_void_p)]


MAX_BATCH = 16


class BatchArgs(Structure):
    _fields_ = [
        ("batch", c_int), ("input_token_ids", c_int * MAX_BATCH), ("positions", c_int * MAX_BATCH),
        ("output_token_ids", c_void_p),
        ("embed_weight", c_void_p), ("layer_weights", c_void_p), ("scales", c_void_p),
        ("final_norm_weight", c_void_p), ("lm_head_weight", c_void_p), ("lm_head_scale", c_void_p),
        ("cos_table", c_void_p), ("sin_table", c_void_p), ("k_cache", c_void_p), ("v_cache", c_void_p),
        ("num_layers", c_int), ("max_seq_len", c_int), ("attn_scale", c_float), ("dims", c_void_p),
        ("workspace", c_void_p), ("workspace_bytes", c_size_t), ("spin_limit", c_uint),
        ("timing_start", c_void_p), ("timing_stop", c_void_p), ("hidden_out", c_void_p),
        ("qkv_out", c_void_p), ("attn_out", c_void_p), ("act_out", c_void_p), ("mlp_out", c_void_p),
        ("trace", c_void_p),
    ]


assert ctypes.sizeof(LayerWeights) == 88 and ctypes.sizeof(ScalePointers) == 56


class MQError(RuntimeError):
    def __init__(self, status: int, message: str):
        super().__init__(f"[status {status}] {message}")
        self.status = status


class MQTimeoutError(MQError):
    pass


# Public C symbols and their signatures; the tests check the header declares exactly these.
_SIGNATURES = {
    "mq_abi_version": (c_int, []),
    "mq_last_error": (ctypes.c_char_p, []),
    "mq_decode_workspace_bytes": (c_size_t, [c_void_p]),
    "mq_workspace_init": (c_int, [c_void_p, c_size_t, c_void_p]),
    "mq_int8_decode_step": (c_int, [POINTER(DecodeArgs), c_void_p]),
    "mq_fp8_decode_step": (c_int, [POINTER(DecodeArgs), c_void_p]),
    "mq_int4_decode_step": (c_int, [POINTER(DecodeArgs), c_void_p]),
    "mq_bf16_decode_step": (c_int, [POINTER(DecodeArgs), c_void_p]),
    "mq_int8_decode_step_noalloc": (c_int, [POINTER(DecodeArgs), c_void_p]),
    "mq_int8_decode_generate": (c_int, [POINTER(DecodeArgs), POINTER(GenerateArgs), c_void_p]),
    "mq_bf16_decode_generate": (c_int, [POINTER(DecodeArgs), POINTER(GenerateArgs), c_void_p]),
    "mq_fp8_decode_generate": (c_int, [POINTER(DecodeArgs), POINTER(GenerateArgs), c_void_p]),
    "mq_int4_decode_generate": (c_int, [POINTER(DecodeArgs), POINTER(GenerateArgs), c_void_p]),
    "mq_prefill_workspace_bytes": (c_size_t, [POINTER(ModelDims), c_int]),
    "mq_int8_prefill": (c_int, [POINTER(DecodeArgs), c_void_p, c_int, c_void_p, c_size_t, c_void_p]),
    "mq_prefill_check": (c_int, [c_void_p, c_size_t, c_void_p]),
    "mq_decode_check": (c_int, [c_void_p, c_void_p]),
    "mq_wait_host_token": (c_int, [c_void_p, c_int, c_uint]),
    "mq_decode_set_variant": (c_int, [c_int]),
    "mq_decode_set_cooperative": (c_int, [c_int]),
    "mq_decode_variant": (c_int, [c_void_p, c_int]),
    "mq_decode_variant_at": (c_int, [c_void_p, c_int, c_int]),
    "mq_batch_workspace_bytes": (c_size_t, [c_void_p]),
    "mq_int8_decode_batch_step": (c_int, [POINTER(BatchArgs), c_void_p]),
    "launch_a10_int8_decode": (None, [c_int, c_void_p] + [c_void_p] * 20 + [c_int] * 4 + [c_float, c_void_p, c_void_p]),
    "launch_a10_decode": (None, [c_int, c_void_p] + [c_void_p] * 19 + [c_int] * 4 + [c_float, c_void_p]),
    "mq_reference_set_spin_limit": (None, [c_uint]),
    "mq_reference_set_dims": (c_int, [c_void_p]),
    "mq_int8_gemv": (c_int, [c_void_p, c_void_p, c_void_p, c_void_p, c_int, c_int, c_void_p]),
    "mq_int8_gemv_repeat": (c_int, [c_void_p, c_void_p, c_int64, c_int, c_void_p, c_void_p, c_int, c_int, c_int,
                                    c_void_p]),
    "mq_quantize_fp8_rows_bf16": (c_int, [c_void_p, c_int, c_int, c_void_p, c_void_p, c_void_p]),
    "mq_quantize_int4_groups_bf16": (c_int, [c_void_p, c_int, c_int, c_void_p, c_void_p, c_void_p]),
    "mq_fp8_gemv": (c_int, [c_void_p, c_void_p, c_void_p, c_void_p, c_int, c_int, c_void_p]),
    "mq_int4_gemv": (c_int, [c_void_p, c_void_p, c_void_p, c_void_p, c_int, c_int, c_void_p]),
    "mq_fp8_gemv_repeat": (c_int, [c_void_p, c_void_p, c_int64, c_int, c_void_p, c_void_p, c_int, c_int, c_int,
                                   c_void_p]),
    "mq_int4_gemv_repeat": (c_int, [c_void_p, c_void_p, c_int64, c_int, c_void_p, c_void_p, c_int, c_int, c_int,
                                    c_void_p]),
    "mq_quantize_per_channel_bf16": (c_int, [c_void_p, c_int, c_int, c_void_p, c_void_p, c_void_p]),
}
EXPORTED = tuple(_SIGNATURES)

_lib = None


def load() -> ctypes.CDLL:
    """Load the HIP library (raises if it has not been built)."""
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise RuntimeError(f"{LIB_PATH} is missing: build it with `python megaqwen-a10_amd/build.py` "
                               "(the library has no CPU fallback)")
        lib = ctypes.CDLL(str(LIB_PATH))
        for name, (res, args) in _SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = args
        _lib = lib
    return _lib


def last_error() -> str:
    return load().mq_last_error().decode(errors="replace")


def check(status: int, what: str) -> None:
    if status != MQ_OK:
        cls = MQTimeoutError if status == MQ_ERR_TIMEOUT else MQError
        raise cls(status, f"{what}: {last_error()}")


def stream_handle(device=None) -> int:
    """The raw hipStream_t of torch's current stream on ``device`` (default: the current
    device). Read without building a torch Stream object: this sits on every decode step's
    host path, where ``torch.cuda.current_stream(device).cuda_stream`` costs about 2 us."""
    if _raw_stream is None:                 # a torch without the raw accessor
        return torch.cuda.current_stream(device).cuda_stream
    if device is None:
        idx = torch.cuda.current_device()
    elif isinstance(device, int):
        idx = device
    else:
        idx = device.index if device.index is not None else torch.cuda.current_device()
    return _raw_stream(idx)


_raw_stream = getattr(torch._C, "_cuda_getCurrentRawStream", None)
