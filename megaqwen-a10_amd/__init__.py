"""MI355X (gfx950) batch-1 decode for Qwen3-shaped models — drop-in for MegaQwen-A10's decode path.

Python host code on PyTorch-ROCm (device memory, streams) over a C-ABI HIP
library (``lib/libmegaqwen_a10.so``, declared in include/megaqwen_a10.h):

* ``quantize_per_channel`` — per-row symmetric INT8 (bench_int8.py:19-24), HIP kernel.
* ``int8_gemv`` — INT8 weight-only matvec (int8_decoder.py:100-115), HIP kernel;
  ``int8_gemv_repeat`` its steady-state form.
* ``quantize_fp8`` / ``quantize_int4`` / ``fp8_gemv`` / ``int4_gemv`` (+ ``_repeat``) —
  FP8 E4M3 per-row and INT4 per-group weights (no counterpart in the reference).
* ``A10Int8MegakernelDecoder`` / ``A10MegakernelDecoder`` / ``A10Decoder`` —
  the reference's decoder classes (bench_int8.py:119-255, a10_decode.py:35-393),
  one persistent-kernel launch per token.
* ``A10Fp8MegakernelDecoder`` / ``A10Int4MegakernelDecoder`` — the same step with FP8
  E4M3 weights, or INT4 weights per group of 128 (no counterpart in the reference).
* ``A10Chat`` — the reference's chat front end (a10_chat.py:222-604) over ``A10Decoder``:
  ChatML prompts, streamed replies, history; ``chat_prompt`` / ``clean_reply`` its host steps.
* ``A10Int8BatchDecoder`` — up to 16 independent sequences per step on the int8
  matrix cores (Qwen3-1.7B shapes; no counterpart in the reference).
* ``precompute_rope_freqs`` / ``make_rope`` — RoPE tables.
* ``random_init_state`` / ``quantize_state`` / ``pack_int8`` / ``pack_bf16`` —
  seeded weights and the reference's tensor packing.
"""
from . import chat
from .chat import A10Chat, chat_prompt, clean_reply
from .config import QWEN3_0_6B, QWEN3_1_7B, ModelConfig
from .decoder import (A10Decoder, A10Fp8MegakernelDecoder, A10Int4MegakernelDecoder, A10Int8BatchDecoder,
                      A10Int8MegakernelDecoder, A10MegakernelDecoder, config_from_checkpoint, decode_variant, load_checkpoint_state,
                      load_tokenizer, set_cooperative_launch, set_decode_variant)
from .formats import fp8_gemv, fp8_gemv_repeat, int4_gemv, int4_gemv_repeat, quantize_fp8, quantize_int4
from .gemv import int8_gemv, int8_gemv_repeat
from .quant import quantize_per_channel
from .rope import make_rope, precompute_rope_freqs
from .weights import pack_bf16, pack_int8, quantize_state, random_init_state, state_digest

__all__ = [
    "ModelConfig", "QWEN3_0_6B", "QWEN3_1_7B",
    "A10Chat", "chat_prompt", "clean_reply",
    "A10Decoder", "A10Fp8MegakernelDecoder", "A10Int4MegakernelDecoder", "A10Int8BatchDecoder", "A10Int8MegakernelDecoder", "A10MegakernelDecoder", "set_decode_variant",
    "decode_variant", "set_cooperative_launch", "config_from_checkpoint", "load_checkpoint_state", "load_tokenizer",
    "int8_gemv", "int8_gemv_repeat", "quantize_per_channel",
    "quantize_fp8", "quantize_int4", "fp8_gemv", "int4_gemv", "fp8_gemv_repeat", "int4_gemv_repeat", "make_rope", "precompute_rope_freqs",
    "pack_bf16", "pack_int8", "quantize_state", "random_init_state", "state_digest",
]
