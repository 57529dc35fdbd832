"""Host-side checks that need no GPU: the C-ABI library loads and exports what
include/megaqwen_a10.h declares, struct layouts agree between C and ctypes,
argument validation rejects bad inputs before any launch, byte accounting,
packing order, and the seeded weight generator."""
from __future__ import annotations

import ctypes
import re
import subprocess

import pytest
import torch

from .conftest import ROOT

HEADER = ROOT / "include" / "megaqwen_a10.h"


def header_functions():
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    names = re.findall(r"^\s*(?:const\s+)?[A-Za-z_][A-Za-z0-9_]*\s*\*?\s*([A-Za-z_][A-Za-z0-9_]*)\s*\(", text, flags=re.M)
    return sorted(set(n for n in names if n not in ("if", "sizeof")))


def test_library_exports_every_declared_symbol(mq):
    from megaqwen_a10_amd import _lib
    lib = _lib.load()
    declared = header_functions()
    assert sorted(_lib.EXPORTED) == declared
    for name in declared:
        assert hasattr(lib, name), name
    assert lib.mq_abi_version() == 3


def test_struct_layout_matches_c(tmp_path, mq):
    """offsetof() of every mq_decode_args field from a C program compiled against the header."""
    from megaqwen_a10_amd import _lib
    fields = [f for f, _ in _lib.DecodeArgs._fields_]
    src = ["#include <stdio.h>", "#include <stddef.h>", f'#include "{HEADER}"', "int main(void){"]
    src.append('printf("%zu %zu %zu %zu\\n", sizeof(LayerWeights), sizeof(ScalePointers), sizeof(mq_model_dims), sizeof(mq_decode_args));')
    for f in fields:
        src.append(f'printf("%zu\\n", offsetof(mq_decode_args, {f}));')
    src.append("return 0;}")
    c = tmp_path / "layout.c"
    c.write_text("\n".join(src))
    exe = tmp_path / "layout"
    subprocess.run(["gcc", "-std=c11", "-o", str(exe), str(c)], check=True)
    out = subprocess.run([str(exe)], capture_output=True, text=True, check=True).stdout.split()
    sizes = list(map(int, out[:4]))
    assert sizes == [ctypes.sizeof(_lib.LayerWeights), ctypes.sizeof(_lib.ScalePointers),
                     ctypes.sizeof(_lib.ModelDims), ctypes.sizeof(_lib.DecodeArgs)]
    assert sizes[:2] == [88, 56]
    offs = list(map(int, out[4:]))
    assert offs == [getattr(_lib.DecodeArgs, f).offset for f in fields]


def test_batch_struct_layout_matches_c(tmp_path, mq):
    """offsetof() of every mq_batch_args field from a C program compiled against the header."""
    from megaqwen_a10_amd import _lib
    fields = [f for f, _ in _lib.BatchArgs._fields_]
    src = ["#include <stdio.h>", "#include <stddef.h>", f'#include "{HEADER}"', "int main(void){"]
    src.append('printf("%zu %d\\n", sizeof(mq_batch_args), MQ_MAX_BATCH);')
    for f in fields:
        src.append(f'printf("%zu\\n", offsetof(mq_batch_args, {f}));')
    src.append("return 0;}")
    c = tmp_path / "blayout.c"
    c.write_text("\n".join(src))
    exe = tmp_path / "blayout"
    subprocess.run(["gcc", "-std=c11", "-o", str(exe), str(c)], check=True)
    out = list(map(int, subprocess.run([str(exe)], capture_output=True, text=True, check=True).stdout.split()))
    assert out[:2] == [ctypes.sizeof(_lib.BatchArgs), _lib.MAX_BATCH]
    assert out[2:] == [getattr(_lib.BatchArgs, f).offset for f in fields]


def test_generate_struct_layout_matches_c(tmp_path, mq):
    """offsetof() of every mq_generate_args field from a C program compiled against the header."""
    from megaqwen_a10_amd import _lib
    fields = [f for f, _ in _lib.GenerateArgs._fields_]
    src = ["#include <stdio.h>", "#include <stddef.h>", f'#include "{HEADER}"', "int main(void){"]
    src.append('printf("%zu\\n", sizeof(mq_generate_args));')
    for f in fields:
        src.append(f'printf("%zu\\n", offsetof(mq_generate_args, {f}));')
    src.append("return 0;}")
    c = tmp_path / "glayout.c"
    c.write_text("\n".join(src))
    exe = tmp_path / "glayout"
    subprocess.run(["gcc", "-std=c11", "-o", str(exe), str(c)], check=True)
    out = list(map(int, subprocess.run([str(exe)], capture_output=True, text=True, check=True).stdout.split()))
    assert out[0] == ctypes.sizeof(_lib.GenerateArgs)
    assert out[1:] == [getattr(_lib.GenerateArgs, f).offset for f in fields]


def test_generate_api_rejects_bad_arguments_without_launching(mq):
    """Host validation of mq_int8_decode_generate: NULLs, counts and prompt ids (no device needed)."""
    from megaqwen_a10_amd import _lib
    lib = _lib.load()
    a = _lib.DecodeArgs()
    g = _lib.GenerateArgs()
    assert lib.mq_int8_decode_generate(None, ctypes.byref(g), None) == _lib.MQ_ERR_INVALID_ARGUMENT
    assert lib.mq_int8_decode_generate(ctypes.byref(a), ctypes.byref(g), None) == _lib.MQ_ERR_INVALID_ARGUMENT
    prompt = (ctypes.c_int * 2)(1, 2)
    g = _lib.GenerateArgs(ctypes.cast(prompt, ctypes.c_void_p), 0, 4, 1234)
    for fn in (lib.mq_int8_decode_generate, lib.mq_int4_decode_generate, lib.mq_fp8_decode_generate,
               lib.mq_bf16_decode_generate):
        assert fn(ctypes.byref(a), ctypes.byref(g), None) == _lib.MQ_ERR_INVALID_ARGUMENT
        assert "n_forced" in _lib.last_error()
        assert fn(None, ctypes.byref(g), None) == _lib.MQ_ERR_INVALID_ARGUMENT


def test_cooperative_switch_is_host_only(mq):
    """mq_decode_set_cooperative only sets the launch mode (no device work, any value is 0/1)."""
    from megaqwen_a10_amd import _lib
    lib = _lib.load()
    assert lib.mq_decode_set_cooperative(1) == _lib.MQ_OK
    assert lib.mq_decode_set_cooperative(7) == _lib.MQ_OK
    assert lib.mq_decode_set_cooperative(0) == _lib.MQ_OK
    mq.set_cooperative_launch(False)


def test_variant_query_rejects_bad_arguments_without_launching(mq):
    """mq_decode_variant_at refuses a cache_len below 1 and dims without a kernel before it looks
    at the device (minus the status, as mq_decode_variant)."""
    from megaqwen_a10_amd import _lib
    lib = _lib.load()
    dims = _lib.ModelDims(1024, 3072, 16, 8, 128, 151936)
    for n in (0, -5):
        assert lib.mq_decode_variant_at(ctypes.byref(dims), 1, n) == -_lib.MQ_ERR_INVALID_ARGUMENT
        assert "cache_len" in _lib.last_error()
    bad = _lib.ModelDims(1000, 3072, 16, 8, 128, 151936)
    assert lib.mq_decode_variant_at(ctypes.byref(bad), 1, 10) == -_lib.MQ_ERR_UNSUPPORTED


def test_batch_api_rejects_bad_arguments_without_launching(mq):
    from megaqwen_a10_amd import _lib
    lib = _lib.load()
    assert lib.mq_batch_workspace_bytes(None) > 0
    assert lib.mq_batch_workspace_bytes(ctypes.byref(_lib.ModelDims(1024, 3072, 16, 8, 128, 151936))) == 0
    a = _lib.BatchArgs()
    a.num_layers, a.max_seq_len = 2, 64
    for bad in (0, 17):
        a.batch = bad
        assert lib.mq_int8_decode_batch_step(ctypes.byref(a), None) == _lib.MQ_ERR_INVALID_ARGUMENT
        assert "batch" in _lib.last_error()
    a.batch = 2
    a.input_token_ids[1] = 151936                              # == vocab
    assert lib.mq_int8_decode_batch_step(ctypes.byref(a), None) == _lib.MQ_ERR_INVALID_ARGUMENT
    assert "sequence 1" in _lib.last_error()
    a.input_token_ids[1] = 7
    a.positions[0] = 64                                        # == max_seq_len
    assert lib.mq_int8_decode_batch_step(ctypes.byref(a), None) == _lib.MQ_ERR_INVALID_ARGUMENT
    assert "position" in _lib.last_error()
    a.positions[0] = 3
    assert lib.mq_int8_decode_batch_step(ctypes.byref(a), None) == _lib.MQ_ERR_INVALID_ARGUMENT
    assert "null" in _lib.last_error()


def test_c_api_rejects_bad_arguments_without_launching(mq):
    from megaqwen_a10_amd import _lib
    lib = _lib.load()
    assert lib.mq_int8_gemv(None, None, None, None, 4, 16, None) == _lib.MQ_ERR_INVALID_ARGUMENT
    assert "NULL" in _lib.last_error()
    fake = ctypes.c_void_p(0x1000)
    assert lib.mq_int8_gemv(fake, fake, fake, fake, 4, 17, None) == _lib.MQ_ERR_INVALID_ARGUMENT
    # the steady-state form: copies, repetitions and the copy stride are checked before any launch
    bad = [(None, 0, 1, 4, 16, 1), (fake, 64, 0, 4, 16, 1), (fake, 64, 1, 4, 16, 0), (fake, 48, 2, 4, 16, 1),
           (fake, 72, 2, 4, 16, 1), (fake, 64, 1, 4, 17, 1), (fake, 64, 1, 2 ** 20, 16, 2 ** 12)]
    for w, stride, n, M, K, reps in bad:
        assert lib.mq_int8_gemv_repeat(fake, w, stride, n, fake, fake, M, K, reps, None) == \
            _lib.MQ_ERR_INVALID_ARGUMENT, (w, stride, n, M, K, reps)
    assert lib.mq_quantize_per_channel_bf16(fake, 0, 16, fake, fake, None) == _lib.MQ_ERR_INVALID_ARGUMENT
    # other weight formats: shapes, strides and group multiples are checked before any launch
    assert lib.mq_quantize_fp8_rows_bf16(None, 4, 16, fake, fake, None) == _lib.MQ_ERR_INVALID_ARGUMENT
    assert lib.mq_quantize_int4_groups_bf16(fake, 4, 100, fake, fake, None) == _lib.MQ_ERR_INVALID_ARGUMENT
    assert lib.mq_fp8_gemv(fake, fake, fake, fake, 4, 24, None) == _lib.MQ_ERR_INVALID_ARGUMENT
    assert lib.mq_int4_gemv(fake, fake, fake, fake, 4, 64, None) == _lib.MQ_ERR_INVALID_ARGUMENT
    assert lib.mq_int4_gemv(fake, fake, fake, fake, 4, 16384 + 128, None) == _lib.MQ_ERR_INVALID_ARGUMENT
    assert lib.mq_int4_gemv_repeat(fake, fake, 4 * 64 - 16, 2, fake, fake, 4, 128, 1, None) == \
        _lib.MQ_ERR_INVALID_ARGUMENT                                    # stride below one copy (M * K / 2)
    assert lib.mq_fp8_gemv_repeat(fake, fake, 64, 2, fake, fake, 4, 16, 0, None) == _lib.MQ_ERR_INVALID_ARGUMENT
    a = _lib.DecodeArgs()
    a.num_layers, a.max_seq_len, a.position, a.cache_len = 2, 16, 0, 1
    a.input_token_id = 151936                                  # == vocab: out of range
    assert lib.mq_int8_decode_step(ctypes.byref(a), None) == _lib.MQ_ERR_INVALID_ARGUMENT
    assert "input_token_id" in _lib.last_error()
    assert lib.mq_fp8_decode_step(ctypes.byref(a), None) == _lib.MQ_ERR_INVALID_ARGUMENT
    assert "input_token_id" in _lib.last_error()
    assert lib.mq_int4_decode_step(ctypes.byref(a), None) == _lib.MQ_ERR_INVALID_ARGUMENT
    assert "input_token_id" in _lib.last_error()
    a.input_token_id, a.position, a.cache_len = 5, 16, 17        # position == max_seq_len
    assert lib.mq_int8_decode_step(ctypes.byref(a), None) == _lib.MQ_ERR_INVALID_ARGUMENT
    assert "position" in _lib.last_error()
    a.position, a.cache_len = 3, 3                               # cache_len != position + 1
    assert lib.mq_int8_decode_step(ctypes.byref(a), None) == _lib.MQ_ERR_INVALID_ARGUMENT
    assert "cache_len" in _lib.last_error()
    a.cache_len = 4                                              # now only NULL pointers remain
    assert lib.mq_int8_decode_step(ctypes.byref(a), None) == _lib.MQ_ERR_INVALID_ARGUMENT
    d = _lib.ModelDims(1536, 4096, 16, 8, 128, 1000)
    assert lib.mq_decode_workspace_bytes(ctypes.byref(d)) == 0   # no kernel for this shape
    assert lib.mq_decode_workspace_bytes(None) > 0


def test_step_byte_accounting(mq):
    cfg = mq.QWEN3_0_6B
    # weights, scales and gains of one step: 28 layers x (15,728,640 B int8 + 49,152 B fp32 scales
    # + 4,608 B bf16 gains) + the 155,582,464 B int8 LM head, its 607,744 B of scales, the 2,048 B
    # final gain and one 2,048 B embedding row
    assert cfg.int8_step_bytes(cache_len=0) - 114688 == 598_101_504
    assert cfg.bf16_step_bytes(cache_len=0) - 114688 == 1_192_101_888
    assert cfg.int8_step_bytes(cache_len=10) - cfg.int8_step_bytes(cache_len=9) == 114_688


def test_packing_order_matches_reference(mq):
    """11 tensors per layer in LayerWeights order and 7 scales (bench_int8.py:291-330)."""
    cfg = mq.QWEN3_0_6B.with_(num_layers=2, vocab_size=64, hidden_size=8, intermediate_size=12)
    keys = {}
    q = {}
    tag = 0
    for i in range(cfg.num_layers):
        p = f"model.layers.{i}"
        for k in ("input_layernorm", "self_attn.q_norm", "self_attn.k_norm", "post_attention_layernorm"):
            tag += 1
            q[f"{p}.{k}.weight"] = torch.full((1,), float(tag))
            keys[tag] = f"{p}.{k}"
        for k in ("self_attn.q_proj", "self_attn.k_proj", "self_attn.v_proj", "self_attn.o_proj",
                  "mlp.gate_proj", "mlp.up_proj", "mlp.down_proj"):
            tag += 1
            q[f"{p}.{k}.weight"] = (torch.full((1,), float(tag)), torch.full((1,), float(-tag)))
            keys[tag] = f"{p}.{k}"
    q["model.embed_tokens.weight"] = torch.zeros(1)
    q["model.norm.weight"] = torch.zeros(1)
    q["lm_head.weight"] = (torch.zeros(1), torch.zeros(1))
    _, layers, scales, _, _, _ = mq.pack_int8(q, cfg)
    names = [keys[int(t.item())].split(".", 3)[3] for t in layers[:11]]
    assert names == ["input_layernorm", "self_attn.q_proj", "self_attn.k_proj", "self_attn.v_proj",
                     "self_attn.q_norm", "self_attn.k_norm", "self_attn.o_proj", "post_attention_layernorm",
                     "mlp.gate_proj", "mlp.up_proj", "mlp.down_proj"]
    snames = [keys[int(-t.item())].split(".", 3)[3] for t in scales[:7]]
    assert snames == ["self_attn.q_proj", "self_attn.k_proj", "self_attn.v_proj", "self_attn.o_proj",
                      "mlp.gate_proj", "mlp.up_proj", "mlp.down_proj"]
    assert keys[int(layers[11].item())].startswith("model.layers.1.")


def test_decoder_validation_before_any_launch(mq):
    cfg = mq.QWEN3_0_6B
    embed = torch.zeros(16, cfg.hidden_size, dtype=torch.bfloat16)       # CPU tensor
    with pytest.raises(ValueError, match="HIP device"):
        mq.A10Int8MegakernelDecoder(embed, [], [], None, None, None, None, None, 1, 8)
    with pytest.raises(TypeError, match="dtype"):
        mq.A10Int8MegakernelDecoder(embed.float(), [], [], None, None, None, None, None, 1, 8)
    with pytest.raises(ValueError, match="num_layers"):
        mq.A10MegakernelDecoder(embed, [], None, None, None, None, 0, 8)
    with pytest.raises(ValueError, match="HIP device"):
        mq.quantize_per_channel(torch.zeros(4, 16, dtype=torch.bfloat16))
    with pytest.raises(TypeError):
        mq.quantize_per_channel(torch.zeros(4, 16))


def test_random_init_is_deterministic(mq):
    cfg = mq.QWEN3_0_6B.with_(num_layers=1, vocab_size=512)
    s1, p1 = mq.random_init_state(cfg, seed=3)
    s2, p2 = mq.random_init_state(cfg, seed=3)
    s3, _ = mq.random_init_state(cfg, seed=4)
    assert mq.state_digest(s1) == mq.state_digest(s2) != mq.state_digest(s3)
    assert torch.equal(p1, p2) and p1.min() >= 0 and p1.max() < 512 and len(p1) == 8
    assert s1["lm_head.weight"] is s1["model.embed_tokens.weight"]
    w = s1["model.layers.0.self_attn.q_proj.weight"]
    assert w.dtype == torch.bfloat16 and tuple(w.shape) == (2048, 1024)
    assert abs(float(w.float().std()) - 0.02) < 1e-3


def test_wait_host_token(mq):
    """mq_wait_host_token returns as soon as the word differs from the sentinel, and reports a
    timeout (without touching the word) when it never does."""
    import time
    from megaqwen_a10_amd import _lib
    lib = _lib.load()
    word = ctypes.c_int(7)
    assert lib.mq_wait_host_token(ctypes.byref(word), -2, 1000) == _lib.MQ_OK
    word.value = -2
    t0 = time.perf_counter()
    assert lib.mq_wait_host_token(ctypes.byref(word), -2, 20_000) == _lib.MQ_ERR_TIMEOUT
    assert time.perf_counter() - t0 >= 0.019
    assert "no token" in _lib.last_error() and word.value == -2
    assert lib.mq_wait_host_token(None, -2, 10) == _lib.MQ_ERR_INVALID_ARGUMENT
