"""Checkpoint loading without a GPU: HF key handling, the shape from config.json and
the tokenizer (a10_decode.py:281-325, bench_int8.py:27-55).

Each test writes a small checkpoint directory under ``tmp_path`` (2 layers of the
Qwen3-0.6B layer shape, a 512-word vocabulary) from seeded weights and checks what
``load_checkpoint_state`` / ``config_from_checkpoint`` / ``load_tokenizer`` return
against the state it was written from.
"""
from __future__ import annotations

import json

import pytest
import torch

from .ckpt import text_of, tied_state_with_defaults, write_checkpoint


@pytest.fixture(scope="module")
def seeded(mq):
    cfg = mq.QWEN3_0_6B.with_(name="ckpt-test", num_layers=2, vocab_size=512)
    state, prompt = mq.random_init_state(cfg, seed=7, norm_jitter=0.2)
    return cfg, state, prompt


def test_loader_merges_shards_ties_head_and_defaults_qk_norms(mq, seeded, tmp_path):
    cfg, state, _ = seeded
    path = write_checkpoint(tmp_path / "m", state, cfg, drop_qk_norm_layers=(1,), fp32_shard=True)
    got = mq.load_checkpoint_state(path, cfg)
    want = tied_state_with_defaults(state, cfg, drop_qk_norm_layers=(1,))
    assert sorted(got) == sorted(want)
    for k, v in want.items():
        assert got[k].dtype == torch.bfloat16, k
        assert torch.equal(got[k], v), k                  # fp32 shard holds bf16 values: exact
    # the jittered layer-0 gains survive, the dropped layer-1 gains are ones
    assert not torch.equal(got["model.layers.0.self_attn.q_norm.weight"], torch.ones(cfg.head_dim, dtype=torch.bfloat16))
    assert torch.equal(got["model.layers.1.self_attn.k_norm.weight"], torch.ones(cfg.head_dim, dtype=torch.bfloat16))


def test_loader_keeps_an_untied_head(mq, seeded, tmp_path):
    cfg, state, _ = seeded
    st = dict(state)
    st["lm_head.weight"] = (state["model.embed_tokens.weight"].float() * 0.5).to(torch.bfloat16)
    path = write_checkpoint(tmp_path / "m", st, cfg, untie=True, fp32_shard=False)
    got = mq.load_checkpoint_state(path, cfg)
    assert torch.equal(got["lm_head.weight"], st["lm_head.weight"])
    assert not torch.equal(got["lm_head.weight"], got["model.embed_tokens.weight"])


def test_loader_errors(mq, seeded, tmp_path):
    cfg, state, _ = seeded
    with pytest.raises(FileNotFoundError):
        mq.load_checkpoint_state(tmp_path, cfg)                       # no shards
    st = {k: v for k, v in state.items() if k != "model.layers.1.mlp.down_proj.weight"}
    path = write_checkpoint(tmp_path / "m", st, cfg)
    with pytest.raises(KeyError, match="model.layers.1.mlp.down_proj.weight"):
        mq.load_checkpoint_state(path, cfg)


def test_config_from_checkpoint(mq, seeded, tmp_path):
    cfg, state, _ = seeded
    path = write_checkpoint(tmp_path / "m", state, cfg)
    got = mq.config_from_checkpoint(path, mq.QWEN3_0_6B)
    assert (got.num_layers, got.hidden_size, got.intermediate_size, got.vocab_size) == (2, 1024, 3072, 512)
    assert (got.num_q_heads, got.num_kv_heads, got.head_dim, got.rms_eps, got.rope_theta) == (16, 8, 128, 1e-6, 1e6)
    assert mq.config_from_checkpoint(tmp_path, mq.QWEN3_1_7B) == mq.QWEN3_1_7B    # no config.json


def test_tokenizer_round_trip_and_eos(mq, tmp_path):
    from .ckpt import write_tokenizer
    write_tokenizer(tmp_path, 512, eos=9)
    tok = mq.load_tokenizer(tmp_path)
    assert tok is not None and tok.eos_token_id == 9
    ids = [5, 17, 300, 9]
    assert tok.encode(text_of(ids[:3])) == ids[:3]
    assert tok.decode(ids, skip_special_tokens=True) == text_of(ids[:3])
    assert mq.load_tokenizer(tmp_path / "missing") is None


def test_a10decoder_refuses_before_touching_the_device(mq, seeded, tmp_path):
    """Host-side refusals of A10Decoder: a missing checkpoint without seed=, and a
    checkpoint whose shape the kernels are not compiled for."""
    cfg, state, _ = seeded
    with pytest.raises(FileNotFoundError):
        mq.A10Decoder(tmp_path / "nothing-here", device="cpu")
    path = write_checkpoint(tmp_path / "m", state, cfg)
    conf = json.loads((path / "config.json").read_text())
    conf["rms_norm_eps"] = 1e-5
    (path / "config.json").write_text(json.dumps(conf))
    with pytest.raises(ValueError, match="eps"):
        mq.A10Decoder(path, device="cpu")
