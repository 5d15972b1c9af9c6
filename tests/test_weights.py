"""Checkpoint loading (stride_amd.weights, the counterpart of the reference's
ModelConfig::load and Weights constructor, src/model.cpp:14-238) on the CPU:
packed layouts against the source matrices, configuration parsing, and the RoPE
table against closed forms, its special cases and the llama3 frequencies of the
transformers library."""
import json
import math
import os

import numpy as np
import pytest
import torch

from stride_amd import layout, weights
import llama_tiny


def bits(a):
    return torch.as_tensor(a).to(torch.bfloat16).view(torch.int16).numpy()


@pytest.mark.parametrize("tied", [True, False])
def test_load_packs_every_matrix(tmp_path, tied):
    t, c = llama_tiny.write(str(tmp_path), seed=1, tied=tied)
    w = weights.Weights.load(str(tmp_path), "cpu", max_positions=16)
    cfg = w.cfg
    D = cfg.head_dim
    for i in range(cfg.layers):
        p = f"model.layers.{i}."
        L = w.layers[i]
        for name, key, rope in (("q", "self_attn.q_proj.weight", True), ("k", "self_attn.k_proj.weight", True),
                                ("v", "self_attn.v_proj.weight", True), ("o", "self_attn.o_proj.weight", False),
                                ("w1", "mlp.gate_proj.weight", False), ("w3", "mlp.up_proj.weight", False),
                                ("w2", "mlp.down_proj.weight", False)):
            src = bits(t[p + key])
            order = layout.rope_rows(src.shape[0], D) if rope else None
            got = layout.unpack_rows(L[name].numpy(), order)
            assert np.array_equal(got, src), f"layer {i} {name}"
            # packed tile rt, slot s, column c holds source row order[16 rt + s], column c
            tiles = L[name].numpy()
            rt, s, col = 1, 9, 37
            row = order[16 * rt + s] if rope else 16 * rt + s
            assert tiles[rt, col // 16, s, col % 16] == src[row, col]
        assert np.array_equal(L["norm_attn"].numpy(), t[p + "input_layernorm.weight"].astype(np.float32))
    # vocabulary padded with zero rows to a multiple of 16
    emb = w.embed.numpy()
    assert emb.shape[0] == (cfg.vocab + 15) // 16
    full = layout.unpack_rows(emb)
    assert np.array_equal(full[: cfg.vocab], bits(t["model.embed_tokens.weight"]))
    assert not full[cfg.vocab:].any()
    if tied:
        assert w.lm is w.embed
    else:
        assert np.array_equal(layout.unpack_rows(w.lm.numpy())[: cfg.vocab], bits(t["lm_head.weight"]))


def test_config_parse(tmp_path):
    c = dict(llama_tiny.TINY)
    with open(tmp_path / "config.json", "w") as f:
        json.dump(c, f)
    m = weights.ModelConfig.load(str(tmp_path))
    assert (m.hidden, m.mlp, m.layers, m.heads, m.kv_heads, m.head_dim, m.vocab) == (256, 512, 2, 8, 2, 32, 1000)
    assert m.rope_llama3 and m.rope_factor == 32.0 and m.rope_orig_ctx == 8192.0 and m.eos_tokens == [7, 9]
    # defaults (src/model.cpp:21-26): kv_heads = heads, head_dim = hidden / heads, no scaling
    c2 = {k: c[k] for k in ("hidden_size", "intermediate_size", "num_hidden_layers", "num_attention_heads",
                            "vocab_size")}
    c2["num_key_value_heads"] = 2
    with open(tmp_path / "config.json", "w") as f:
        json.dump(c2, f)
    m2 = weights.ModelConfig.load(str(tmp_path))
    assert m2.head_dim == 32 and m2.rope_theta == 10000.0 and not m2.rope_llama3 and m2.eos_tokens == []
    for bad, msg in (({"num_key_value_heads": 8}, "head layout"), ({"rope_scaling": {"rope_type": "yarn"}}, "rope type"),
                     ({"head_dim": 30}, "head_dim")):
        with open(tmp_path / "config.json", "w") as f:
            json.dump({**c, **bad}, f)
        with pytest.raises(RuntimeError, match=msg):
            weights.ModelConfig.load(str(tmp_path))
    with pytest.raises(RuntimeError, match="config.json"):
        weights.ModelConfig.load(str(tmp_path / "absent"))


def test_rope_table_special_cases_and_closed_form():
    cfg = weights.ModelConfig(rope_llama3=False, rope_theta=10000.0, head_dim=64)
    tab = weights.build_rope_table(cfg, 4097)
    assert tab.shape == (4097, 32, 2) and tab.dtype == np.float32
    assert np.all(tab[0, :, 0] == 1.0) and np.all(tab[0, :, 1] == 0.0)
    assert tab[1, 0, 0] == np.float32(math.cos(1.0)) and tab[1, 0, 1] == np.float32(math.sin(1.0))  # f_0 = 1
    ang = np.arange(4097)[:, None] * 10000.0 ** (-np.arange(32) * 2 / 64)[None, :]
    tol = np.abs(ang) * 2.0 ** -21 + 2.0 ** -24
    assert np.all(np.abs(tab[..., 0] - np.cos(ang)) <= tol)
    assert np.all(np.abs(tab[..., 1] - np.sin(ang)) <= tol)
    assert np.allclose(tab[..., 0] ** 2 + tab[..., 1] ** 2, 1.0, atol=1e-6)


def test_llama3_frequency_bands():
    """Bands of the llama3 rule (src/model.cpp:57-71): wavelengths beyond
    orig_ctx/low are divided by the factor, below orig_ctx/high kept, blended
    in between; equal to the transformers library's llama3 frequencies."""
    scaled = weights.rope_frequencies(weights.ModelConfig())
    plain = weights.rope_frequencies(weights.ModelConfig(rope_llama3=False))
    wave = 2 * math.pi / plain.astype(np.float64)
    lo, hi = wave > 8192.0, wave < 2048.0
    assert lo.any() and hi.any() and (~lo & ~hi).any()
    assert np.array_equal(scaled[hi], plain[hi])
    assert np.array_equal(scaled[lo], (plain[lo] / np.float32(32.0)).astype(np.float32))
    mid = ~lo & ~hi
    assert np.all(scaled[mid] < plain[mid]) and np.all(scaled[mid] > plain[mid] / 32)
    try:
        from transformers import LlamaConfig
        from transformers.modeling_rope_utils import _compute_llama3_parameters
    except ImportError:
        pytest.skip("transformers not importable")
    hc = LlamaConfig(hidden_size=2048, num_attention_heads=32, num_key_value_heads=8, head_dim=64,
                     max_position_embeddings=131072, rope_theta=500000.0,
                     rope_scaling={"rope_type": "llama3", "factor": 32.0, "low_freq_factor": 1.0,
                                   "high_freq_factor": 4.0, "original_max_position_embeddings": 8192})
    inv, _ = _compute_llama3_parameters(hc, "cpu")
    assert np.array_equal(scaled, inv.numpy().astype(np.float32))


def test_random_weights_shapes():
    cfg = weights.ModelConfig(hidden=256, mlp=512, layers=1, heads=8, kv_heads=2, head_dim=32, vocab=1000)
    w = weights.Weights.random(cfg, "cpu", seed=2, max_positions=8)
    assert w.embed.shape == (63, 16, 16, 16) and w.lm is w.embed
    assert w.layers[0]["q"].shape == (16, 16, 16, 16) and w.layers[0]["w2"].shape == (16, 32, 16, 16)


@pytest.mark.parametrize("cfg", [weights.ModelConfig(), weights.ModelConfig(rope_llama3=False, rope_theta=10000.0),
                                 weights.ModelConfig(rope_llama3=False, head_dim=128)])
def test_rope_table_bit_equal_to_restatement(exact, cfg):
    """The loader's RoPE table equals, bit for bit, the C restatement of the
    reference's build_rope_table (src/model.cpp:54-88) compiled with the C
    library's cos/sin, at 4097 positions, plain and llama3-scaled."""
    got = weights.build_rope_table(cfg, 4097)
    want = exact.rope_table(cfg, 4097)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


def test_engine_rejects_context_beyond_rope_table():
    """The QKV epilogue reads rope[pos]: an engine whose context exceeds the
    table is refused before anything is allocated."""
    from stride_amd import engine

    cfg = weights.ModelConfig(hidden=128, mlp=256, layers=1, heads=4, kv_heads=1, head_dim=32, vocab=64)
    w = weights.Weights.random(cfg, "cpu", seed=0, max_positions=16)
    with pytest.raises(ValueError, match="RoPE table"):
        engine.Engine(w, slots=1, max_ctx=17, max_rows=16)
