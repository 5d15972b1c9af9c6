"""A tiny Llama checkpoint in the Hugging Face layout (config.json +
model.safetensors) written from a seed, and a float64 NumPy forward of the same
model that rounds to bf16 exactly where the tensor-core path stores bf16 (the
normalised activations, K and V in the cache, the attention output, the gated
MLP activation). Used to check weight loading and the decode engine."""
import json
import os

import numpy as np
import torch

TINY = dict(hidden_size=256, intermediate_size=512, num_hidden_layers=2, num_attention_heads=8,
            num_key_value_heads=2, head_dim=32, vocab_size=1000, rms_norm_eps=1e-5, rope_theta=500000.0,
            rope_scaling={"rope_type": "llama3", "factor": 32.0, "low_freq_factor": 1.0, "high_freq_factor": 4.0,
                          "original_max_position_embeddings": 8192},
            eos_token_id=[7, 9], tie_word_embeddings=True)


def write(path, seed=0, tied=True, cfg=None):
    from safetensors.torch import save_file

    c = dict(TINY if cfg is None else cfg)
    g = torch.Generator().manual_seed(seed)
    H, F, V, D = c["hidden_size"], c["intermediate_size"], c["vocab_size"], c["head_dim"]
    nq, nkv = c["num_attention_heads"], c["num_key_value_heads"]

    def w(*shape, std=0.05):
        return (torch.randn(*shape, generator=g) * std).to(torch.bfloat16)

    t = {"model.embed_tokens.weight": w(V, H, std=1.0), "model.norm.weight": (1 + w(H, std=0.2).float()).to(torch.bfloat16)}
    for i in range(c["num_hidden_layers"]):
        p = f"model.layers.{i}."
        t[p + "self_attn.q_proj.weight"] = w(nq * D, H)
        t[p + "self_attn.k_proj.weight"] = w(nkv * D, H)
        t[p + "self_attn.v_proj.weight"] = w(nkv * D, H)
        t[p + "self_attn.o_proj.weight"] = w(H, nq * D)
        t[p + "mlp.gate_proj.weight"] = w(F, H)
        t[p + "mlp.up_proj.weight"] = w(F, H)
        t[p + "mlp.down_proj.weight"] = w(H, F)
        t[p + "input_layernorm.weight"] = (1 + w(H, std=0.2).float()).to(torch.bfloat16)
        t[p + "post_attention_layernorm.weight"] = (1 + w(H, std=0.2).float()).to(torch.bfloat16)
    if not tied:
        t["lm_head.weight"] = w(V, H)
        c["tie_word_embeddings"] = False
    os.makedirs(path, exist_ok=True)
    save_file(t, os.path.join(path, "model.safetensors"))
    with open(os.path.join(path, "config.json"), "w") as f:
        json.dump(c, f)
    return {k: v.float().numpy() for k, v in t.items()}, c


def bf16(a):
    """float64 -> fp32 -> bf16 (round to nearest even on the bits), as float64."""
    u = np.asarray(a, np.float32).view(np.uint32).astype(np.uint64)
    r = ((u + 0x7FFF + ((u >> 16) & 1)) & 0xFFFF0000).astype(np.uint32)
    return r.view(np.float32).astype(np.float64)


def forward_last_logits(t, c, tokens, rope, round_bf16=True):
    """Logits (float64) of the last position of `tokens` for one sequence.
    rope: [pos][D/2][cos, sin]. RoPE rotates pairs (i, i + D/2). round_bf16=False
    keeps every intermediate in float64 (the exact path stores fp32 throughout)."""
    bf16 = globals()["bf16"] if round_bf16 else (lambda a: np.asarray(a, np.float64))
    H, D = c["hidden_size"], c["head_dim"]
    nq, nkv, eps = c["num_attention_heads"], c["num_key_value_heads"], c["rms_norm_eps"]
    n = len(tokens)
    h = t["model.embed_tokens.weight"][tokens].astype(np.float64)

    def norm(x, gname):
        return bf16(x / np.sqrt((x * x).mean(axis=1, keepdims=True) + eps) * t[gname].astype(np.float64))

    def rot(x, heads):  # x [n][heads*D]
        x = x.reshape(n, heads, D).copy()
        cs = rope[:n].astype(np.float64)
        cos, sin = cs[:, None, :, 0], cs[:, None, :, 1]
        a, b = x[..., : D // 2].copy(), x[..., D // 2:].copy()
        x[..., : D // 2] = a * cos - b * sin
        x[..., D // 2:] = b * cos + a * sin
        return x

    for i in range(c["num_hidden_layers"]):
        p = f"model.layers.{i}."
        x = norm(h, p + "input_layernorm.weight")
        q = rot(x @ t[p + "self_attn.q_proj.weight"].T, nq)
        k = bf16(rot(x @ t[p + "self_attn.k_proj.weight"].T, nkv))
        v = bf16((x @ t[p + "self_attn.v_proj.weight"].T).reshape(n, nkv, D))
        att = np.zeros((n, nq, D))
        for j in range(n):
            for hh in range(nq):
                g = hh // (nq // nkv)
                s = k[: j + 1, g] @ q[j, hh] / np.sqrt(D)
                e = np.exp(s - s.max())
                att[j, hh] = (e / e.sum()) @ v[: j + 1, g]
        h = h + bf16(att.reshape(n, nq * D)) @ t[p + "self_attn.o_proj.weight"].T
        x = norm(h, p + "post_attention_layernorm.weight")
        a = x @ t[p + "mlp.gate_proj.weight"].T
        z = bf16(a / (1 + np.exp(-a)) * (x @ t[p + "mlp.up_proj.weight"].T))
        h = h + z @ t[p + "mlp.down_proj.weight"].T
    x = norm(h[-1:], "model.norm.weight")
    lm = t["lm_head.weight"] if "lm_head.weight" in t else t["model.embed_tokens.weight"]
    return (x @ lm.T)[0]
