"""Llama checkpoints for the tensor-core path: config.json + safetensors ->
packed weight tiles on the device, as the reference's ModelConfig::load and
Weights constructor produce them (src/model.cpp:14-48, 139-238).

* Projections are packed into 16-row tiles [row tile][col tile][16][16]
  (src/model.cpp:114-133). q, k and v use the RoPE row order: a row tile holds
  eight RoPE pairs, rows d0+i and d0+D/2+i of one head (src/model.cpp:178-183);
  o, gate, up and down keep the plain order.
* The embedding is padded with zero rows to a multiple of 16 and serves as the
  LM head unless the checkpoint holds lm_head.weight (src/model.cpp:218-232).
* RMSNorm gains are widened to fp32 (src/model.cpp:135-146).
* The RoPE table is [position][head_dim/2][cos, sin] fp32 with the reference's
  float arithmetic, including llama3 frequency scaling (src/model.cpp:50-90).

Only BF16 tensors are accepted, as in the reference. The checkpoint is read
with safetensors (no pickle); a sharded checkpoint (model.safetensors.index.json)
is accepted as well.
"""
from __future__ import annotations

import dataclasses
import json
import math
import os

import numpy as np
import torch

from . import layout

MAX_HEAD_DIM = 256  # src/kernels.h kMaxHeadDim


@dataclasses.dataclass
class ModelConfig:
    """Model shape and numerics (src/model.h:12-31). The defaults are
    Llama-3.2-1B's."""
    hidden: int = 2048
    mlp: int = 8192
    layers: int = 16
    heads: int = 32
    kv_heads: int = 8
    head_dim: int = 64
    vocab: int = 128256
    rms_eps: float = 1e-5
    rope_theta: float = 500000.0
    rope_llama3: bool = True
    rope_factor: float = 32.0
    rope_low: float = 1.0
    rope_high: float = 4.0
    rope_orig_ctx: float = 8192.0
    eos_tokens: list = dataclasses.field(default_factory=lambda: [128001, 128008, 128009])

    def repeat(self) -> int:
        return self.heads // self.kv_heads

    @staticmethod
    def load(model_dir: str) -> "ModelConfig":
        """config.json -> ModelConfig with the reference's defaults and checks
        (src/model.cpp:14-48)."""
        path = os.path.join(model_dir, "config.json")
        if not os.path.exists(path):
            raise RuntimeError("cannot open config.json in " + model_dir)
        with open(path) as f:
            j = json.load(f)
        c = ModelConfig(rope_llama3=False, rope_factor=1.0, rope_low=1.0, rope_high=4.0, rope_orig_ctx=8192.0,
                        eos_tokens=[])
        c.hidden = int(j["hidden_size"])
        c.mlp = int(j["intermediate_size"])
        c.layers = int(j["num_hidden_layers"])
        c.heads = int(j["num_attention_heads"])
        c.kv_heads = int(j.get("num_key_value_heads", c.heads))
        c.head_dim = int(j.get("head_dim", c.hidden // c.heads))
        c.vocab = int(j["vocab_size"])
        c.rms_eps = float(j.get("rms_norm_eps", 1e-5))
        c.rope_theta = float(j.get("rope_theta", 10000.0))
        r = j.get("rope_scaling")
        if r is not None:
            kind = r.get("rope_type", r.get("type", ""))
            if kind == "llama3":
                c.rope_llama3 = True
                c.rope_factor = float(r.get("factor", 32.0))
                c.rope_low = float(r.get("low_freq_factor", 1.0))
                c.rope_high = float(r.get("high_freq_factor", 4.0))
                c.rope_orig_ctx = float(r.get("original_max_position_embeddings", 8192.0))
            elif kind and kind != "default":
                raise RuntimeError("unsupported rope type " + kind)
        eos = j.get("eos_token_id")
        if eos is not None:
            c.eos_tokens = list(eos) if isinstance(eos, list) else [int(eos)]
        if c.heads % c.kv_heads != 0 or c.repeat() != 4:
            raise RuntimeError("unsupported head layout")
        if c.head_dim % 4 != 0 or c.head_dim > MAX_HEAD_DIM:
            raise RuntimeError("unsupported head_dim")
        return c


def rope_frequencies(cfg: ModelConfig) -> np.ndarray:
    """Inverse frequencies [head_dim/2] fp32 (src/model.cpp:50-75): base =
    fp32(theta ** fp32(2i/D)), f = 1/base in fp32, then llama3 scaling on the
    wavelength 2*pi/f (low-frequency bands divided by the factor, the middle band
    blended, high-frequency bands kept)."""
    dim, half = cfg.head_dim, cfg.head_dim // 2
    f32 = np.float32
    pi2 = f32(2.0 * math.pi)
    inv = np.empty(half, dtype=np.float32)
    for i in range(half):
        e = f32(2 * i) / f32(dim)
        base = f32(math.pow(cfg.rope_theta, float(e)))
        f = f32(1.0) / base
        if cfg.rope_llama3:
            factor = f32(cfg.rope_factor)
            low_wave = f32(cfg.rope_orig_ctx / cfg.rope_low)
            high_wave = f32(cfg.rope_orig_ctx / cfg.rope_high)
            wave = pi2 / f
            smooth = (f32(cfg.rope_orig_ctx) / wave - f32(cfg.rope_low)) / f32(cfg.rope_high - cfg.rope_low)
            if wave > low_wave:
                f = f / factor
            elif not (wave < high_wave):
                f = (f32(1.0) - smooth) * (f / factor) + smooth * f
        inv[i] = f
    return inv


def build_rope_table(cfg: ModelConfig, max_positions: int) -> np.ndarray:
    """[max_positions][head_dim/2][cos, sin] fp32: angle = fp32(f_i * fp32(pos)),
    then cos/sin in double rounded to fp32 (src/model.cpp:76-88)."""
    inv = rope_frequencies(cfg)
    pos = np.arange(max_positions, dtype=np.float32)
    ang = (pos[:, None] * inv[None, :]).astype(np.float32)  # one fp32 product per entry
    # cos/sin of the C library (Python's math module calls it), as std::cos and
    # std::sin on double do; NumPy's vectorised versions may round differently
    # depending on the host's SIMD dispatch.
    a64 = ang.astype(np.float64).ravel().tolist()
    cs = np.empty((len(a64), 2), np.float64)
    cs[:, 0] = [math.cos(a) for a in a64]
    cs[:, 1] = [math.sin(a) for a in a64]
    return cs.astype(np.float32).reshape(max_positions, inv.size, 2)


class Checkpoint:
    """Read-only view of a safetensors checkpoint (single file or index)."""

    def __init__(self, model_dir: str):
        from safetensors import safe_open

        single = os.path.join(model_dir, "model.safetensors")
        index = os.path.join(model_dir, "model.safetensors.index.json")
        self._files = {}
        self._where = {}
        if os.path.exists(single):
            files = [single]
        elif os.path.exists(index):
            with open(index) as f:
                wm = json.load(f)["weight_map"]
            files = sorted({os.path.join(model_dir, v) for v in wm.values()})
        else:
            raise RuntimeError("no model.safetensors in " + model_dir)
        for path in files:
            h = safe_open(path, framework="pt", device="cpu")
            self._files[path] = h
            for k in h.keys():
                self._where[k] = path

    def has(self, name: str) -> bool:
        return name in self._where

    def get(self, name: str) -> torch.Tensor:
        if name not in self._where:
            raise RuntimeError("missing tensor " + name)
        t = self._files[self._where[name]].get_tensor(name)
        if t.dtype != torch.bfloat16:
            raise RuntimeError(f"expected BF16 weights, got {t.dtype} for {name}")
        return t


class Weights:
    """Device-resident packed weights in the layout the tensor-core operators
    consume: `embed` and `lm` tiles (the same tensor when tied), per layer q, k,
    v, o, w1, w3, w2 tiles and fp32 norm gains, `norm_final`, and `rope`."""

    def __init__(self, cfg: ModelConfig, embed, lm, layers, norm_final, rope):
        self.cfg, self.embed, self.lm, self.layers, self.norm_final, self.rope = cfg, embed, lm, layers, norm_final, rope
        self.bytes_per_pass = sum(int(t.numel()) * 2 for L in layers for k, t in L.items() if k not in
                                  ("norm_attn", "norm_mlp")) + cfg.vocab * cfg.hidden * 2

    @staticmethod
    def load(model_dir: str, device, cfg: ModelConfig | None = None, max_positions: int = 4097) -> "Weights":
        cfg = cfg or ModelConfig.load(model_dir)
        ck = Checkpoint(model_dir)
        D = cfg.head_dim

        def mat(name, rope):
            t = ck.get(name)
            n, k = t.shape
            if n % 16 or k % 16:
                raise RuntimeError("matrix shape incompatible with the packed kernels")
            bits = t.view(torch.int16).to(device)
            return layout.pack_tiles(bits, layout.rope_rows(n, D) if rope else None)

        def gains(name):
            return ck.get(name).float().to(device)

        layers = []
        for i in range(cfg.layers):
            pre = f"model.layers.{i}."
            layers.append(dict(
                q=mat(pre + "self_attn.q_proj.weight", True), k=mat(pre + "self_attn.k_proj.weight", True),
                v=mat(pre + "self_attn.v_proj.weight", True), o=mat(pre + "self_attn.o_proj.weight", False),
                w1=mat(pre + "mlp.gate_proj.weight", False), w3=mat(pre + "mlp.up_proj.weight", False),
                w2=mat(pre + "mlp.down_proj.weight", False),
                norm_attn=gains(pre + "input_layernorm.weight"), norm_mlp=gains(pre + "post_attention_layernorm.weight")))
        vocab_tiles = (cfg.vocab + 15) // 16

        def vocab_mat(name):
            t = ck.get(name)[: cfg.vocab]
            return layout.pack_tiles(t.view(torch.int16).to(device), None, vocab_tiles)

        embed = vocab_mat("model.embed_tokens.weight")
        lm = vocab_mat("lm_head.weight") if ck.has("lm_head.weight") else embed
        rope = torch.from_numpy(build_rope_table(cfg, max_positions)).to(device)
        return Weights(cfg, embed, lm, layers, gains("model.norm.weight"), rope)

    @staticmethod
    def random(cfg: ModelConfig, device, seed: int = 0, max_positions: int = 4097) -> "Weights":
        """Random-init weights ~N(0, 0.02) in bf16 with unit norm gains and a tied
        LM head (no checkpoint)."""
        g = torch.Generator(device=device).manual_seed(seed)
        D, H = cfg.head_dim, cfg.hidden

        def w(n, k, rows=None, row_tiles=None):
            t = (torch.randn(n, k, generator=g, device=device) * 0.02).to(torch.bfloat16).view(torch.int16)
            return layout.pack_tiles(t, rows, row_tiles)

        embed = w(cfg.vocab, H, None, (cfg.vocab + 15) // 16)
        layers = []
        for _ in range(cfg.layers):
            layers.append(dict(
                q=w(cfg.heads * D, H, layout.rope_rows(cfg.heads * D, D)),
                k=w(cfg.kv_heads * D, H, layout.rope_rows(cfg.kv_heads * D, D)),
                v=w(cfg.kv_heads * D, H, layout.rope_rows(cfg.kv_heads * D, D)),
                o=w(H, cfg.heads * D), w1=w(cfg.mlp, H), w3=w(cfg.mlp, H), w2=w(H, cfg.mlp),
                norm_attn=torch.ones(H, device=device), norm_mlp=torch.ones(H, device=device)))
        rope = torch.from_numpy(build_rope_table(cfg, max_positions)).to(device)
        return Weights(cfg, embed, embed, layers, torch.ones(H, device=device), rope)
