"""A minimal greedy decode engine over the tensor-core operators.

It drives one decode step exactly as the reference's Engine::step_tensor_core
(src/engine.cpp:300-462) does: tc_embed, then per layer tc_norm, tc_qkv,
tc_attention, tc_gemm_residual (O), tc_norm, tc_mlp13, tc_gemm_residual (down),
then the final tc_norm, tc_compact of the rows that need a token and
tc_lm_greedy. Rows are (slot, position, token) triples; prompts are processed as
ordinary rows (chunked prefill), so a prompt token and a decode token go through
identical arithmetic. Every row's result depends only on its own slot contents
and position, never on the batch it shares a step with, its lane, or where its
KV pages live; the full-step engine test runs sequences alone and in shuffled batches
and compares their token streams and fingerprints.

Each sequence keeps the reference scheduler's fingerprint (src/scheduler.cpp:
15-24, 280): FNV-1a over the little-endian bytes of each generated token id and
of the fp32 bits of its logit, starting from the FNV offset basis.

Weights come from stride_amd.weights: a safetensors checkpoint packed as the
reference's Weights constructor packs it (src/model.cpp:139-238), or random-init
tiles of the same shapes.
"""
from __future__ import annotations

import dataclasses
import math

import numpy as np
import torch

from . import harness, layout, tc
from .weights import ModelConfig
from .weights import Weights as PackedWeights

FNV_OFFSET = 14695981039346656037
FNV_PRIME = 1099511628211
MASK64 = (1 << 64) - 1


def fnv_bytes(h: int, data: bytes) -> int:
    """64-bit FNV-1a over `data`, continuing from state h."""
    for byte in data:
        h ^= byte
        h = (h * FNV_PRIME) & MASK64
    return h


def fnv_mix(h: int, v: int) -> int:
    """FNV-1a over the four little-endian bytes of a 32-bit value
    (src/scheduler.cpp:15-24)."""
    return fnv_bytes(h, (v & 0xFFFFFFFF).to_bytes(4, "little"))


# Model shape and weights: stride_amd.weights (checkpoint loading or random init).
LlamaConfig = ModelConfig


def Weights(cfg: ModelConfig, device, seed: int = 0, max_positions: int = 4097) -> PackedWeights:
    """Random-init weights of shape `cfg` (no checkpoint); see
    stride_amd.weights.Weights.load for real checkpoints."""
    return PackedWeights.random(cfg, device, seed, max_positions)


@dataclasses.dataclass
class Sequence:
    slot: int
    prompt: list
    tokens: list = dataclasses.field(default_factory=list)
    values: list = dataclasses.field(default_factory=list)
    fingerprint: int = FNV_OFFSET

    @property
    def length(self) -> int:
        return len(self.prompt) + len(self.tokens)


class Engine:
    """One model, a paged bf16 KV cache and the step buffers for up to max_rows rows."""

    def __init__(self, weights: Weights, slots: int, max_ctx: int, max_rows: int, page_tokens: int = 16,
                 shuffle_seed: int = 0, attention_one_kernel: bool = False):
        self.w = weights
        cfg = self.cfg = weights.cfg
        dev = self.dev = weights.embed.device
        if cfg.head_dim not in (32, 64, 128) or cfg.repeat() != 4:
            raise ValueError("the tensor-core attention serves head_dim 32/64/128 with four query heads per KV head")
        rope_positions = int(weights.rope.shape[0])
        if max_ctx > rope_positions:
            raise ValueError(f"max_ctx {max_ctx} exceeds the RoPE table's {rope_positions} positions "
                             "(the QKV epilogue reads rope[pos] for every pos < max_ctx)")
        self.max_rows = max_rows
        self.max_pages = (max_ctx + 63) // 64
        # Every step passes the reference's item list (every page of every row),
        # and the library runs pages and combine as one kernel when the records
        # fit its LDS, else the page + combine pair. attention_one_kernel = True
        # passes item_count = -1 instead (the same kernel without the list check),
        # which only the LDS-fitting sizes accept, so it is dropped otherwise.
        self.one_kernel = attention_one_kernel and harness.attention_one_kernel_fits(
            self.max_pages, cfg.head_dim, page_tokens)
        lt = (max_rows + 15) // 16
        H, D = cfg.hidden, cfg.head_dim
        self.kv = harness.PagedKv.create(slots, max_ctx, cfg.kv_heads, D, cfg.layers, page_tokens, dev,
                                         shuffle_seed=shuffle_seed)
        self.h = torch.zeros((lt, H // 16, 16, 16), dtype=torch.float32, device=dev)
        self.x = torch.zeros((lt, H // 16, 16, 16), dtype=torch.int16, device=dev)
        self.attn = torch.zeros((lt, cfg.heads * D // 16, 16, 16), dtype=torch.int16, device=dev)
        self.z = torch.zeros((lt, cfg.mlp // 16, 16, 16), dtype=torch.int16, device=dev)
        self.lm_x = torch.zeros((lt, H // 16, 16, 16), dtype=torch.int16, device=dev)
        self.q = torch.zeros((max_rows, cfg.heads * D), dtype=torch.float32, device=dev)
        self.scratch = torch.zeros(max_rows * cfg.kv_heads * self.max_pages * (4 * D + 8), dtype=torch.float32,
                                   device=dev)

    def launch(self, n: int, slot, pos, tok, items, greedy=None, best=None) -> None:
        """Enqueue one step over n rows described by device tensors (row slots,
        positions, tokens, attention items); no host synchronization, so it can
        be captured in a HIP graph. `greedy` (device int32 row indices) selects
        the rows whose token is wanted (None: all n), `best` receives them."""
        cfg, w = self.cfg, self.w
        scale = float(math.pow(cfg.head_dim, -0.5))
        harness.embed(w.embed, tok, n, cfg.hidden, h_out=self.h)
        for li, L in enumerate(w.layers):
            harness.norm(self.h, n, L["norm_attn"], cfg.rms_eps, x_out=self.x)
            harness.qkv(L["q"], L["k"], L["v"], self.x, n, cfg.head_dim, w.rope, slot, pos, self.kv, layer=li,
                        q_out=self.q)
            harness.attention(self.q[:n], self.kv, slot, pos, cfg.kv_heads, cfg.head_dim, scale, layer=li,
                              max_pages=self.max_pages, out_tiles=self.attn, items=items, scratch=self.scratch,
                              one_kernel=self.one_kernel)
            harness.gemm_residual(L["o"], self.attn, self.h, n)
            harness.norm(self.h, n, L["norm_mlp"], cfg.rms_eps, x_out=self.x)
            harness.mlp13(L["w1"], L["w3"], self.x, n, out=self.z)
            harness.gemm_residual(L["w2"], self.z, self.h, n)
        harness.norm(self.h, n, w.norm_final, cfg.rms_eps, x_out=self.x)
        if best is None:
            return
        count = n if greedy is None else int(greedy.numel())
        x = self.x
        if greedy is not None:
            harness.compact(self.x, greedy, out_tiles=self.lm_x)
            x = self.lm_x
        harness.best_reset(best)
        harness.lm_greedy(w.lm, x, count, cfg.vocab, best=best)

    def device_rows(self, rows):
        """Device tensors (slot, pos, tok, items) for rows [(slot, pos, token)];
        items lists every (row, 64-position page) up to each row's position
        (src/engine.cpp:93-103)."""
        dev = self.dev
        slot = torch.tensor([r[0] for r in rows], dtype=torch.int32, device=dev)
        pos = torch.tensor([r[1] for r in rows], dtype=torch.int32, device=dev)
        tok = torch.tensor([r[2] for r in rows], dtype=torch.int32, device=dev)
        items = torch.tensor([[j, pg] for j, r in enumerate(rows) for pg in range((r[1] >> 6) + 1)],
                             dtype=torch.int32, device=dev).reshape(-1)
        return slot, pos, tok, items

    def step(self, rows, greedy):
        """One step over rows [(slot, pos, token)]; returns (index, value bits) for
        the rows listed in `greedy` (indices into rows), in that order."""
        n = len(rows)
        assert 0 < n <= self.max_rows
        slot, pos, tok, items = self.device_rows(rows)
        if not greedy:
            self.launch(n, slot, pos, tok, items)
            return []
        count = len(greedy)
        sel = None if count == n else torch.tensor(greedy, dtype=torch.int32, device=self.dev)
        best = torch.empty((count, 2), dtype=torch.int32, device=self.dev)
        self.launch(n, slot, pos, tok, items, greedy=sel, best=best)
        b = best.cpu().numpy().view(np.uint32).reshape(count, 2)
        return [(int(b[i, 1].view(np.int32)), int(b[i, 0])) for i in range(count)]

    def _record(self, seq: Sequence, index: int, value_bits: int) -> None:
        seq.tokens.append(index)
        seq.values.append(value_bits)
        seq.fingerprint = fnv_mix(fnv_mix(seq.fingerprint, index & 0xFFFFFFFF), value_bits)

    def prefill(self, seqs, order=None):
        """Prompt rows of every sequence, in chunks of at most max_rows, each
        sequence's positions ascending; the last prompt row yields token 1."""
        rows = []
        for s in seqs:
            rows += [(s, p) for p in range(len(s.prompt))]
        if order is not None:  # shuffle lanes inside a chunk, keeping each sequence's chunks ordered
            rows = [rows[i] for i in order]
            rows.sort(key=lambda r: r[1])
        for c0 in range(0, len(rows), self.max_rows):
            chunk = rows[c0:c0 + self.max_rows]
            step_rows = [(s.slot, p, s.prompt[p]) for s, p in chunk]
            greedy = [i for i, (s, p) in enumerate(chunk) if p == len(s.prompt) - 1]
            for i, (idx, val) in zip(greedy, self.step(step_rows, greedy)):
                self._record(chunk[i][0], idx, val)

    def decode(self, seqs, steps: int, perm_seed: int = 0):
        rng = np.random.default_rng(perm_seed)
        for _ in range(steps):
            order = rng.permutation(len(seqs)) if perm_seed else np.arange(len(seqs))
            batch = [seqs[i] for i in order]
            rows = [(s.slot, s.length - 1, s.tokens[-1]) for s in batch]
            for s, (idx, val) in zip(batch, self.step(rows, list(range(len(rows))))):
                self._record(s, idx, val)


def run(batch: int, prompt_len: int, new_tokens: int, device="cuda:0", seed: int = 0, cfg: ModelConfig | None = None,
        page_tokens: int = 16, max_rows: int = 4096, shuffle_seed: int = 0, perm_seed: int = 0, weights=None):
    """Greedy decode of `batch` random prompts; returns the sequences."""
    cfg = cfg or ModelConfig()
    weights = weights or Weights(cfg, device, seed)
    rng = np.random.default_rng(seed + 1)
    prompts = [rng.integers(0, cfg.vocab, prompt_len).tolist() for _ in range(batch)]
    eng = Engine(weights, batch, prompt_len + new_tokens, max_rows, page_tokens, shuffle_seed)
    seqs = [Sequence(i, p) for i, p in enumerate(prompts)]
    eng.prefill(seqs)
    eng.decode(seqs, new_tokens - 1, perm_seed)
    return seqs
