"""The exact (FP32) path end to end: a greedy decode engine that runs a whole
model through the exact-path operators in the order of the reference's
Engine::step_exact (src/engine.cpp:144-297):

    k_embed; per layer: k_norm, k_qkv, k_attention, k_gemm_residual (O),
    k_norm, k_mlp13, k_gemm_residual (down); k_norm; then k_compact of the rows
    that want a token (unless they are all of them) and k_lm_greedy, and the
    same for rows that want full logits with k_lm_full.

Layouts are the reference's exact-path ones (src/kernels.h:3-10, model.cpp:
94-111, 168-174, kv_cache.cpp:10-40): activations dim-major fp32 with one lane
(stride 1) for a lone row and lane groups of four otherwise, weights in
four-row groups (q, k, v in RoPE pair order, the vocabulary zero padded), KV
fp32 in 64-token blocks [block][layer][K|V][group][token][dim] assigned to
slots through a shuffled block table.

The engine is written against a small backend interface, so the same step
sequence drives the MI355X exact-path kernels (GpuBackend: stride_amd.exact's
stride_k_* entry points) or any other implementation of the reference's
k_* surface with the same parameter blocks. Every output word of the GPU run
equals the reference's CPU exact path on the same weights and inputs, which is
the reference's CPU == GPU claim (README.md:57) for a whole model.

Backend interface: zeros(count, dtype) and array(numpy) allocate, ptr(buf)
gives the address the parameter blocks carry, put(buf, numpy) and get(buf,
count, dtype) copy, call(name, params, J) runs k_<name> (J is None for the
operators without a lane-group argument).
"""
from __future__ import annotations

import dataclasses
import math

import numpy as np

from . import exact
from ._lib import (AttentionParams, CompactParams, EmbedParams, GemmMat, GemmResidualParams, KvRef, Lanes,
                   LmFullParams, LmGreedyParams, Mlp13Params, NormParams, QkvParams)
from .weights import ModelConfig, build_rope_table

KV_BLOCK_TOKENS = 64  # src/kernels.h kKvBlockTokens
ATTN_PAGE = 64        # attention summation page (kKvBlockShift)


def _bf16(a: np.ndarray) -> np.ndarray:
    """fp32 -> bf16 bits, round to nearest even."""
    u = np.ascontiguousarray(a, np.float32).view(np.uint32).astype(np.uint64)
    return ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)


@dataclasses.dataclass
class ExactModel:
    """Host-side exact-path weights (numpy): four-row groups and fp32 gains."""
    cfg: ModelConfig
    embed: np.ndarray          # [vocab_groups][hidden][4] bf16
    lm: np.ndarray             # same layout (the embedding itself when tied)
    layers: list               # dicts: q, k, v, o, w1, w3, w2 groups; norm_attn, norm_mlp fp32
    norm_final: np.ndarray
    rope: np.ndarray           # [positions][head_dim/2][2] fp32

    @staticmethod
    def from_rows(cfg: ModelConfig, mats: dict, max_positions: int) -> "ExactModel":
        """Packs row-major bf16 matrices (names as in weights.Checkpoint without
        the model prefix: embed, lm (optional), and per layer i 'i.q', 'i.k',
        'i.v', 'i.o', 'i.w1', 'i.w3', 'i.w2', 'i.norm_attn', 'i.norm_mlp') and
        'norm_final' (fp32)."""
        D = cfg.head_dim
        groups = (cfg.vocab + 3) // 4
        embed = exact.pack_groups(mats["embed"][: cfg.vocab], None, groups)
        lm = exact.pack_groups(mats["lm"][: cfg.vocab], None, groups) if "lm" in mats else embed
        layers = []
        for i in range(cfg.layers):
            def g(name, rope=False):
                w = mats[f"{i}.{name}"]
                return exact.pack_groups(w, exact.rope_group_rows(w.shape[0], D) if rope else None)
            layers.append(dict(q=g("q", True), k=g("k", True), v=g("v", True), o=g("o"), w1=g("w1"), w3=g("w3"),
                               w2=g("w2"), norm_attn=np.ascontiguousarray(mats[f"{i}.norm_attn"], np.float32),
                               norm_mlp=np.ascontiguousarray(mats[f"{i}.norm_mlp"], np.float32)))
        return ExactModel(cfg, embed, lm, layers, np.ascontiguousarray(mats["norm_final"], np.float32),
                          build_rope_table(cfg, max_positions))

    @staticmethod
    def random(cfg: ModelConfig, seed: int = 0, max_positions: int = 2049, gain_std: float = 0.1) -> "ExactModel":
        """Random-init weights: bf16 ~N(0, 0.02), norm gains ~N(1, gain_std), tied LM head."""
        rng = np.random.default_rng(seed)
        D, H = cfg.head_dim, cfg.hidden

        def w(n, k):
            return _bf16(rng.standard_normal((n, k), dtype=np.float32) * np.float32(0.02))

        def gain(n):
            return (1.0 + gain_std * rng.standard_normal(n)).astype(np.float32)

        mats = {"embed": w(cfg.vocab, H), "norm_final": gain(H)}
        for i in range(cfg.layers):
            mats.update({f"{i}.q": w(cfg.heads * D, H), f"{i}.k": w(cfg.kv_heads * D, H),
                         f"{i}.v": w(cfg.kv_heads * D, H), f"{i}.o": w(H, cfg.heads * D), f"{i}.w1": w(cfg.mlp, H),
                         f"{i}.w3": w(cfg.mlp, H), f"{i}.w2": w(H, cfg.mlp), f"{i}.norm_attn": gain(H),
                         f"{i}.norm_mlp": gain(H)})
        return ExactModel.from_rows(cfg, mats, max_positions)

    @staticmethod
    def load(model_dir: str, max_positions: int = 2049) -> "ExactModel":
        """A safetensors checkpoint (the reference's Weights with KernelPath::kExact,
        src/model.cpp:139-238)."""
        from .weights import Checkpoint

        cfg = ModelConfig.load(model_dir)
        ck = Checkpoint(model_dir)

        def bits(name):
            return ck.get(name).view(__import__("torch").int16).numpy().view(np.uint16)

        def gains(name):
            return ck.get(name).float().numpy()

        mats = {"embed": bits("model.embed_tokens.weight"), "norm_final": gains("model.norm.weight")}
        if ck.has("lm_head.weight"):
            mats["lm"] = bits("lm_head.weight")
        for i in range(cfg.layers):
            pre = f"model.layers.{i}."
            for key, name in (("q", "self_attn.q_proj"), ("k", "self_attn.k_proj"), ("v", "self_attn.v_proj"),
                              ("o", "self_attn.o_proj"), ("w1", "mlp.gate_proj"), ("w3", "mlp.up_proj"),
                              ("w2", "mlp.down_proj")):
                mats[f"{i}.{key}"] = bits(pre + name + ".weight")
            mats[f"{i}.norm_attn"] = gains(pre + "input_layernorm.weight")
            mats[f"{i}.norm_mlp"] = gains(pre + "post_attention_layernorm.weight")
        return ExactModel.from_rows(cfg, mats, max_positions)


class GpuBackend:
    """The MI355X exact-path kernels (include/stride_exact.h) over torch device memory."""

    def __init__(self, device="cuda:0"):
        import torch

        self.torch, self.dev = torch, device
        self._dt = {np.float32: torch.float32, np.int32: torch.int32, np.uint16: torch.int16}

    def zeros(self, count, dtype):
        return self.torch.zeros(int(count), dtype=self._dt[dtype], device=self.dev)

    def array(self, a):
        a = np.ascontiguousarray(a)
        if a.dtype == np.uint16:
            a = a.view(np.int16)
        return self.torch.from_numpy(a.reshape(-1)).to(self.dev)

    def ptr(self, buf):
        return buf.data_ptr()

    def put(self, buf, a):
        a = np.ascontiguousarray(a)
        if a.dtype == np.uint16:
            a = a.view(np.int16)
        buf[: a.size].copy_(self.torch.from_numpy(a.reshape(-1)))

    def get(self, buf, count, dtype):
        out = buf[:count].cpu().numpy()
        return out.view(dtype) if dtype == np.uint16 else out.astype(dtype, copy=False)

    def call(self, name, p, J=None):
        fn = getattr(exact, "k_" + name)
        if J is None:
            fn(p)
        else:
            fn(p, J)

    def sync(self):
        self.torch.cuda.synchronize()


class ExactEngine:
    """Buffers and the step of the reference's exact path (src/engine.cpp:56-92,
    109-297) for up to max_rows rows per step and `slots` sequences."""

    def __init__(self, model: ExactModel, backend, slots: int, max_ctx: int, max_rows: int, shuffle_seed: int = 0):
        cfg = self.cfg = model.cfg
        if cfg.repeat() != 4 or cfg.head_dim not in (32, 64, 128):
            raise ValueError("the exact attention serves head_dim 32/64/128 with four query heads per KV head")
        if max_ctx > model.rope.shape[0]:
            raise ValueError("max_ctx exceeds the RoPE table")
        B = self.B = backend
        self.max_rows = max_rows
        D, H = cfg.head_dim, cfg.hidden
        self.embed = B.array(model.embed)
        self.lm = self.embed if model.lm is model.embed else B.array(model.lm)
        self.vocab_groups = int(model.embed.shape[0])
        self.layers = [{k: B.array(v) for k, v in L.items()} for L in model.layers]
        self.norm_final = B.array(model.norm_final)
        self.rope = B.array(model.rope)
        self.mats = [{k: GemmMat(B.ptr(L[k]), int(model.layers[i][k].shape[0]), int(model.layers[i][k].shape[1]))
                      for k in ("q", "k", "v", "o", "w1", "w3", "w2")} for i, L in enumerate(self.layers)]
        self.lm_mat = GemmMat(B.ptr(self.lm), self.vocab_groups, H)
        lanes = (max_rows + 15) // 16 * 16
        q_row = cfg.heads * D
        self.h = B.zeros(lanes * H, np.float32)
        self.nx = B.zeros(lanes * H, np.float32)
        self.q = B.zeros(lanes * q_row, np.float32)
        self.attn = B.zeros(lanes * q_row, np.float32)
        self.z = B.zeros(lanes * cfg.mlp, np.float32)
        self.lm_x = B.zeros(lanes * H, np.float32)
        self.logits = B.zeros(self.vocab_groups * 4 * lanes, np.float32)
        self.best = B.zeros(lanes * 2, np.int32)
        self.tokens = B.zeros(lanes, np.int32)
        self.row_slot = B.zeros(lanes, np.int32)
        self.row_pos = B.zeros(lanes, np.int32)
        self.lm_rows = B.zeros(lanes, np.int32)
        # KV: fp32 64-token blocks, each slot's blocks drawn from a shuffled pool.
        self.max_blocks = (max_ctx + KV_BLOCK_TOKENS - 1) // KV_BLOCK_TOKENS
        group = KV_BLOCK_TOKENS * D
        which = group * cfg.kv_heads
        layer = which * 2
        block = layer * cfg.layers
        nblocks = slots * self.max_blocks
        order = np.random.default_rng(shuffle_seed).permutation(nblocks) if shuffle_seed else np.arange(nblocks)
        self.arena = B.zeros(nblocks * block, np.float32)
        self.table = B.array(order.astype(np.int32).reshape(slots, self.max_blocks))
        self.kv = KvRef(B.ptr(self.arena), B.ptr(self.table), block, layer, which, group, self.max_blocks, D)
        self.max_pages = (max_ctx + ATTN_PAGE - 1) // ATTN_PAGE
        self.rec_floats = 4 * D + 8
        self.items = B.zeros(lanes * self.max_pages * 2, np.int32)
        self.scratch = B.zeros(lanes * cfg.kv_heads * self.max_pages * self.rec_floats, np.float32)

    def upload(self, rows):
        """Host part of a step: the rows' tokens, slots, positions and attention
        items into their device buffers. Returns the item count."""
        B = self.B
        n = len(rows)
        if not 0 < n <= self.max_rows:
            raise ValueError("step needs 1 .. max_rows rows")
        B.put(self.tokens, np.array([r[2] for r in rows], np.int32))
        B.put(self.row_slot, np.array([r[0] for r in rows], np.int32))
        B.put(self.row_pos, np.array([r[1] for r in rows], np.int32))
        items = np.array([[j, pg] for j, r in enumerate(rows) for pg in range((r[1] >> 6) + 1)], np.int32)
        B.put(self.items, items.reshape(-1))
        return len(items)

    def launch_layers(self, n, item_count):
        """Device part of a step up to the final RMSNorm (self.nx), for n uploaded
        rows: only kernel launches on the current stream, so it can be captured in
        a HIP graph."""
        cfg, B = self.cfg, self.B
        J, lg, stride = exact.lane_shape(n)
        lanes = Lanes(n, lg, stride, 0)
        H, D = cfg.hidden, cfg.head_dim
        q_stride = cfg.heads * D
        scale = float(math.pow(D, -0.5))
        P = B.ptr
        B.call("embed", EmbedParams(lanes, P(self.embed), P(self.tokens), P(self.h), H))
        for li, L in enumerate(self.layers):
            m = self.mats[li]
            B.call("norm", NormParams(lanes, P(self.h), P(self.nx), P(L["norm_attn"]), H, cfg.rms_eps), J)
            B.call("qkv", QkvParams(lanes, P(self.nx), m["q"], m["k"], m["v"], P(self.q), q_stride, self.kv,
                                    P(self.rope), P(self.row_slot), P(self.row_pos), li, D), J)
            a = AttentionParams()
            a.l = lanes
            a.q, a.q_stride, a.out, a.out_cols = P(self.q), q_stride, P(self.attn), q_stride
            a.kv = self.kv
            a.row_slot, a.row_pos, a.items, a.item_count = P(self.row_slot), P(self.row_pos), P(self.items), item_count
            a.scratch, a.max_pages, a.rec_floats = P(self.scratch), self.max_pages, self.rec_floats
            a.layer, a.n_kv, a.n_q, a.head_dim, a.scale = li, cfg.kv_heads, cfg.repeat(), D, scale
            B.call("attention", a)
            B.call("gemm_residual", GemmResidualParams(lanes, P(self.attn), m["o"], P(self.h)), J)
            B.call("norm", NormParams(lanes, P(self.h), P(self.nx), P(L["norm_mlp"]), H, cfg.rms_eps), J)
            B.call("mlp13", Mlp13Params(lanes, P(self.nx), m["w1"], m["w3"], P(self.z)), J)
            B.call("gemm_residual", GemmResidualParams(lanes, P(self.z), m["w2"], P(self.h)), J)
        B.call("norm", NormParams(lanes, P(self.h), P(self.nx), P(self.norm_final), H, cfg.rms_eps), J)
        return J, lanes

    def launch_lm_greedy_all(self, n):
        """The greedy LM head over all n rows in lane order (self.nx), writing
        self.best; the caller initialises self.best to (-inf, -1) per row."""
        cJ, clg, cstride = exact.lane_shape(n)
        self.B.call("lm_greedy", LmGreedyParams(Lanes(n, clg, cstride, 0), self.B.ptr(self.nx), self.lm_mat,
                                                self.cfg.vocab, self.B.ptr(self.best)), cJ)

    def step(self, rows, greedy=(), full=()):
        """One step over rows [(slot, pos, token)]. Returns ([(index, value bits)]
        for the rows listed in `greedy`, [fp32 logits[vocab]] for those in `full`),
        both in list order."""
        cfg, B = self.cfg, self.B
        n = len(rows)
        item_count = self.upload(rows)
        J, lanes = self.launch_layers(n, item_count)
        H = cfg.hidden
        P = B.ptr

        def lm_input(wanted):
            """Lane shape of the wanted rows and the activations holding them in
            lane order (compacted unless they are all rows, in order)."""
            cJ, clg, cstride = exact.lane_shape(len(wanted))
            if len(wanted) == n:
                return cJ, Lanes(n, clg, cstride, 0), self.nx
            B.put(self.lm_rows, np.array(wanted, np.int32))
            B.call("compact", CompactParams(lanes, P(self.nx), P(self.lm_x), P(self.lm_rows), len(wanted), cstride, H))
            return cJ, Lanes(len(wanted), clg, cstride, 0), self.lm_x

        out_greedy, out_full = [], []
        if greedy:
            cJ, cl, x = lm_input(list(greedy))
            init = np.zeros((len(greedy), 2), np.int32)
            init[:, 0] = np.float32(-np.inf).view(np.int32)
            init[:, 1] = -1
            B.put(self.best, init.reshape(-1))
            B.call("lm_greedy", LmGreedyParams(cl, P(x), self.lm_mat, cfg.vocab, P(self.best)), cJ)
            b = B.get(self.best, 2 * len(greedy), np.int32).reshape(-1, 2)
            out_greedy = [(int(b[i, 1]), int(np.uint32(b[i, 0]))) for i in range(len(greedy))]
        if full:
            cJ, cl, x = lm_input(list(full))
            B.call("lm_full", LmFullParams(cl, P(x), self.lm_mat, P(self.logits)), cJ)
            rows_v = self.vocab_groups * 4
            lg = B.get(self.logits, rows_v * cl.stride, np.float32).reshape(rows_v, cl.stride)
            out_full = [lg[: cfg.vocab, i].copy() for i in range(len(full))]
        return out_greedy, out_full


def decode(engine: ExactEngine, prompts, new_tokens: int, slots=None, chunk: int | None = None, full_last=False):
    """Greedy decode of `prompts` (lists of token ids) together: prompt rows in
    chunks of at most `chunk` rows (positions ascending per sequence), then one
    row per sequence per step. Returns per sequence (tokens, value bits, and the
    full logits of the last step if full_last)."""
    slots = list(range(len(prompts))) if slots is None else slots
    chunk = chunk or engine.max_rows
    toks = [[] for _ in prompts]
    vals = [[] for _ in prompts]
    last = [None for _ in prompts]
    rows = [(s, p) for s in range(len(prompts)) for p in range(len(prompts[s]))]
    rows.sort(key=lambda r: r[1])
    for c0 in range(0, len(rows), chunk):
        part = rows[c0:c0 + chunk]
        step_rows = [(slots[s], p, prompts[s][p]) for s, p in part]
        want = [i for i, (s, p) in enumerate(part) if p == len(prompts[s]) - 1]
        g, _ = engine.step(step_rows, greedy=want)
        for i, (idx, val) in zip(want, g):
            s = part[i][0]
            toks[s].append(idx)
            vals[s].append(val)
    for step in range(new_tokens - 1):
        step_rows = [(slots[s], len(prompts[s]) + len(toks[s]) - 1, toks[s][-1]) for s in range(len(prompts))]
        idx = list(range(len(prompts)))
        g, f = engine.step(step_rows, greedy=idx, full=idx if (full_last and step == new_tokens - 2) else ())
        for s, (t, v) in enumerate(g):
            toks[s].append(t)
            vals[s].append(v)
        if f:
            last = f
    return toks, vals, last
