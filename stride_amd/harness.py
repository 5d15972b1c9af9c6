"""Convenience runners over the operator surface for torch device tensors.

Each runner fills the reference-shaped parameter block for one call of the C ABI
and launches it on the current stream; tensors must already be in the tile
layouts of stride_amd.layout. Used by the tests, the benchmark and smoke().
"""
from __future__ import annotations

from dataclasses import dataclass

import torch

from . import tc
from .tc import (GemmMat, KvRef, TcGemmResidualParams, TcLmFullParams, TcLmGreedyParams, TcMlp13Params,
                 TcQkvParams, lanes, mat, ptr)

U16 = torch.int16  # bf16 bit patterns travel as int16 tensors


def gemm_residual(w_tiles, x_tiles, h_tiles, rows: int, r: int = 1, lt: int = 1) -> None:
    p = TcGemmResidualParams(lanes(rows), ptr(x_tiles), mat(w_tiles), ptr(h_tiles))
    tc.tc_gemm_residual(p, r, lt)


def lm_full(w_tiles, x_tiles, rows: int, out=None):
    T = (rows + 15) // 16
    if out is None:
        out = torch.empty((w_tiles.shape[0], T, 16, 16), dtype=torch.float32, device=x_tiles.device)
    p = TcLmFullParams(lanes(rows), ptr(x_tiles), mat(w_tiles), ptr(out))
    tc.tc_lm_full(p, 1)
    return out


def mlp13(w1_tiles, w3_tiles, x_tiles, rows: int, out=None, r: int = 1, lt: int = 1):
    T = (rows + 15) // 16
    if out is None:
        out = torch.zeros((T, w1_tiles.shape[0], 16, 16), dtype=U16, device=x_tiles.device)
    p = TcMlp13Params(lanes(rows), ptr(x_tiles), mat(w1_tiles), mat(w3_tiles), ptr(out))
    tc.tc_mlp13(p, r, lt)
    return out


def best_init(rows: int, device) -> torch.Tensor:
    """BestEntry[rows] = {-inf, -1} as the engine uploads it (src/engine.cpp:423-424),
    stored as int32 pairs (value bits, index)."""
    b = torch.empty((rows, 2), dtype=torch.int32, device=device)
    b[:, 0] = -8388608  # 0xFF800000 = -inf
    b[:, 1] = -1
    return b


# {-inf, -1} as one little-endian 64-bit word (value bits low, index high).
BEST_INIT_WORD = (-1 << 32) | 0xFF800000


def best_reset(best: torch.Tensor) -> torch.Tensor:
    """Re-arms a BestEntry buffer to {-inf, -1} in place with a fill kernel. (A
    device-to-device copy from a template would become a memcpy node in a
    captured HIP graph, which measured about 20 us per replay on MI355X against
    a few for the kernel.)"""
    best.view(torch.int64).fill_(BEST_INIT_WORD)
    return best


def lm_greedy(w_tiles, x_tiles, rows: int, vocab: int, best=None, r: int = 1, lt: int = 1):
    if best is None:
        best = best_init(rows, x_tiles.device)
    p = TcLmGreedyParams(lanes(rows), ptr(x_tiles), mat(w_tiles), vocab, ptr(best))
    tc.tc_lm_greedy(p, r, lt)
    return best


def best_split(best: torch.Tensor):
    """(values fp32, indices int32) from a BestEntry buffer."""
    b = best.cpu()
    return b[:, 0].contiguous().view(torch.float32), b[:, 1].contiguous()


@dataclass
class PagedKv:
    """A paged KV arena in the reference layout [block][layer][K|V][group][token][dim]
    (src/kernels.h:10, src/kv_cache.cpp:10-40), bf16 elements."""

    arena: torch.Tensor
    table: torch.Tensor
    ref: KvRef
    page_tokens: int
    max_blocks: int

    @staticmethod
    def create(slots: int, max_ctx: int, kv_heads: int, head_dim: int, layers: int, page_tokens: int, device,
               shuffle_seed: int = 0) -> "PagedKv":
        max_blocks = (max_ctx + page_tokens - 1) // page_tokens
        group = page_tokens * head_dim
        which = group * kv_heads
        layer = which * 2
        block = layer * layers
        nblocks = slots * max_blocks
        order = torch.arange(nblocks, dtype=torch.int32)
        if shuffle_seed:
            g = torch.Generator().manual_seed(shuffle_seed)
            order = order[torch.randperm(nblocks, generator=g)]
        table = order.reshape(slots, max_blocks).contiguous().to(device)
        arena = torch.zeros(nblocks * block, dtype=U16, device=device)
        ref = KvRef(ptr(arena), ptr(table), block, layer, which, group, max_blocks, head_dim)
        return PagedKv(arena, table, ref, page_tokens, max_blocks)

    @property
    def slots(self) -> int:
        return int(self.table.shape[0])

    @property
    def capacity(self) -> int:
        """Positions per slot."""
        return self.max_blocks * self.page_tokens

    def gather(self, layer: int, which: int, slots, positions, kv_heads: int, head_dim: int) -> torch.Tensor:
        """Dense [rows][kv_heads * head_dim] bf16 bits of the entries at (slot, pos)."""
        r = self.ref
        tab = self.table.cpu()
        rows = []
        for s, p in zip(list(slots), list(positions)):
            blk = int(tab[int(s), int(p) // self.page_tokens])
            tok = int(p) % self.page_tokens
            base = blk * r.block_elems + layer * r.layer_elems + which * r.which_elems + tok * head_dim
            idx = torch.tensor([base + h * r.group_elems + d for h in range(kv_heads) for d in range(head_dim)],
                               device=self.arena.device)
            rows.append(self.arena[idx])
        return torch.stack(rows)


    def fill_dense(self, layer: int, which: int, dense) -> None:
        """Write dense bf16 bits [slots][kv_heads][cap][head_dim] (cap <= pages * page
        tokens) into the arena through the page table."""
        slots, kvh, cap, hd = dense.shape
        r = self.ref
        dev = self.arena.device
        pos = torch.arange(cap, device=dev)
        blk = self.table.long()[:, (pos // self.page_tokens)]                       # [slots][cap]
        base = blk * r.block_elems + layer * r.layer_elems + which * r.which_elems + (pos % self.page_tokens) * hd
        idx = (base[:, None, :, None] + torch.arange(kvh, device=dev)[None, :, None, None] * r.group_elems
               + torch.arange(hd, device=dev)[None, None, None, :])
        self.arena[idx.reshape(-1)] = dense.reshape(-1).to(dev)


def gemm_f32x(w_tiles, x_f32, rows: int, y_out=None, workspace=None):
    """y tiles (h layout, fp32) = W x for row-major fp32 activations x [rows][K]."""
    lt = (rows + 15) // 16
    k = int(w_tiles.shape[1]) * 16
    dev = x_f32.device
    if y_out is None:
        y_out = torch.empty((lt, w_tiles.shape[0], 16, 16), dtype=torch.float32, device=dev)
    if workspace is None:
        workspace = torch.empty(2 * lt * 16 * k, dtype=U16, device=dev)
    p = tc.TcGemmF32xParams(lanes(rows), ptr(x_f32), mat(w_tiles), ptr(y_out), ptr(workspace))
    tc.tc_gemm_f32x(p)
    return y_out


def gemm_f32x_noalloc(w_tiles, x_f32, rows: int, y_out):
    """gemm_f32x through the allocation-free entry point: y_out (h-layout fp32
    tiles, at least ceil(rows/16) lane tiles) is overwritten."""
    p = tc.TcGemmF32xParams(lanes(rows), ptr(x_f32), mat(w_tiles), ptr(y_out), None)
    tc.tc_gemm_f32x_noalloc(p)
    return y_out


def embed(emb_tiles, tokens, rows: int, dim: int, h_out=None):
    """tc_embed: lane j of fp32 h tiles <- embedding row tokens[j]."""
    lt = (rows + 15) // 16
    if h_out is None:
        h_out = torch.zeros((lt, dim // 16, 16, 16), dtype=torch.float32, device=emb_tiles.device)
    p = tc.TcEmbedParams()
    p.l = lanes(rows)
    p.embed, p.tokens, p.h, p.dim = ptr(emb_tiles), ptr(tokens), ptr(h_out), dim
    tc.tc_embed(p)
    return h_out


def norm(h_tiles, rows: int, weight, eps: float, per_lane: bool = True, x_out=None):
    """tc_norm: bf16 x tiles = RMSNorm(h tiles) * weight."""
    if x_out is None:
        x_out = torch.full(tuple(h_tiles.shape), 0x7FFF, dtype=U16, device=h_tiles.device)
    p = tc.TcNormParams()
    p.l = lanes(rows)
    p.h, p.x, p.weight = ptr(h_tiles), ptr(x_out), ptr(weight)
    p.dim, p.eps = int(h_tiles.shape[1]) * 16, eps
    tc.tc_norm(p, per_lane)
    return x_out


def compact(in_tiles, lm_rows, out_tiles=None):
    """tc_compact: out lane l <- in lane lm_rows[l]."""
    count = int(lm_rows.numel())
    if out_tiles is None:
        out_tiles = torch.zeros(((count + 15) // 16, in_tiles.shape[1], 16, 16), dtype=U16, device=in_tiles.device)
    p = tc.TcCompactParams()
    p.l = lanes(int(in_tiles.shape[0]) * 16)
    p.in_, p.out, p.lm_rows = ptr(in_tiles), ptr(out_tiles), ptr(lm_rows)
    p.lm_count, p.col_tiles = count, int(in_tiles.shape[1])
    tc.tc_compact(p)
    return out_tiles


def attention_one_kernel_fits(max_pages: int, head_dim: int, page_tokens: int) -> bool:
    """Whether tc_attention's one-kernel form serves rows of up to max_pages
    64-position pages (the library's LDS budget: the records and page factors,
    the row's KV page numbers and the staging of four waves within 159 KiB)."""
    blocks = (max_pages * 64 + page_tokens - 1) // page_tokens
    dynamic = max_pages * (8 + 4 * head_dim + 4) * 4 + blocks * 4
    static = 4 * 64 * 16 + 4 * 64 * head_dim * 2 + 320 // 8 + 4 * 4
    return dynamic + static <= 159 * 1024


def attention(q, kv: PagedKv, row_slot, row_pos, n_kv: int, head_dim: int, scale: float, layer: int = 0,
              max_pages: int = 32, out_tiles=None, items=None, scratch=None, one_kernel: bool = False):
    """tc_attention over the (row, page) list `items` (default: every page of every
    row, the engine's list, src/engine.cpp:93-103). q: [rows][n_kv*4*head_dim] fp32.
    Returns bf16 x tiles. one_kernel: pass item_count = -1 instead (every page of
    every row, no item list, no scratch)."""
    rows = int(q.shape[0])
    cols = n_kv * 4 * head_dim
    dev = q.device
    if one_kernel:
        if out_tiles is None:
            out_tiles = torch.zeros(((rows + 15) // 16, cols // 16, 16, 16), dtype=U16, device=dev)
        p = tc.AttentionParams()
        p.l = lanes(rows)
        p.q, p.q_stride, p.out, p.out_cols = ptr(q), cols, ptr(out_tiles), cols
        p.kv = kv.ref
        p.row_slot, p.row_pos, p.items, p.item_count = ptr(row_slot), ptr(row_pos), None, -1
        p.scratch, p.max_pages, p.rec_floats = None, max_pages, 4 * head_dim + 8
        p.layer, p.n_kv, p.n_q, p.head_dim, p.scale = layer, n_kv, 4, head_dim, scale
        tc.tc_attention(p)
        return out_tiles
    if items is None:
        pos = row_pos.cpu().tolist()
        items = torch.tensor([[j, pg] for j in range(rows) for pg in range((pos[j] >> 6) + 1)], dtype=torch.int32,
                             device=dev).reshape(-1)
    rec = 4 * head_dim + 8
    if scratch is None:
        scratch = torch.zeros(rows * n_kv * max_pages * rec, dtype=torch.float32, device=dev)
    if out_tiles is None:
        out_tiles = torch.zeros(((rows + 15) // 16, cols // 16, 16, 16), dtype=U16, device=dev)
    p = tc.AttentionParams()
    p.l = lanes(rows)
    p.q, p.q_stride, p.out, p.out_cols = ptr(q), cols, ptr(out_tiles), cols
    p.kv = kv.ref
    p.row_slot, p.row_pos, p.items, p.item_count = ptr(row_slot), ptr(row_pos), ptr(items), int(items.numel()) // 2
    p.scratch, p.max_pages, p.rec_floats = ptr(scratch), max_pages, rec
    p.layer, p.n_kv, p.n_q, p.head_dim, p.scale = layer, n_kv, 4, head_dim, scale
    tc.tc_attention(p)
    return out_tiles


def qkv(wq_tiles, wk_tiles, wv_tiles, x_tiles, rows: int, head_dim: int, rope, row_slot, row_pos, kv: PagedKv,
        layer: int = 0, q_out=None):
    nq = wq_tiles.shape[0] * 16
    if q_out is None:
        q_out = torch.zeros((max(rows, 1), nq), dtype=torch.float32, device=x_tiles.device)
    p = TcQkvParams()
    p.l = lanes(rows)
    p.x = ptr(x_tiles)
    p.q, p.k, p.v = mat(wq_tiles), mat(wk_tiles), mat(wv_tiles)
    p.q_out = ptr(q_out)
    p.q_stride = nq
    p.kv = kv.ref
    p.rope = ptr(rope)
    p.row_slot = ptr(row_slot)
    p.row_pos = ptr(row_pos)
    p.layer = layer
    p.head_dim = head_dim
    tc.tc_qkv(p)
    return q_out
