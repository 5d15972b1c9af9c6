"""Tile layouts of the stride tensor-core path, for numpy arrays and torch tensors.

    weights  W[row tile][col tile][16 rows][16 cols]    pack_tiles  (src/model.cpp:114-133)
    x / z    X[lane tile][col tile][16 lanes][16 cols]  lane_tiles  (src/kernels_tc.cu:8-11)
    h        the same grid as x, fp32                   lane_tiles
    logits   [row tile][lane tile][16 rows][16 lanes]   untile_logits (src/engine.cpp:449-460)

Row orders: plain (row tile rt, slot s -> row 16*rt + s), RoPE (a row tile holds
the eight pairs (d0+i, d0+D/2+i), src/model.cpp:178-183) and vocabulary padding
(rows past the vocabulary are zero, src/model.cpp:219-226).
"""
from __future__ import annotations

import numpy as np

try:  # torch is plumbing for device memory; numpy-only callers do not need it
    import torch
except Exception:  # pragma: no cover
    torch = None


def _is_torch(a) -> bool:
    return torch is not None and isinstance(a, torch.Tensor)


def _pad_rows(a, rows: int):
    if a.shape[0] == rows:
        return a
    if _is_torch(a):
        out = torch.zeros((rows,) + tuple(a.shape[1:]), dtype=a.dtype, device=a.device)
    else:
        out = np.zeros((rows,) + a.shape[1:], dtype=a.dtype)
    out[: a.shape[0]] = a
    return out


def _tile(a, rows_padded: int):
    """[R][K] -> [R/16][K/16][16][16] (row-in-tile, col-in-tile)."""
    a = _pad_rows(a, rows_padded)
    r, k = a.shape
    a = a.reshape(r // 16, 16, k // 16, 16)
    if _is_torch(a):
        return a.permute(0, 2, 1, 3).contiguous()
    return np.ascontiguousarray(a.transpose(0, 2, 1, 3))


def _untile(t, rows: int):
    rt, ct = t.shape[0], t.shape[1]
    if _is_torch(t):
        a = t.permute(0, 2, 1, 3).reshape(rt * 16, ct * 16)
    else:
        a = t.transpose(0, 2, 1, 3).reshape(rt * 16, ct * 16)
    return a[:rows]


def plain_rows(n: int) -> np.ndarray:
    return np.arange(n, dtype=np.int64)


def rope_rows(n: int, head_dim: int) -> np.ndarray:
    """Source row for each packed row: packed row 16*rt + slot holds HF row
    head*D + (d0 + slot) for slot < 8 and head*D + (d0 + D/2 + slot - 8) otherwise,
    with head = rt / (D/16), d0 = 8 * (rt % (D/16))."""
    D = head_dim
    per = D // 16
    idx = np.arange(n, dtype=np.int64)
    rt, slot = idx // 16, idx % 16
    head, d0 = rt // per, (rt % per) * 8
    return head * D + np.where(slot < 8, d0 + slot, d0 + D // 2 + slot - 8)


def pack_tiles(w, rows_order: np.ndarray | None = None, row_tiles: int | None = None):
    """Row-major bf16 weights [N][K] -> packed tiles. ``rows_order`` permutes
    source rows (RoPE); ``row_tiles`` pads with zero rows (vocabulary padding)."""
    if rows_order is not None:
        idx = rows_order if not _is_torch(w) else torch.as_tensor(rows_order, device=w.device)
        w = w[idx]
    n = w.shape[0]
    rt = row_tiles if row_tiles is not None else (n + 15) // 16
    return _tile(w, rt * 16)


def lane_tiles(a, lane_groups: int | None = None):
    """Row-major activations [M][K] (bf16 bits or fp32) -> lane tiles, zero-padded
    to 16 * lane_groups lanes."""
    m = a.shape[0]
    t = lane_groups if lane_groups is not None else (m + 15) // 16
    return _tile(a, t * 16)


def untile_lanes(t, rows: int):
    """Lane tiles -> row-major [rows][K]."""
    return _untile(t, rows)


def untile_logits(t, rows: int, vocab: int):
    """Logits tiles [rt][lt][16 rows][16 lanes] -> [rows][vocab]."""
    rt, lt = t.shape[0], t.shape[1]
    if _is_torch(t):
        a = t.permute(1, 3, 0, 2).reshape(lt * 16, rt * 16)
    else:
        a = t.transpose(1, 3, 0, 2).reshape(lt * 16, rt * 16)
    return a[:rows, :vocab]


def unpack_rows(tiles, rows_order: np.ndarray | None = None):
    """Inverse of pack_tiles (for tests): packed tiles -> row-major [N][K]."""
    a = _untile(tiles, tiles.shape[0] * 16)
    if rows_order is None:
        return a
    out = np.zeros_like(a) if not _is_torch(a) else torch.zeros_like(a)
    out[rows_order] = a[: len(rows_order)]
    return out
