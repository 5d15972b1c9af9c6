"""Host-side mirror of stride's exact-path operator surface (src/kernels.h:146-155),
run on the GPU with the same bits as the reference's CPU exact path:

    k_embed(p)              k_norm(p, J)          k_qkv(p, J)
    k_attention(p)          k_gemm_residual(p, J) k_mlp13(p, J)
    k_compact(p)            k_lm_greedy(p, J)     k_lm_full(p, J)

J is 1 for a single row (stride 1) and 4 for lane groups of four
(src/engine.cpp:23-28). Parameter blocks are those of src/kernels.h (ctypes
structs in stride_amd._lib); pointers are device addresses. Launches go on
stride_amd.tc.kernel_stream(); errors raise StrideTcError.

Layout helpers: ``pack_groups`` packs a row-major bf16 matrix into the exact
path's four-row groups W[group][col][4] (src/model.cpp:94-111), ``rope_group_rows``
is the RoPE order of q/k/v (rows d, d+1, d+D/2, d+D/2+1 of a head per group,
src/model.cpp:168-174), ``dim_major`` lays activations out as A[dim*stride+lane].
"""
from __future__ import annotations

import ctypes as C

import numpy as np

from . import _lib, tc
from ._lib import (CompactParams, EmbedParams, GemmResidualParams, LmFullParams, LmGreedyParams, Mlp13Params,
                   NormParams, QkvParams)

try:
    import torch
except ImportError:  # layout helpers still work on numpy arrays
    torch = None


def _call(name: str, p, J=None) -> None:
    fn = getattr(_lib.load(), name)
    rc = fn(C.byref(p), tc.kernel_stream()) if J is None else fn(C.byref(p), J, tc.kernel_stream())
    _lib.check(rc)


def k_embed(p: EmbedParams) -> None: _call("stride_k_embed", p)
def k_norm(p: NormParams, J: int) -> None: _call("stride_k_norm", p, J)
def k_qkv(p: QkvParams, J: int) -> None: _call("stride_k_qkv", p, J)
def k_attention(p) -> None: _call("stride_k_attention", p)
def k_gemm_residual(p: GemmResidualParams, J: int) -> None: _call("stride_k_gemm_residual", p, J)
def k_mlp13(p: Mlp13Params, J: int) -> None: _call("stride_k_mlp13", p, J)
def k_compact(p: CompactParams) -> None: _call("stride_k_compact", p)
def k_lm_greedy(p: LmGreedyParams, J: int) -> None: _call("stride_k_lm_greedy", p, J)
def k_lm_full(p: LmFullParams, J: int) -> None: _call("stride_k_lm_full", p, J)


def lane_shape(rows: int):
    """(J, lane_groups, stride): one row runs J = 1 with stride 1, anything else
    lane groups of four (src/engine.cpp:23-28)."""
    if rows == 1:
        return 1, 1, 1
    g = (rows + 3) // 4
    return 4, g, 4 * g


def rope_group_rows(n: int, head_dim: int) -> np.ndarray:
    """Source row of packed row 4*group + slot for q/k/v: group g of head h holds
    rows h*D + (d0, d0+1, d0+D/2, d0+D/2+1), d0 = 2*(g mod D/4)."""
    D = head_dim
    idx = np.arange(n, dtype=np.int64)
    g, slot = idx // 4, idx % 4
    head, d0 = g // (D // 4), 2 * (g % (D // 4))
    off = np.where(slot < 2, d0 + slot, d0 + D // 2 + slot - 2)
    return head * D + off


def pack_groups(w, rows_order=None, groups: int | None = None):
    """Row-major [N][K] bf16 bits -> [groups][K][4]; rows past N are zero."""
    if rows_order is not None:
        w = w[rows_order if not (torch is not None and isinstance(w, torch.Tensor))
              else torch.as_tensor(rows_order, device=w.device)]
    n, k = w.shape
    g = groups if groups is not None else (n + 3) // 4
    if torch is not None and isinstance(w, torch.Tensor):
        out = torch.zeros((g * 4, k), dtype=w.dtype, device=w.device)
        out[:n] = w
        return out.reshape(g, 4, k).permute(0, 2, 1).contiguous()
    out = np.zeros((g * 4, k), dtype=w.dtype)
    out[:n] = w
    return np.ascontiguousarray(out.reshape(g, 4, k).transpose(0, 2, 1))


def dim_major(a, stride: int):
    """Row-major [rows][dim] -> dim-major [dim][stride] (lanes past rows zero)."""
    rows, dim = a.shape
    if torch is not None and isinstance(a, torch.Tensor):
        out = torch.zeros((dim, stride), dtype=a.dtype, device=a.device)
        out[:, :rows] = a.T
        return out
    out = np.zeros((dim, stride), dtype=a.dtype)
    out[:, :rows] = a.T
    return out


def mat(w_groups, cols: int) -> tc.GemmMat:
    return tc.GemmMat(tc.ptr(w_groups), int(w_groups.shape[0]), cols)


def lanes(rows: int) -> tc.Lanes:
    J, g, stride = lane_shape(rows)
    return tc.Lanes(rows, g, stride, 0)
