"""Host-side mirror of stride's tensor-core operator surface (src/kernels_tc.h:79-87).

Same names, same parameter blocks, same argument meaning as the reference:

    tc_qkv(p)                                  src/kernels_tc.h:81
    tc_gemm_residual(p, row_tiles, lane_tiles) src/kernels_tc.h:83
    tc_mlp13(p, row_tiles, lane_tiles)         src/kernels_tc.h:84
    tc_lm_greedy(p, row_tiles, lane_tiles)     src/kernels_tc.h:86
    tc_lm_full(p, lane_tiles_per_block)        src/kernels_tc.h:87
    tc_embed(p)                                src/kernels_tc.h:79
    tc_norm(p, per_lane)                       src/kernels_tc.h:80
    tc_attention(p)                            src/kernels_tc.h:82
    tc_compact(p)                              src/kernels_tc.h:85

Launches are asynchronous on ``kernel_stream()`` (the reference keeps one stream,
src/kernels.cu:457-460); by default that is torch's current HIP stream. An error
raises StrideTcError, as the reference's check() throws std::runtime_error.
Pointers are device addresses: ``mat``/``lanes`` build the structs from torch
tensors already laid out in the tile formats of stride_amd.layout.
"""
from __future__ import annotations

import ctypes as C

from . import _lib
from ._lib import (AttentionParams, BestEntry, GemmMat, KvRef, Lanes, StrideTcError, TcCompactParams, TcEmbedParams,
                   TcGemmF32xParams, TcGemmResidualParams, TcLmFullParams, TcLmGreedyParams, TcMlp13Params, TcNormParams, TcQkvParams)

__all__ = [
    "BestEntry", "GemmMat", "KvRef", "Lanes", "StrideTcError", "TcGemmResidualParams", "TcLmFullParams",
    "TcLmGreedyParams", "TcMlp13Params", "TcQkvParams", "tc_qkv", "tc_gemm_residual", "tc_mlp13", "tc_lm_greedy",
    "tc_lm_full", "kernel_stream", "set_kernel_stream", "mat", "lanes", "ptr", "split_count", "AttentionParams",
    "TcCompactParams", "TcEmbedParams", "TcNormParams", "TcGemmF32xParams", "tc_gemm_f32x", "tc_gemm_f32x_noalloc", "tc_embed", "tc_norm", "tc_attention", "tc_compact",
]

_stream = None  # None -> torch's current stream at call time


def set_kernel_stream(stream) -> None:
    """Select the stream every entry point launches on (an int handle, a
    torch.cuda.Stream, or None for torch's current stream)."""
    global _stream
    _stream = stream


def kernel_stream() -> int:
    s = _stream
    if s is None:
        import torch

        return torch.cuda.current_stream().cuda_stream
    return int(getattr(s, "cuda_stream", s))


def ptr(t) -> int:
    """Device address of a torch tensor (0 for None)."""
    return 0 if t is None else int(t.data_ptr())


def lanes(rows: int) -> Lanes:
    """Lanes{rows, ceil(rows/16), 0, 0} as the engine builds it (src/engine.cpp:303-304)."""
    return Lanes(rows, (rows + 15) // 16, 0, 0)


def mat(tiles, cols: int | None = None) -> GemmMat:
    """GemmMat for packed weight tiles [rt][ct][16][16]."""
    rt, ct = int(tiles.shape[0]), int(tiles.shape[1])
    return GemmMat(ptr(tiles), rt, cols if cols is not None else ct * 16)


def split_count(n: int, k: int) -> int:
    return _lib.split_count(n, k)


def _lib_():
    return _lib.load()


def tc_qkv(p: TcQkvParams) -> None:
    _lib.check(_lib_().stride_tc_qkv(C.byref(p), kernel_stream()))


def tc_gemm_residual(p: TcGemmResidualParams, row_tiles_per_warp: int = 1, lane_tiles_per_warp: int = 1) -> None:
    _lib.check(_lib_().stride_tc_gemm_residual(C.byref(p), row_tiles_per_warp, lane_tiles_per_warp, kernel_stream()))


def tc_mlp13(p: TcMlp13Params, row_tiles_per_warp: int = 1, lane_tiles_per_warp: int = 1) -> None:
    _lib.check(_lib_().stride_tc_mlp13(C.byref(p), row_tiles_per_warp, lane_tiles_per_warp, kernel_stream()))


def tc_lm_greedy(p: TcLmGreedyParams, row_tiles_per_warp: int = 1, lane_tiles_per_warp: int = 1) -> None:
    _lib.check(_lib_().stride_tc_lm_greedy(C.byref(p), row_tiles_per_warp, lane_tiles_per_warp, kernel_stream()))


def tc_lm_full(p: TcLmFullParams, lane_tiles_per_block: int = 1) -> None:
    _lib.check(_lib_().stride_tc_lm_full(C.byref(p), lane_tiles_per_block, kernel_stream()))


def tc_embed(p: TcEmbedParams) -> None:
    _lib.check(_lib_().stride_tc_embed(C.byref(p), kernel_stream()))


def tc_norm(p: TcNormParams, per_lane: bool = True) -> None:
    _lib.check(_lib_().stride_tc_norm(C.byref(p), 1 if per_lane else 0, kernel_stream()))


def tc_attention(p: AttentionParams) -> None:
    _lib.check(_lib_().stride_tc_attention(C.byref(p), kernel_stream()))


def tc_compact(p: TcCompactParams) -> None:
    _lib.check(_lib_().stride_tc_compact(C.byref(p), kernel_stream()))


def tc_gemm_f32x(p: TcGemmF32xParams) -> None:
    """y = W x for fp32 activations (no reference counterpart; see include/stride_tc.h)."""
    _lib.check(_lib_().stride_tc_gemm_f32x(C.byref(p), kernel_stream()))


def tc_gemm_f32x_noalloc(p: TcGemmF32xParams) -> None:
    """tc_gemm_f32x staged in the library's device scratch (p.workspace must be
    null): allocates nothing, for callers that cannot allocate."""
    _lib.check(_lib_().stride_tc_gemm_f32x_noalloc(C.byref(p), kernel_stream()))
