"""ctypes binding of libstride_tc.so (the C ABI declared in include/stride_tc.h).

The Structure classes mirror the reference's POD parameter blocks byte for byte
(src/kernels.h:23-46, 79-98, 125-128; src/kernels_tc.h:10-77); ``check_layout`` asserts
the sizes the C++ side static_asserts. Loading fails loudly: there is no fallback
path, so a missing or stale library is an error, never a silent CPU substitute.
"""
from __future__ import annotations

import ctypes as C
import os

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libstride_tc.so")

EINVAL = 0x5354


class GemmMat(C.Structure):  # src/kernels.h:23-27
    _fields_ = [("w", C.c_void_p), ("groups", C.c_int32), ("cols", C.c_int32)]


class KvRef(C.Structure):  # src/kernels.h:30-39
    _fields_ = [
        ("arena", C.c_void_p),
        ("table", C.c_void_p),
        ("block_elems", C.c_int64),
        ("layer_elems", C.c_int64),
        ("which_elems", C.c_int64),
        ("group_elems", C.c_int64),
        ("max_blocks", C.c_int32),
        ("head_dim", C.c_int32),
    ]


class Lanes(C.Structure):  # src/kernels.h:41-46
    _fields_ = [("rows", C.c_int32), ("lane_groups", C.c_int32), ("stride", C.c_int32), ("bug", C.c_int32)]


class BestEntry(C.Structure):  # src/kernels.h:125-128
    _fields_ = [("value", C.c_float), ("index", C.c_int32)]


class TcQkvParams(C.Structure):  # src/kernels_tc.h:27-39
    _fields_ = [
        ("l", Lanes),
        ("x", C.c_void_p),
        ("q", GemmMat),
        ("k", GemmMat),
        ("v", GemmMat),
        ("q_out", C.c_void_p),
        ("q_stride", C.c_int32),
        ("kv", KvRef),
        ("rope", C.c_void_p),
        ("row_slot", C.c_void_p),
        ("row_pos", C.c_void_p),
        ("layer", C.c_int32),
        ("head_dim", C.c_int32),
    ]


class TcGemmResidualParams(C.Structure):  # src/kernels_tc.h:41-46
    _fields_ = [("l", Lanes), ("x", C.c_void_p), ("m", GemmMat), ("h", C.c_void_p)]


class TcMlp13Params(C.Structure):  # src/kernels_tc.h:48-53
    _fields_ = [("l", Lanes), ("x", C.c_void_p), ("w1", GemmMat), ("w3", GemmMat), ("z", C.c_void_p)]


class TcLmGreedyParams(C.Structure):  # src/kernels_tc.h:64-70
    _fields_ = [("l", Lanes), ("x", C.c_void_p), ("m", GemmMat), ("vocab", C.c_int32), ("best", C.c_void_p)]


class TcLmFullParams(C.Structure):  # src/kernels_tc.h:72-77
    _fields_ = [("l", Lanes), ("x", C.c_void_p), ("m", GemmMat), ("logits", C.c_void_p)]


class TcGemmF32xParams(C.Structure):  # no reference counterpart (fp32 activations)
    _fields_ = [("l", Lanes), ("x", C.c_void_p), ("m", GemmMat), ("y", C.c_void_p), ("workspace", C.c_void_p)]


class TcEmbedParams(C.Structure):  # src/kernels_tc.h:10-16
    _fields_ = [("l", Lanes), ("embed", C.c_void_p), ("tokens", C.c_void_p), ("h", C.c_void_p), ("dim", C.c_int32)]


class TcNormParams(C.Structure):  # src/kernels_tc.h:18-25
    _fields_ = [("l", Lanes), ("h", C.c_void_p), ("x", C.c_void_p), ("weight", C.c_void_p), ("dim", C.c_int32),
                ("eps", C.c_float)]


class TcCompactParams(C.Structure):  # src/kernels_tc.h:55-62
    _fields_ = [("l", Lanes), ("in_", C.c_void_p), ("out", C.c_void_p), ("lm_rows", C.c_void_p),
                ("lm_count", C.c_int32), ("col_tiles", C.c_int32)]


class AttentionParams(C.Structure):  # src/kernels.h:79-98
    _fields_ = [
        ("l", Lanes),
        ("q", C.c_void_p),
        ("q_stride", C.c_int32),
        ("out", C.c_void_p),
        ("out_cols", C.c_int32),
        ("kv", KvRef),
        ("row_slot", C.c_void_p),
        ("row_pos", C.c_void_p),
        ("items", C.c_void_p),
        ("item_count", C.c_int32),
        ("scratch", C.c_void_p),
        ("max_pages", C.c_int32),
        ("rec_floats", C.c_int32),
        ("layer", C.c_int32),
        ("n_kv", C.c_int32),
        ("n_q", C.c_int32),
        ("head_dim", C.c_int32),
        ("scale", C.c_float),
    ]


# Exact-path parameter blocks (include/stride_exact.h, src/kernels.h:48-143).
class EmbedParams(C.Structure):
    _fields_ = [("l", Lanes), ("embed", C.c_void_p), ("tokens", C.c_void_p), ("h", C.c_void_p), ("dim", C.c_int32)]


class NormParams(C.Structure):
    _fields_ = [("l", Lanes), ("in_", C.c_void_p), ("out", C.c_void_p), ("weight", C.c_void_p), ("dim", C.c_int32),
                ("eps", C.c_float)]


class QkvParams(C.Structure):
    _fields_ = [("l", Lanes), ("x", C.c_void_p), ("q", GemmMat), ("k", GemmMat), ("v", GemmMat), ("q_out", C.c_void_p),
                ("q_stride", C.c_int32), ("kv", KvRef), ("rope", C.c_void_p), ("row_slot", C.c_void_p),
                ("row_pos", C.c_void_p), ("layer", C.c_int32), ("head_dim", C.c_int32)]


class GemmResidualParams(C.Structure):
    _fields_ = [("l", Lanes), ("x", C.c_void_p), ("m", GemmMat), ("h", C.c_void_p)]


class Mlp13Params(C.Structure):
    _fields_ = [("l", Lanes), ("x", C.c_void_p), ("w1", GemmMat), ("w3", GemmMat), ("z", C.c_void_p)]


class CompactParams(C.Structure):
    _fields_ = [("l", Lanes), ("in_", C.c_void_p), ("out", C.c_void_p), ("lm_rows", C.c_void_p),
                ("lm_count", C.c_int32), ("lm_stride", C.c_int32), ("dim", C.c_int32)]


class LmGreedyParams(C.Structure):
    _fields_ = [("l", Lanes), ("x", C.c_void_p), ("m", GemmMat), ("vocab", C.c_int32), ("best", C.c_void_p)]


class LmFullParams(C.Structure):
    _fields_ = [("l", Lanes), ("x", C.c_void_p), ("m", GemmMat), ("logits", C.c_void_p)]


EXACT_ENTRIES = {  # name -> (params type, takes J)
    "stride_k_embed": (EmbedParams, False),
    "stride_k_norm": (NormParams, True),
    "stride_k_qkv": (QkvParams, True),
    "stride_k_attention": (AttentionParams, False),
    "stride_k_gemm_residual": (GemmResidualParams, True),
    "stride_k_mlp13": (Mlp13Params, True),
    "stride_k_compact": (CompactParams, False),
    "stride_k_lm_greedy": (LmGreedyParams, True),
    "stride_k_lm_full": (LmFullParams, True),
}


# Symbols the library must export (everything include/stride_tc.h and
# include/stride_exact.h declare).
EXPORTS = (
    "stride_tc_qkv",
    "stride_tc_gemm_residual",
    "stride_tc_mlp13",
    "stride_tc_lm_greedy",
    "stride_tc_lm_full",
    "stride_tc_gemm_f32x",
    "stride_tc_gemm_f32x_noalloc",
    "stride_tc_f32x_scratch_elems",
    "stride_tc_embed",
    "stride_tc_norm",
    "stride_tc_attention",
    "stride_tc_compact",
    "stride_tc_split_count",
    "stride_tc_last_error",
    "stride_tc_version",
    "stride_tc_set_stream_config",
    "stride_tc_stream_config_count",
    "stride_tc_pipe_config_count",
    "stride_tc_dec_config_count",
    "stride_tc_stream_config",
    "stride_tc_last_stream_config",
) + tuple(EXACT_ENTRIES)


def check_layout() -> None:
    """Sizes and offsets the C++ side static_asserts (reference PODs on x86-64)."""
    assert C.sizeof(GemmMat) == 16
    assert C.sizeof(KvRef) == 56
    assert C.sizeof(Lanes) == 16
    assert C.sizeof(BestEntry) == 8
    assert TcQkvParams.kv.offset == 88 and C.sizeof(TcQkvParams) == 176
    assert C.sizeof(TcGemmResidualParams) == 48
    assert C.sizeof(TcMlp13Params) == 64
    assert C.sizeof(TcLmGreedyParams) == 56
    assert C.sizeof(TcLmFullParams) == 48
    assert C.sizeof(TcGemmF32xParams) == 56
    assert C.sizeof(TcEmbedParams) == 48 and C.sizeof(TcNormParams) == 48 and C.sizeof(TcCompactParams) == 48
    assert AttentionParams.kv.offset == 48 and C.sizeof(AttentionParams) == 176
    assert C.sizeof(EmbedParams) == 48 and C.sizeof(NormParams) == 48
    assert QkvParams.kv.offset == 88 and QkvParams.rope.offset == 144 and C.sizeof(QkvParams) == 176
    assert C.sizeof(GemmResidualParams) == 48 and C.sizeof(Mlp13Params) == 64 and C.sizeof(CompactParams) == 56
    assert LmGreedyParams.best.offset == 48 and C.sizeof(LmGreedyParams) == 56 and C.sizeof(LmFullParams) == 48


class StrideTcError(RuntimeError):
    """Raised when an entry point returns nonzero (the reference's device.cu
    check() throws std::runtime_error for the same condition)."""


_lib = None


def load(path: str = LIB_PATH) -> C.CDLL:
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(path):
        raise ImportError(
            f"libstride_tc.so not found at {path}; build it with "
            "`python -c 'import __graft_entry__ as g; g.build()'` (there is no fallback path)")
    lib = C.CDLL(path)
    for name in EXPORTS:
        getattr(lib, name)  # raises AttributeError if a symbol is missing
    vp = C.c_void_p
    lib.stride_tc_qkv.argtypes = [C.POINTER(TcQkvParams), vp]
    lib.stride_tc_gemm_residual.argtypes = [C.POINTER(TcGemmResidualParams), C.c_int, C.c_int, vp]
    lib.stride_tc_mlp13.argtypes = [C.POINTER(TcMlp13Params), C.c_int, C.c_int, vp]
    lib.stride_tc_lm_greedy.argtypes = [C.POINTER(TcLmGreedyParams), C.c_int, C.c_int, vp]
    lib.stride_tc_lm_full.argtypes = [C.POINTER(TcLmFullParams), C.c_int, vp]
    lib.stride_tc_gemm_f32x.argtypes = [C.POINTER(TcGemmF32xParams), vp]
    lib.stride_tc_gemm_f32x_noalloc.argtypes = [C.POINTER(TcGemmF32xParams), vp]
    lib.stride_tc_f32x_scratch_elems.argtypes = []
    lib.stride_tc_f32x_scratch_elems.restype = C.c_int
    lib.stride_tc_embed.argtypes = [C.POINTER(TcEmbedParams), vp]
    lib.stride_tc_norm.argtypes = [C.POINTER(TcNormParams), C.c_int, vp]
    lib.stride_tc_attention.argtypes = [C.POINTER(AttentionParams), vp]
    lib.stride_tc_compact.argtypes = [C.POINTER(TcCompactParams), vp]
    for name in ("stride_tc_qkv", "stride_tc_gemm_residual", "stride_tc_mlp13", "stride_tc_lm_greedy",
                 "stride_tc_lm_full", "stride_tc_gemm_f32x", "stride_tc_gemm_f32x_noalloc", "stride_tc_embed", "stride_tc_norm", "stride_tc_attention", "stride_tc_compact",
                 "stride_tc_split_count"):
        getattr(lib, name).restype = C.c_int
    lib.stride_tc_split_count.argtypes = [C.c_int32, C.c_int32]
    for name, (ptype, with_j) in EXACT_ENTRIES.items():
        fn = getattr(lib, name)
        fn.argtypes = [C.POINTER(ptype), C.c_int32, vp] if with_j else [C.POINTER(ptype), vp]
        fn.restype = C.c_int
    lib.stride_tc_set_stream_config.argtypes = [C.c_int32]
    lib.stride_tc_set_stream_config.restype = C.c_int
    lib.stride_tc_stream_config_count.argtypes = []
    lib.stride_tc_stream_config_count.restype = C.c_int
    lib.stride_tc_pipe_config_count.argtypes = []
    lib.stride_tc_pipe_config_count.restype = C.c_int
    lib.stride_tc_dec_config_count.argtypes = []
    lib.stride_tc_dec_config_count.restype = C.c_int
    lib.stride_tc_stream_config.argtypes = [C.c_int32, C.POINTER(C.c_int32)]
    lib.stride_tc_stream_config.restype = C.c_int
    lib.stride_tc_last_stream_config.argtypes = []
    lib.stride_tc_last_stream_config.restype = C.c_int
    lib.stride_tc_last_error.restype = C.c_char_p
    lib.stride_tc_last_error.argtypes = []
    lib.stride_tc_version.restype = C.c_char_p
    lib.stride_tc_version.argtypes = []
    check_layout()
    _lib = lib
    return lib


def check(rc: int) -> None:
    if rc != 0:
        msg = load().stride_tc_last_error().decode()
        raise StrideTcError(f"stride_tc error {rc:#x}: {msg}")


def split_count(n: int, k: int) -> int:
    s = load().stride_tc_split_count(n, k)
    if s < 0:
        check(s)
    return s


def pipe_config_count() -> int:
    """Number of LDS-pipelined kernel configurations (forced as -3 - i)."""
    return load().stride_tc_pipe_config_count()


DEC_CONFIG_BASE = 1000


def dec_config_count() -> int:
    """Configurations of the register-streamed weight / LDS-ring activation
    kernel, selected with set_stream_config(DEC_CONFIG_BASE + i)."""
    return load().stride_tc_dec_config_count()


def stream_configs():
    """[(R, LT, WS, WR, U, flags)] of the decode-regime kernel configurations
    (flags bit 0: x staged in LDS, bit 1: one split per workgroup)."""
    lib = load()
    out = []
    for i in range(lib.stride_tc_stream_config_count()):
        buf = (C.c_int32 * 6)()
        check(lib.stride_tc_stream_config(i, buf))
        out.append(tuple(buf))
    return out


def set_stream_config(index: int) -> None:
    """Force a decode-regime configuration (-1 = automatic); results never change."""
    check(load().stride_tc_set_stream_config(index))


def last_stream_config() -> int:
    """Configuration index the last launch used (-2 = prefill kernel)."""
    return load().stride_tc_last_stream_config()
