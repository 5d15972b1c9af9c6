"""ctypes binding of libstride_probe.so (include/stride_probe.h): the MFMA
position-invariance probe and the HBM read-throughput probe."""
from __future__ import annotations

import ctypes as C
import os

HERE = os.path.dirname(os.path.abspath(__file__))
PATH = os.path.join(HERE, "libstride_probe.so")
_lib = None


def load():
    global _lib
    if _lib is None:
        if not os.path.exists(PATH):
            raise ImportError(f"{PATH} not built (python -m stride_amd.build)")
        lib = C.CDLL(PATH)
        vp = C.c_void_p
        lib.stride_probe_mfma_tiles.argtypes = [vp, vp, vp, vp, C.c_int32, vp]
        lib.stride_probe_mfma_tiles.restype = C.c_int
        lib.stride_probe_read.argtypes = [vp, C.c_int64, vp, C.c_int32, C.c_int32, vp]
        lib.stride_probe_read.restype = C.c_int
        lib.stride_probe_mfma_rate.argtypes = [vp, C.c_int32, C.c_int32, vp]
        lib.stride_probe_mfma_rate.restype = C.c_int
        lib.stride_probe_mfma_rate_variant.argtypes = [vp, C.c_int32, C.c_int32, C.c_int32, vp]
        lib.stride_probe_mfma_rate_variant.restype = C.c_int
        lib.stride_probe_mfma_equiv.argtypes = [vp, vp, vp, vp, vp, C.c_int32, C.c_int32, vp]
        lib.stride_probe_mfma_equiv.restype = C.c_int
        lib.stride_probe_strip_read.argtypes = [vp, C.c_int64, C.c_int64, C.c_int32, C.c_int32, C.c_int32, vp, vp]
        lib.stride_probe_strip_read.restype = C.c_int
        _lib = lib
    return _lib


def mfma_tiles(a, b, c, out, stream: int) -> None:
    rc = load().stride_probe_mfma_tiles(a.data_ptr(), b.data_ptr(), c.data_ptr(), out.data_ptr(), a.shape[0], stream)
    if rc:
        raise RuntimeError(f"stride_probe_mfma_tiles failed ({rc})")


def read(buf, out, blocks: int, unroll: int, stream: int) -> None:
    rc = load().stride_probe_read(buf.data_ptr(), buf.numel() * buf.element_size(), out.data_ptr(), blocks, unroll,
                                  stream)
    if rc:
        raise RuntimeError(f"stride_probe_read failed ({rc})")


def strip_read(buf, strip: int, out, blocks: int, unroll: int, rotate: int, stream: int) -> None:
    rc = load().stride_probe_strip_read(buf.data_ptr(), buf.numel() * buf.element_size(), strip, blocks, unroll,
                                        rotate, out.data_ptr(), stream)
    if rc:
        raise RuntimeError(f"stride_probe_strip_read failed ({rc})")


def mfma_rate(out, blocks: int, iters: int, stream: int) -> None:
    rc = load().stride_probe_mfma_rate(out.data_ptr(), blocks, iters, stream)
    if rc:
        raise RuntimeError(f"stride_probe_mfma_rate failed ({rc})")


def mfma_rate_variant(out, blocks: int, iters: int, variant: int, stream: int) -> None:
    rc = load().stride_probe_mfma_rate_variant(out.data_ptr(), blocks, iters, variant, stream)
    if rc:
        raise RuntimeError(f"stride_probe_mfma_rate_variant failed ({rc})")


def mfma_equiv(a, b, c0, o16, o32, chunks: int, stream: int) -> None:
    rc = load().stride_probe_mfma_equiv(a.data_ptr(), b.data_ptr(), c0.data_ptr(), o16.data_ptr(), o32.data_ptr(),
                                        c0.shape[0], chunks, stream)
    if rc:
        raise RuntimeError(f"stride_probe_mfma_equiv failed ({rc})")
