"""ctypes binding of tests/kat/libmfma_kat.so (built by build_kat.py; test
infrastructure): the MFMA known-answer kernels of the GPU tests."""
from __future__ import annotations

import ctypes as C
import os

PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "libmfma_kat.so")
_lib = None


def load():
    global _lib
    if _lib is None:
        if not os.path.exists(PATH):
            raise ImportError(f"{PATH} not built (python tests/kat/build_kat.py)")
        lib = C.CDLL(PATH)
        vp = C.c_void_p
        lib.mfma_kat_tiles.argtypes = [vp, vp, vp, vp, C.c_int32, vp]
        lib.mfma_kat_tiles.restype = C.c_int
        lib.mfma_kat_equiv.argtypes = [vp, vp, vp, vp, vp, C.c_int32, C.c_int32, vp]
        lib.mfma_kat_equiv.restype = C.c_int
        _lib = lib
    return _lib


def mfma_tiles(a, b, c, out, stream: int) -> None:
    rc = load().mfma_kat_tiles(a.data_ptr(), b.data_ptr(), c.data_ptr(), out.data_ptr(), a.shape[0], stream)
    if rc:
        raise RuntimeError(f"mfma_kat_tiles failed ({rc})")


def mfma_equiv(a, b, c0, o16, o32, chunks: int, stream: int) -> None:
    rc = load().mfma_kat_equiv(a.data_ptr(), b.data_ptr(), c0.data_ptr(), o16.data_ptr(), o32.data_ptr(),
                               c0.shape[0], chunks, stream)
    if rc:
        raise RuntimeError(f"mfma_kat_equiv failed ({rc})")
