"""TEST INFRASTRUCTURE: a backend for stride_amd.exact_engine that runs the
reference's own exact-path operators on the CPU (src/kernels.cu and device.cu
compiled as C++ into oracle/_ref/libstride_ref.so, entry points ref_k_* in
oracle/ref_harness.cpp), on numpy buffers. Driving the engine's step through it
is the reference's Engine::step_exact on the CPU (src/engine.cpp:144-297)."""
import ctypes as C
import os

import numpy as np

from oracle import oracle as O
from stride_amd import _lib

_TAKES_J = {"embed": False, "norm": True, "qkv": True, "attention": False, "gemm_residual": True, "mlp13": True,
            "compact": False, "lm_greedy": True, "lm_full": True}


class CpuBackend:
    def __init__(self, threads: int = 16):
        # the reference's pool reads its size once, at its first use
        os.environ.setdefault("STRIDE_CPU_THREADS", str(threads))
        self.lib = C.CDLL(O.REF_PATH)
        for name, takes_j in _TAKES_J.items():
            fn = getattr(self.lib, "ref_k_" + name)
            fn.argtypes = [C.c_void_p, C.c_int] if takes_j else [C.c_void_p]
            fn.restype = None

    def zeros(self, count, dtype):
        return np.zeros(int(count), dtype)

    def array(self, a):
        return np.array(a, copy=True).reshape(-1)

    def ptr(self, buf):
        return buf.ctypes.data

    def put(self, buf, a):
        a = np.ascontiguousarray(a).reshape(-1)
        buf[: a.size] = a.view(buf.dtype) if a.dtype.itemsize == buf.dtype.itemsize else a

    def get(self, buf, count, dtype):
        return buf[:count].view(dtype).copy()

    def call(self, name, p, J=None):
        fn = getattr(self.lib, "ref_k_" + name)
        if _TAKES_J[name]:
            fn(C.addressof(p), J)
        else:
            fn(C.addressof(p))

    def sync(self):
        pass
