"""TEST INFRASTRUCTURE ONLY: ctypes front-end for the CPU oracle.

``Exact`` wraps liboracle.so (this repository's restatement of the reference's CPU
exact path, oracle/exact.cpp). ``Ref`` wraps oracle/_ref/libstride_ref.so, the
reference's own src/kernels.cu compiled as C++ (present only where it was built).
Both expose the same functions on row-major numpy operands:

  gemm(w, x)                      y[m][n] = W[n].x[m]          (k_lm_full)
  gemm_residual(w, x, h)          h + W.x                      (k_gemm_residual)
  mlp13(w1, w3, x)                det_silu(W1.x) * (W3.x)      (k_mlp13)
  lm_greedy(w, vocab, x)          (best value, best index)     (k_lm_greedy)
  qkv(wq, wk, wv, x, D, rope, pos) q, k, v with RoPE           (k_qkv)

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg import this.
"""
from __future__ import annotations

import ctypes as C
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "liboracle.so")
REF_PATH = os.path.join(HERE, "_ref", "libstride_ref.so")

_u16p = np.ctypeslib.ndpointer(np.uint16, flags="C_CONTIGUOUS")
_f32p = np.ctypeslib.ndpointer(np.float32, flags="C_CONTIGUOUS")
_i32p = np.ctypeslib.ndpointer(np.int32, flags="C_CONTIGUOUS")
_f32p_opt = C.c_void_p


def build() -> None:
    """Compile liboracle.so (and _ref when the reference tree is present)."""
    import subprocess

    subprocess.run(["make", "-s", "-B", "-C", HERE], check=True)


def _u16(a):
    return np.ascontiguousarray(a, dtype=np.uint16)


def _f32(a):
    return np.ascontiguousarray(a, dtype=np.float32)


class _Base:
    prefix = ""
    has_threads = False

    def __init__(self, path: str):
        if not os.path.exists(path):
            raise FileNotFoundError(f"oracle library missing: {path} (run make -C oracle)")
        self.lib = C.CDLL(path)
        p = self.prefix
        T = [C.c_int] if self.has_threads else []
        getattr(self.lib, p + "det_exp").restype = C.c_float
        getattr(self.lib, p + "det_exp").argtypes = [C.c_float]
        getattr(self.lib, p + "det_silu").restype = C.c_float
        getattr(self.lib, p + "det_silu").argtypes = [C.c_float]
        f = getattr(self.lib, p + "gemm")
        f.argtypes = [_u16p, C.c_int, C.c_int, _f32p, C.c_int, _f32p] + T
        f = getattr(self.lib, p + "gemm_residual")
        f.argtypes = [_u16p, C.c_int, C.c_int, _f32p, C.c_int, _f32p] + T
        f = getattr(self.lib, p + "lm_greedy")
        f.argtypes = [_u16p, C.c_int, C.c_int, C.c_int, _f32p, C.c_int, _f32p, _i32p] + T
        f = getattr(self.lib, p + "qkv")
        f.argtypes = [_u16p, _u16p, _u16p, C.c_int, C.c_int, C.c_int, _f32p, C.c_int, C.c_int, _f32p, _i32p, _f32p,
                      _f32p, _f32p] + T
        self.threads = 0

    def _t(self):
        return (self.threads,) if self.has_threads else ()

    def _call(self, name, *args):
        rc = getattr(self.lib, self.prefix + name)(*args, *self._t())
        if rc != 0:
            raise ValueError(f"{self.prefix}{name} rejected its arguments (rc={rc})")

    def det_exp(self, v: float) -> float:
        return getattr(self.lib, self.prefix + "det_exp")(v)

    def det_silu(self, v: float) -> float:
        return getattr(self.lib, self.prefix + "det_silu")(v)

    def gemm(self, w, x):
        w, x = _u16(w), _f32(x)
        n, k = w.shape
        m = x.shape[0]
        y = np.zeros((m, n), np.float32)
        self._call("gemm", w, n, k, x, m, y)
        return y

    def gemm_residual(self, w, x, h):
        w, x = _u16(w), _f32(x)
        h = np.array(h, dtype=np.float32, copy=True, order="C")
        n, k = w.shape
        self._call("gemm_residual", w, n, k, x, x.shape[0], h)
        return h

    def lm_greedy(self, w, vocab, x):
        w, x = _u16(w), _f32(x)
        n, k = w.shape
        m = x.shape[0]
        bv = np.zeros(m, np.float32)
        bi = np.zeros(m, np.int32)
        self._call("lm_greedy", w, n, vocab, k, x, m, bv, bi)
        return bv, bi

    def qkv(self, wq, wk, wv, x, head_dim, rope, row_pos):
        wq, wk, wv, x = _u16(wq), _u16(wk), _u16(wv), _f32(x)
        nq, k = wq.shape
        nkv = wk.shape[0]
        m = x.shape[0]
        q = np.zeros((m, nq), np.float32)
        ko = np.zeros((m, nkv), np.float32)
        vo = np.zeros((m, nkv), np.float32)
        self._call("qkv", wq, wk, wv, nq, nkv, k, x, m, head_dim, _f32(rope),
                   np.ascontiguousarray(row_pos, dtype=np.int32), q, ko, vo)
        return q, ko, vo


class Exact(_Base):
    """This repository's restatement (oracle/exact.cpp)."""

    prefix = "oracle_"
    has_threads = True

    def __init__(self, path: str = LIB_PATH, threads: int = 0):
        super().__init__(path)
        self.threads = threads
        f = self.lib.oracle_mlp13
        f.argtypes = [_u16p, _u16p, C.c_int, C.c_int, _f32p, C.c_int, _f32p, _f32p_opt, _f32p_opt, C.c_int]
        self.lib.oracle_bf16_rne.restype = C.c_uint16
        self.lib.oracle_bf16_rne.argtypes = [C.c_float]

    def mlp13(self, w1, w3, x, want_preact: bool = False):
        w1, w3, x = _u16(w1), _u16(w3), _f32(x)
        n, k = w1.shape
        m = x.shape[0]
        z = np.zeros((m, n), np.float32)
        a = np.zeros((m, n), np.float32) if want_preact else None
        b = np.zeros((m, n), np.float32) if want_preact else None
        rc = self.lib.oracle_mlp13(w1, w3, n, k, x, m, z,
                                   a.ctypes.data if a is not None else None,
                                   b.ctypes.data if b is not None else None, self.threads)
        if rc != 0:
            raise ValueError("oracle_mlp13 rejected its arguments")
        return (z, a, b) if want_preact else z

    def bf16_rne(self, v: float) -> int:
        return self.lib.oracle_bf16_rne(v)

    def tc_norm(self, h, weight, eps: float):
        """Tensor-core-path RMSNorm of rows h [m][dim] -> bf16 bits [m][dim]."""
        h, weight = _f32(h), _f32(weight)
        m, dim = h.shape
        x = np.zeros((m, dim), np.uint16)
        f = self.lib.oracle_tc_norm
        f.argtypes = [_f32p, C.c_int, C.c_int, _f32p, C.c_float, _u16p]
        if f(h, m, dim, weight, eps, x) != 0:
            raise ValueError("oracle_tc_norm rejected its arguments")
        return x

    def rope_table(self, cfg, max_positions: int):
        """RoPE table [max_positions][head_dim/2][2] of a stride_amd.weights.ModelConfig."""
        half = cfg.head_dim // 2
        out = np.zeros((max_positions, half, 2), np.float32)
        f = self.lib.oracle_rope_table
        f.argtypes = [C.c_int, C.c_double, C.c_int, C.c_double, C.c_double, C.c_double, C.c_double, C.c_int, _f32p]
        if f(cfg.head_dim, cfg.rope_theta, int(cfg.rope_llama3), cfg.rope_factor, cfg.rope_low, cfg.rope_high,
             cfg.rope_orig_ctx, max_positions, out) != 0:
            raise ValueError("oracle_rope_table rejected its arguments")
        return out

    def tc_attention(self, q, k, v, row_slot, row_pos, scale: float):
        """Tensor-core-path attention. q [m][n_kv*4][hd] fp32; k, v [slots][n_kv][cap][hd]
        bf16 bits -> out bf16 bits [m][n_kv*4*hd]."""
        q, k, v = _f32(q), _u16(k), _u16(v)
        m, heads, hd = q.shape
        n_kv, cap = k.shape[1], k.shape[2]
        out = np.zeros((m, heads * hd), np.uint16)
        f = self.lib.oracle_tc_attention
        f.argtypes = [_f32p, _u16p, _u16p, C.c_int, _i32p, _i32p, C.c_int, C.c_int, C.c_int, C.c_float, _u16p]
        if f(q, k, v, cap, np.ascontiguousarray(row_slot, dtype=np.int32), np.ascontiguousarray(row_pos, dtype=np.int32),
             m, n_kv, hd, scale, out) != 0:
            raise ValueError("oracle_tc_attention rejected its arguments")
        return out


class Ref(_Base):
    """The reference's own exact path (oracle/_ref/libstride_ref.so)."""

    prefix = "ref_"
    has_threads = False

    def __init__(self, path: str = REF_PATH):
        super().__init__(path)
        self.lib.ref_mlp13.argtypes = [_u16p, _u16p, C.c_int, C.c_int, _f32p, C.c_int, _f32p]

    def mlp13(self, w1, w3, x):
        w1, w3, x = _u16(w1), _u16(w3), _f32(x)
        n, k = w1.shape
        m = x.shape[0]
        z = np.zeros((m, n), np.float32)
        self._call("mlp13", w1, w3, n, k, x, m, z)
        return z

    def embed(self, emb, tokens):
        """Exact-path embedding of bf16 rows emb [vocab][dim] -> fp32 [m][dim]."""
        emb = _u16(emb)
        vocab, dim = emb.shape
        tokens = np.ascontiguousarray(tokens, dtype=np.int32)
        h = np.zeros((tokens.size, dim), np.float32)
        f = self.lib.ref_embed
        f.argtypes = [_u16p, C.c_int, C.c_int, _i32p, C.c_int, _f32p]
        self._call("embed", emb, vocab, dim, tokens, tokens.size, h)
        return h

    def norm(self, h, weight, eps: float):
        """Exact-path RMSNorm of rows h [m][dim] -> fp32 [m][dim]."""
        h, weight = _f32(h), _f32(weight)
        m, dim = h.shape
        out = np.zeros((m, dim), np.float32)
        f = self.lib.ref_norm
        f.argtypes = [_f32p, C.c_int, C.c_int, _f32p, C.c_float, _f32p]
        self._call("norm", h, m, dim, weight, eps, out)
        return out

    def attention(self, q, k, v, row_slot, row_pos, scale: float):
        """Exact-path attention over fp32 KV holding the widened bf16 k, v
        [slots][n_kv][cap][hd] -> fp32 [m][n_kv*4*hd]."""
        q, k, v = _f32(q), _u16(k), _u16(v)
        m, heads, hd = q.shape
        slots, n_kv, cap = k.shape[0], k.shape[1], k.shape[2]
        out = np.zeros((m, heads * hd), np.float32)
        f = self.lib.ref_attention
        f.argtypes = [_f32p, _u16p, _u16p, C.c_int, C.c_int, _i32p, _i32p, C.c_int, C.c_int, C.c_int, C.c_float, _f32p]
        self._call("attention", q, k, v, slots, cap, np.ascontiguousarray(row_slot, dtype=np.int32),
                   np.ascontiguousarray(row_pos, dtype=np.int32), m, n_kv, hd, scale, out)
        return out


def ref_available() -> bool:
    return os.path.exists(REF_PATH)


def rope_table(head_dim: int, positions: int, theta: float = 500000.0) -> np.ndarray:
    """[pos][D/2][cos, sin] fp32 table with plain (un-scaled) RoPE frequencies.

    The reference builds the same shape of table (src/model.cpp:54-88); the GEMM
    only reads it, so any fixed table exercises the epilogue.
    """
    half = head_dim // 2
    inv = 1.0 / (theta ** (np.arange(half, dtype=np.float64) * 2.0 / head_dim))
    ang = np.arange(positions, dtype=np.float64)[:, None] * inv[None, :]
    t = np.stack([np.cos(ang), np.sin(ang)], axis=-1).astype(np.float32)
    return np.ascontiguousarray(t)
