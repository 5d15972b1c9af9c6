"""Portable seeded synthetic inputs (weights, activations, residuals).

Every element is a pure function of (seed, tensor id, row, column): a splitmix64
finaliser over a counter gives two uniforms, Box-Muller in float64 gives a normal,
which is scaled, cast to fp32 and (for bf16 tensors) rounded to nearest-even bf16.
Row ``i`` of a tensor is therefore identical whatever number of rows is generated,
which is what the batch-invariance checks rely on: the M=1 run and the M=4096 run
see the same bits for their common rows. ``std::normal_distribution`` is not used
because its output is implementation-defined.
"""
from __future__ import annotations

import numpy as np

_GOLDEN = np.uint64(0x9E3779B97F4A7C15)
_M1 = np.uint64(0xBF58476D1CE4E5B9)
_M2 = np.uint64(0x94D049BB133111EB)


def _mix(z: np.ndarray) -> np.ndarray:
    z = (z ^ (z >> np.uint64(30))) * _M1
    z = (z ^ (z >> np.uint64(27))) * _M2
    return z ^ (z >> np.uint64(31))


def _uniform(bits: np.ndarray) -> np.ndarray:
    # 53 random bits -> (0, 1), never exactly 0 so log() is finite.
    return ((bits >> np.uint64(11)).astype(np.float64) + 0.5) * (1.0 / 9007199254740992.0)


def normal(seed: int, tensor: int, rows: int, cols: int, row0: int = 0) -> np.ndarray:
    """float64 N(0,1) array [rows, cols] for rows row0 .. row0+rows-1 of a tensor."""
    with np.errstate(over="ignore"):
        key = _mix(np.uint64(seed) * _GOLDEN ^ _mix(np.uint64(tensor) + np.uint64(0x632BE59BD9B4E019)))
        r = np.arange(row0, row0 + rows, dtype=np.uint64)[:, None]
        c = np.arange(cols, dtype=np.uint64)[None, :]
        ctr = r * np.uint64(cols) + c
        u1 = _uniform(_mix(key + (ctr * np.uint64(2)) * _GOLDEN))
        u2 = _uniform(_mix(key + (ctr * np.uint64(2) + np.uint64(1)) * _GOLDEN))
    return np.sqrt(-2.0 * np.log(u1)) * np.cos(2.0 * np.pi * u2)


def bf16_bits(f32: np.ndarray) -> np.ndarray:
    """Round-to-nearest-even fp32 -> bf16 bit patterns (uint16), on the bit pattern."""
    u = np.ascontiguousarray(f32, dtype=np.float32).view(np.uint32).astype(np.uint64)
    return ((u + np.uint64(0x7FFF) + ((u >> np.uint64(16)) & np.uint64(1))) >> np.uint64(16)).astype(np.uint16)


def bf16_to_f32(bits: np.ndarray) -> np.ndarray:
    """Exact widening of bf16 bit patterns to fp32."""
    return (np.asarray(bits, dtype=np.uint16).astype(np.uint32) << np.uint32(16)).view(np.float32)


def bf16_normal(seed: int, tensor: int, rows: int, cols: int, std: float = 1.0, row0: int = 0) -> np.ndarray:
    """bf16 bit patterns (uint16) of std * N(0,1)."""
    return bf16_bits((normal(seed, tensor, rows, cols, row0) * std).astype(np.float32))


def f32_normal(seed: int, tensor: int, rows: int, cols: int, std: float = 1.0, row0: int = 0) -> np.ndarray:
    return (normal(seed, tensor, rows, cols, row0) * std).astype(np.float32)


def permutation(seed: int, n: int) -> np.ndarray:
    """Seeded Fisher-Yates permutation of range(n) driven by the same counter hash."""
    perm = np.arange(n, dtype=np.int64)
    with np.errstate(over="ignore"):
        key = _mix(np.uint64(seed) ^ np.uint64(0xD1B54A32D192ED03))
        draws = _mix(key + np.arange(n, dtype=np.uint64) * _GOLDEN)
    for i in range(n - 1, 0, -1):
        j = int(draws[i] % np.uint64(i + 1))
        perm[i], perm[j] = perm[j], perm[i]
    return perm


# Tensor ids used by tests and the benchmark, so every consumer draws the same data.
class Ids:
    X = 1
    H = 2
    WQ, WK, WV, WO, W1, W3, W2 = 10, 11, 12, 13, 14, 15, 16
    LM = 20
    LAYER_STRIDE = 100  # layer l uses id + l * LAYER_STRIDE
