"""Writes the golden fixtures under tests/golden/ from the reference's own CPU exact
path (oracle/_ref/libstride_ref.so: the reference's src/kernels.cu compiled as C++
by oracle/Makefile). Run in the container that has /root/reference:

    make -C oracle && python tests/golden/make_golden.py

Inputs come from stride_amd.synth (seeded, portable); each fixture stores the seed
and shape, a SHA-256 of the generated input bytes (so a change in the generator is
caught) and the reference outputs as raw fp32/int32 bit patterns.
"""
from __future__ import annotations

import hashlib
import json
import os
import sys

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, ROOT)

from oracle.oracle import Ref, rope_table  # noqa: E402
from stride_amd import synth  # noqa: E402
from stride_amd.synth import Ids  # noqa: E402

OUT = os.path.dirname(os.path.abspath(__file__))


def sha(*arrays) -> str:
    h = hashlib.sha256()
    for a in arrays:
        h.update(np.ascontiguousarray(a).tobytes())
    return h.hexdigest()


def inputs_gemm(seed, m, n, k, x_bf16):
    w = synth.bf16_normal(seed, Ids.WO, n, k, 0.02)
    if x_bf16:
        x = synth.bf16_to_f32(synth.bf16_normal(seed, Ids.X, m, k, 1.0))
    else:
        x = synth.f32_normal(seed, Ids.X, m, k, 1.0)
    return w, x


def main() -> None:
    ref = Ref()
    cases = {}

    # Config 1: y = x W^T, x fp32 [1, 2048], W bf16 [2048, 2048], seed 0.
    for tag, xb in (("c1_f32x", False), ("c1_bf16x", True)):
        w, x = inputs_gemm(0, 1, 2048, 2048, xb)
        y = ref.gemm(w, x)
        cases[tag] = dict(kind="gemm", seed=0, m=1, n=2048, k=2048, x_bf16=xb, input_sha=sha(w, x), y=y)

    # Small GEMM shapes covering the J=1 and J=4 lane layouts and ragged M.
    for (m, n, k) in ((1, 64, 256), (3, 48, 512), (17, 32, 1024)):
        w, x = inputs_gemm(1, m, n, k, True)
        cases[f"gemm_{m}x{n}x{k}"] = dict(kind="gemm", seed=1, m=m, n=n, k=k, x_bf16=True, input_sha=sha(w, x),
                                         y=ref.gemm(w, x))

    # Residual.
    m, n, k = 5, 64, 512
    w, x = inputs_gemm(2, m, n, k, True)
    h = synth.f32_normal(2, Ids.H, m, n, 1.0)
    cases["residual"] = dict(kind="residual", seed=2, m=m, n=n, k=k, x_bf16=True, input_sha=sha(w, x, h),
                             y=ref.gemm_residual(w, x, h))

    # Gate/up with SiLU.
    m, n, k = 6, 48, 512
    w1 = synth.bf16_normal(3, Ids.W1, n, k, 0.02)
    w3 = synth.bf16_normal(3, Ids.W3, n, k, 0.02)
    x = synth.bf16_to_f32(synth.bf16_normal(3, Ids.X, m, k, 4.0))
    cases["mlp13"] = dict(kind="mlp13", seed=3, m=m, n=n, k=k, x_std=4.0, input_sha=sha(w1, w3, x),
                          y=ref.mlp13(w1, w3, x))

    # LM greedy with a padded vocabulary and a planted tie (rows 7 and 19 equal).
    m, n, k, vocab = 4, 64, 256, 61
    w = synth.bf16_normal(4, Ids.LM, n, k, 0.02)
    w[19] = w[7]
    x = synth.bf16_to_f32(synth.bf16_normal(4, Ids.X, m, k, 1.0))
    x[2] = synth.bf16_to_f32(w[7]) * 50.0  # row 2 prefers rows 7 / 19 (tie -> 7)
    bv, bi = ref.lm_greedy(w, vocab, x)
    cases["lm_greedy"] = dict(kind="lm_greedy", seed=4, m=m, n=n, k=k, vocab=vocab, input_sha=sha(w, x),
                              best_value=bv, best_index=bi)

    # QKV with RoPE, head_dim 16 (toy) and 64 (Llama-3.2-1B).
    for D, nq, nkv, m in ((16, 64, 32, 6), (64, 256, 128, 3)):
        k = 256
        wq = synth.bf16_normal(5, Ids.WQ, nq, k, 0.02)
        wk = synth.bf16_normal(5, Ids.WK, nkv, k, 0.02)
        wv = synth.bf16_normal(5, Ids.WV, nkv, k, 0.02)
        x = synth.bf16_to_f32(synth.bf16_normal(5, Ids.X, m, k, 1.0))
        rope = rope_table(D, 300)
        pos = (np.arange(m, dtype=np.int32) * 37 + 5) % 300
        q, ko, vo = ref.qkv(wq, wk, wv, x, D, rope, pos)
        cases[f"qkv_d{D}"] = dict(kind="qkv", seed=5, m=m, nq=nq, nkv=nkv, k=k, head_dim=D, input_sha=sha(wq, wk, wv, x),
                                  row_pos=pos, q=q, k_out=ko, v_out=vo)

    # det_exp / det_silu sweep.
    xs = np.concatenate([np.linspace(-90, 90, 4001, dtype=np.float32), np.float32([-87.0, 88.0, 0.0, -0.0, 1e-30])])
    cases["det_exp"] = dict(kind="det_exp", x=xs, exp=np.float32([ref.det_exp(float(v)) for v in xs]),
                            silu=np.float32([ref.det_silu(float(v)) for v in xs]))

    arrays, meta = {}, {}
    for name, c in cases.items():
        entry = {}
        for key, val in c.items():
            if isinstance(val, np.ndarray):
                arrays[f"{name}.{key}"] = val
            else:
                entry[key] = val
        meta[name] = entry
    np.savez_compressed(os.path.join(OUT, "exact_path.npz"), **arrays)
    with open(os.path.join(OUT, "exact_path.json"), "w") as f:
        json.dump(meta, f, indent=1, sort_keys=True)
    print("wrote", len(cases), "cases")


if __name__ == "__main__":
    main()
