"""CPU oracle pinning (no GPU).

The oracle (oracle/exact.cpp) restates the reference's CPU exact path. It is pinned
three ways: bit-exact against the golden fixtures written from the reference's own
kernels.cu (tests/golden/make_golden.py), bit-exact against that compiled
reference directly where oracle/_ref exists, and against closed forms chosen so
that a dropped term, a wrong sign, a wrong index or a transposed operand fails.
"""
import hashlib
import json
import math
import os

import numpy as np
import pytest

from oracle.oracle import Ref, ref_available, rope_table
from stride_amd import synth
from stride_amd.synth import Ids

GOLD = os.path.join(os.path.dirname(__file__), "golden")


def _sha(*arrays):
    h = hashlib.sha256()
    for a in arrays:
        h.update(np.ascontiguousarray(a).tobytes())
    return h.hexdigest()


def _bits(a):
    return np.ascontiguousarray(a, dtype=np.float32).view(np.uint32)


@pytest.fixture(scope="module")
def golden():
    meta = json.load(open(os.path.join(GOLD, "exact_path.json")))
    arr = np.load(os.path.join(GOLD, "exact_path.npz"))
    return meta, arr


def _gemm_inputs(c):
    w = synth.bf16_normal(c["seed"], Ids.WO, c["n"], c["k"], 0.02)
    if c["x_bf16"]:
        x = synth.bf16_to_f32(synth.bf16_normal(c["seed"], Ids.X, c["m"], c["k"], 1.0))
    else:
        x = synth.f32_normal(c["seed"], Ids.X, c["m"], c["k"], 1.0)
    return w, x


def test_golden_gemm(golden, exact):
    meta, arr = golden
    names = [n for n, c in meta.items() if c["kind"] == "gemm"]
    assert "c1_f32x" in names and "c1_bf16x" in names
    for name in names:
        c = meta[name]
        w, x = _gemm_inputs(c)
        assert _sha(w, x) == c["input_sha"], f"{name}: synthetic generator changed"
        y = exact.gemm(w, x)
        assert np.array_equal(_bits(y), _bits(arr[f"{name}.y"])), name


def test_golden_residual(golden, exact):
    meta, arr = golden
    c = meta["residual"]
    w, x = _gemm_inputs(c)
    h = synth.f32_normal(c["seed"], Ids.H, c["m"], c["n"], 1.0)
    assert _sha(w, x, h) == c["input_sha"]
    assert np.array_equal(_bits(exact.gemm_residual(w, x, h)), _bits(arr["residual.y"]))


def test_golden_mlp13(golden, exact):
    meta, arr = golden
    c = meta["mlp13"]
    w1 = synth.bf16_normal(c["seed"], Ids.W1, c["n"], c["k"], 0.02)
    w3 = synth.bf16_normal(c["seed"], Ids.W3, c["n"], c["k"], 0.02)
    x = synth.bf16_to_f32(synth.bf16_normal(c["seed"], Ids.X, c["m"], c["k"], c["x_std"]))
    assert _sha(w1, w3, x) == c["input_sha"]
    assert np.array_equal(_bits(exact.mlp13(w1, w3, x)), _bits(arr["mlp13.y"]))


def test_golden_lm_greedy(golden, exact):
    meta, arr = golden
    c = meta["lm_greedy"]
    w = synth.bf16_normal(c["seed"], Ids.LM, c["n"], c["k"], 0.02)
    w[19] = w[7]
    x = synth.bf16_to_f32(synth.bf16_normal(c["seed"], Ids.X, c["m"], c["k"], 1.0))
    x[2] = synth.bf16_to_f32(w[7]) * 50.0
    assert _sha(w, x) == c["input_sha"]
    bv, bi = exact.lm_greedy(w, c["vocab"], x)
    assert np.array_equal(bi, arr["lm_greedy.best_index"])
    assert np.array_equal(_bits(bv), _bits(arr["lm_greedy.best_value"]))
    assert bi[2] == 7  # planted tie between rows 7 and 19 resolves to the smaller index


@pytest.mark.parametrize("D", [16, 64])
def test_golden_qkv(golden, exact, D):
    meta, arr = golden
    name = f"qkv_d{D}"
    c = meta[name]
    k = c["k"]
    wq = synth.bf16_normal(c["seed"], Ids.WQ, c["nq"], k, 0.02)
    wk = synth.bf16_normal(c["seed"], Ids.WK, c["nkv"], k, 0.02)
    wv = synth.bf16_normal(c["seed"], Ids.WV, c["nkv"], k, 0.02)
    x = synth.bf16_to_f32(synth.bf16_normal(c["seed"], Ids.X, c["m"], k, 1.0))
    assert _sha(wq, wk, wv, x) == c["input_sha"]
    q, ko, vo = exact.qkv(wq, wk, wv, x, D, rope_table(D, 300), arr[f"{name}.row_pos"])
    for got, key in ((q, "q"), (ko, "k_out"), (vo, "v_out")):
        assert np.array_equal(_bits(got), _bits(arr[f"{name}.{key}"])), key


def test_golden_det_exp(golden, exact):
    _, arr = golden
    xs = arr["det_exp.x"]
    got_e = np.float32([exact.det_exp(float(v)) for v in xs])
    got_s = np.float32([exact.det_silu(float(v)) for v in xs])
    assert np.array_equal(_bits(got_e), _bits(arr["det_exp.exp"]))
    assert np.array_equal(_bits(got_s), _bits(arr["det_exp.silu"]))


@pytest.mark.skipif(not ref_available(), reason="oracle/_ref not built (reference tree absent)")
@pytest.mark.parametrize("m,n,k", [(1, 32, 64), (2, 16, 2048), (9, 48, 768), (33, 16, 256)])
def test_restatement_matches_reference_build(exact, m, n, k):
    ref = Ref()
    w = synth.bf16_normal(11, Ids.W2, n, k, 0.05)
    x = synth.f32_normal(11, Ids.X, m, k, 2.0)
    h = synth.f32_normal(11, Ids.H, m, n, 1.0)
    assert np.array_equal(_bits(exact.gemm(w, x)), _bits(ref.gemm(w, x)))
    assert np.array_equal(_bits(exact.gemm_residual(w, x, h)), _bits(ref.gemm_residual(w, x, h)))
    w3 = synth.bf16_normal(12, Ids.W3, n, k, 0.05)
    assert np.array_equal(_bits(exact.mlp13(w, w3, x)), _bits(ref.mlp13(w, w3, x)))


# ---- closed forms -----------------------------------------------------------

def test_one_hot_extracts_column(exact):
    n, k = 16, 512
    w = synth.bf16_normal(3, Ids.WO, n, k, 0.02)
    x = np.zeros((3, k), np.float32)
    cols = [0, 255, 511]
    for j, c in enumerate(cols):
        x[j, c] = 1.0
    y = exact.gemm(w, x)
    for j, c in enumerate(cols):
        assert np.array_equal(y[j], synth.bf16_to_f32(w[:, c])), "wrong column or transposed operand"


def test_zero_weights_leave_residual(exact):
    n, k = 32, 256
    h = synth.f32_normal(4, Ids.H, 3, n)
    out = exact.gemm_residual(np.zeros((n, k), np.uint16), synth.f32_normal(4, Ids.X, 3, k), h)
    assert np.array_equal(_bits(out), _bits(h))


def test_dot_matches_float64_and_sign(exact):
    n, k = 24, 2048
    w = synth.bf16_normal(5, Ids.WO, n, k, 0.02)
    x = synth.f32_normal(5, Ids.X, 4, k)
    y = exact.gemm(w, x).astype(np.float64)
    wf = synth.bf16_to_f32(w).astype(np.float64)
    y64 = x.astype(np.float64) @ wf.T
    bound = (np.abs(x).astype(np.float64) @ np.abs(wf).T) * (k * 2.0 ** -24)
    assert np.all(np.abs(y - y64) <= bound)
    # a single dropped product would exceed 1e-4 here; the bound above is ~1e-5
    assert np.max(np.abs(y - y64)) < 5e-5
    assert np.array_equal(_bits(exact.gemm(w, -x)), _bits(-exact.gemm(w, x)))


def test_det_exp_accuracy(exact):
    for v in np.linspace(-86.5, 87.5, 3001):
        e = exact.det_exp(float(np.float32(v)))
        t = math.exp(float(np.float32(v)))
        assert abs(e - t) <= 4 * np.spacing(np.float32(t)), v
    assert exact.det_exp(-88.0) == 0.0 and math.isinf(exact.det_exp(89.0))
    for v in (-20.0, -1.0, 0.0, 0.5, 3.0, 20.0):
        assert abs(exact.det_silu(v) - v / (1 + math.exp(-v))) <= 1e-6 * max(1.0, abs(v))


def test_bf16_round_known_answers(exact):
    cases = {1.0: 0x3F80, 1.0 + 2 ** -8: 0x3F80, 1.0 + 3 * 2 ** -8: 0x3F82, -2.0: 0xC000, 1.0 + 2 ** -7: 0x3F81,
             1.0 + 2 ** -8 + 2 ** -20: 0x3F81, 0.0: 0x0000}
    for v, want in cases.items():
        assert exact.bf16_rne(v) == want, v
        assert int(synth.bf16_bits(np.float32([v]))[0]) == want, v


def test_lm_greedy_ties_and_padding(exact):
    n, k = 48, 64
    w = np.zeros((n, k), np.uint16)
    x = np.ones((2, k), np.float32)
    w[5, 0] = w[30, 0] = synth.bf16_bits(np.float32([1.0]))[0]  # tie between rows 5 and 30
    w[47, 0] = synth.bf16_bits(np.float32([9.0]))[0]  # beyond vocab: must be ignored
    bv, bi = exact.lm_greedy(w, 40, x)
    assert list(bi) == [5, 5] and list(bv) == [1.0, 1.0]


def test_qkv_rope_closed_form(exact):
    D, nq, nkv, k, m = 16, 32, 16, 128, 3
    wq = synth.bf16_normal(6, Ids.WQ, nq, k, 0.05)
    wk = synth.bf16_normal(6, Ids.WK, nkv, k, 0.05)
    wv = synth.bf16_normal(6, Ids.WV, nkv, k, 0.05)
    x = synth.f32_normal(6, Ids.X, m, k)
    rope = rope_table(D, 64)
    pos = np.array([0, 1, 63], np.int32)
    q, ko, vo = exact.qkv(wq, wk, wv, x, D, rope, pos)
    yq, yk = exact.gemm(wq, x), exact.gemm(wk, x)
    # pos 0: cos 1, sin 0 -> no rotation, exactly the plain projection
    assert np.array_equal(_bits(q[0]), _bits(yq[0]))
    assert np.array_equal(_bits(vo), _bits(exact.gemm(wv, x)))
    half = D // 2
    for j in (1, 2):
        for base, y, out in ((0, yq, q), (16, yq, q), (0, yk, ko)):
            a = y[j, base:base + half].astype(np.float64)
            b = y[j, base + half:base + D].astype(np.float64)
            co, si = rope[pos[j], :, 0].astype(np.float64), rope[pos[j], :, 1].astype(np.float64)
            np.testing.assert_allclose(out[j, base:base + half], a * co - b * si, atol=1e-6)
            np.testing.assert_allclose(out[j, base + half:base + D], b * co + a * si, atol=1e-6)
