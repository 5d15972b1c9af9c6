"""Pins of the oracle's restatements of the tensor-core path's non-GEMM operators
(oracle/exact.cpp: oracle_tc_norm, oracle_tc_attention) on the CPU.

* Attention: the reference's exact path (k_attention over fp32 KV holding the
  same bf16 values, src/kernels.cu:474-485) evaluates the same tree as the
  tensor-core path (src/kernel_common.h:84-309, identical templates), so after
  the tensor-core writer's bf16 rounding the two must agree bit for bit; and a
  float64 softmax attention bounds both.
* RMSNorm: the exact path groups 4 columns per partial chain, the tensor-core
  path 16 (src/kernels.cu:119-200 vs src/kernels_tc.cu:205-271), so their sums
  agree exactly when every partial is exact (small-integer inputs) and to within
  one bf16 step otherwise; a float64 RMSNorm bounds both.
* Embedding: an exact widening; the exact path's k_embed gives the same values.
"""
import numpy as np
import pytest

from oracle import oracle as O

ref_only = pytest.mark.skipif(not O.ref_available(), reason="oracle/_ref not built (reference tree absent)")


def bf16_bits(a):
    return (np.ascontiguousarray(a, np.float32).view(np.uint32) >> 16).astype(np.uint16)


def widen(b):
    return (b.astype(np.uint32) << 16).view(np.float32)


def rne(exact, a):
    return np.array([exact.bf16_rne(float(t)) for t in np.ravel(a)], np.uint16).reshape(np.shape(a))


def attention_case(seed, m, n_kv, hd, slots, cap):
    rng = np.random.default_rng(seed)
    q = rng.standard_normal((m, n_kv * 4, hd)).astype(np.float32)
    k = bf16_bits(rng.standard_normal((slots, n_kv, cap, hd)))
    v = bf16_bits(rng.standard_normal((slots, n_kv, cap, hd)))
    slot = rng.integers(0, slots, m).astype(np.int32)
    pos = rng.integers(0, cap, m).astype(np.int32)
    pos[: min(m, 6)] = np.array([0, 63, 64, 127, 128, cap - 1], np.int32)[: min(m, 6)]
    return q, k, v, slot, pos


@ref_only
@pytest.mark.parametrize("n_kv,hd", [(1, 32), (2, 64), (1, 128)])
def test_attention_restatement_matches_reference(exact, n_kv, hd):
    ref = O.Ref()
    q, k, v, slot, pos = attention_case(11 + hd, 9, n_kv, hd, 3, 200)
    scale = hd ** -0.5
    ours = exact.tc_attention(q, k, v, slot, pos, scale)
    theirs = ref.attention(q, k, v, slot, pos, scale)
    assert np.array_equal(ours, rne(exact, theirs))


def test_attention_closed_form(exact):
    q, k, v, slot, pos = attention_case(5, 7, 2, 64, 2, 300)
    scale = 64 ** -0.5
    ours = widen(exact.tc_attention(q, k, v, slot, pos, scale)).reshape(7, 8, 64)
    K, V = widen(k).astype(np.float64), widen(v).astype(np.float64)
    for j in range(7):
        for h in range(8):
            g = h // 4
            kk = K[slot[j], g, : pos[j] + 1]
            s = kk @ q[j, h].astype(np.float64) * scale
            w = np.exp(s - s.max())
            want = (w / w.sum()) @ V[slot[j], g, : pos[j] + 1]
            assert np.allclose(ours[j, h], want, rtol=2 ** -7, atol=2 ** -7 * np.abs(want).max())


def test_attention_single_position_returns_value(exact):
    """With one visible position the softmax weight is exactly 1: out = bf16(v)."""
    q, k, v, slot, pos = attention_case(3, 4, 1, 64, 2, 64)
    pos[:] = 0
    out = exact.tc_attention(q, k, v, slot, pos, 0.125).reshape(4, 4, 64)
    for j in range(4):
        for h in range(4):
            assert np.array_equal(out[j, h], v[slot[j], 0, 0])


@ref_only
def test_norm_matches_reference(exact):
    ref = O.Ref()
    rng = np.random.default_rng(2)
    w = rng.standard_normal(2048).astype(np.float32)
    hi = rng.integers(-4, 5, (9, 2048)).astype(np.float32)
    assert np.array_equal(exact.tc_norm(hi, w, 1e-5), rne(exact, ref.norm(hi, w, 1e-5)))
    h = rng.standard_normal((9, 2048)).astype(np.float32)
    ours = widen(exact.tc_norm(h, w, 1e-5)).astype(np.float64)
    theirs = ref.norm(h, w, 1e-5).astype(np.float64)
    assert np.all(np.abs(ours - theirs) <= 2 ** -8 * np.abs(theirs) + 1e-30)


def test_norm_closed_form(exact):
    rng = np.random.default_rng(4)
    h = rng.standard_normal((5, 512)).astype(np.float32) * 3
    w = rng.standard_normal(512).astype(np.float32)
    got = widen(exact.tc_norm(h, w, 1e-5)).astype(np.float64)
    hd = h.astype(np.float64)
    want = w * hd / np.sqrt((hd * hd).mean(axis=1, keepdims=True) + 1e-5)
    assert np.all(np.abs(got - want) <= 2 ** -8 * np.abs(want) + 1e-30)


@ref_only
def test_embed_matches_reference():
    ref = O.Ref()
    rng = np.random.default_rng(6)
    emb = bf16_bits(rng.standard_normal((300, 128)))
    tokens = rng.integers(0, 300, 21).astype(np.int32)
    assert np.array_equal(ref.embed(emb, tokens), widen(emb[tokens]))


def test_norm_tree_pinned(exact):
    """The oracle's tc_norm sum follows the reference tree: on rows where the fp32
    sum depends on the grouping (tests/norm_tree.py states each closed form and
    the sum a wrong tree gives), its output equals the closed form of the stated
    sum and differs from every wrong tree's."""
    import norm_tree

    h, g, want, wrong = norm_tree.pinned_inputs()
    for i in range(h.shape[0]):
        got = exact.tc_norm(h[i:i + 1], g[i], float(norm_tree.EPS))[0]
        assert np.array_equal(got, want[i]), f"row {i}"
        for name, w in wrong[i]:
            assert not np.array_equal(got, w), f"row {i}: indistinguishable from {name}"
