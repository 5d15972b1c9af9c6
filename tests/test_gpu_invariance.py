"""Batch invariance on the GPU: each output row's bits (SHA-256) are identical for
every M in {1 .. 4096}, under a random permutation of the rows, and whichever
kernel family (streaming for M <= 128, LDS-tiled above) serves the call. Shapes
are Llama-3.2-1B's (hidden 2048, 32/8 heads x 64, FFN 8192, vocab 128256).

This needs no oracle: the M=4096 (or largest) run is the reference for the others.
"""
import hashlib

import numpy as np
import pytest
import torch

from stride_amd import harness, layout, synth

pytestmark = pytest.mark.gpu

DEV = "cuda:0"
MS = [1, 8, 32, 64, 128, 160, 290, 1024, 1536, 2048, 4096]


def say(*a):
    print(*a, flush=True)


def rand_bf16(g, rows, cols, std):
    return (torch.randn(rows, cols, generator=g, device=DEV) * std).to(torch.bfloat16).view(torch.int16)


def row_hashes(a: torch.Tensor):
    b = a.contiguous().cpu().numpy()
    return [hashlib.sha256(r.tobytes()).hexdigest() for r in b.reshape(b.shape[0], -1)]


@pytest.fixture(scope="module")
def gen():
    return torch.Generator(device=DEV).manual_seed(1234)


@pytest.fixture(scope="module")
def xs(gen):
    return {k: rand_bf16(gen, max(MS), k, 1.0) for k in (2048, 8192)}


def _perm(n, seed):
    return torch.from_numpy(synth.permutation(seed, n)).to(DEV)


def check_invariant(run, x_full, name, out_rows):
    """run(x_rows) -> [rows][...] output; compares every M's rows with the largest."""
    ref = run(x_full)
    ref_h = row_hashes(ref[:out_rows(x_full.shape[0])])
    for m in MS:
        say(name, "M =", m)
        out = run(x_full[:m])
        assert row_hashes(out[:m]) == ref_h[:m], f"{name}: rows differ at M={m}"
    for m in (128, 1024):
        p = _perm(m, m)
        say(name, "permuted M =", m)
        out = run(x_full[:m][p])
        h = row_hashes(out[:m])
        assert h == [ref_h[i] for i in p.tolist()], f"{name}: permutation changes bits at M={m}"


def test_residual_o_and_down(gen, xs):
    for n, k, name in ((2048, 2048, "O"), (2048, 8192, "down")):
        w = layout.pack_tiles(rand_bf16(gen, n, k, 0.02))
        h0 = torch.randn(max(MS), n, generator=gen, device=DEV)

        def _run_res(w, x, ht, m):
            harness.gemm_residual(w, layout.lane_tiles(x), ht, m)
            return layout.untile_lanes(ht, m)

        # residual rows follow their activation rows under the permutation
        ref = _run_res(w, xs[k], layout.lane_tiles(h0.clone()), max(MS))
        ref_h = row_hashes(ref)
        for m in MS:
            say(name, "M =", m)
            out = _run_res(w, xs[k][:m], layout.lane_tiles(h0[:m].clone()), m)
            assert row_hashes(out) == ref_h[:m], f"{name}: rows differ at M={m}"
        for m in (128, 1024):
            p = _perm(m, m)
            out = _run_res(w, xs[k][:m][p], layout.lane_tiles(h0[:m][p].clone()), m)
            assert row_hashes(out) == [ref_h[i] for i in p.tolist()], f"{name}: permutation, M={m}"


def test_gate_up(gen, xs):
    w1 = layout.pack_tiles(rand_bf16(gen, 8192, 2048, 0.02))
    w3 = layout.pack_tiles(rand_bf16(gen, 8192, 2048, 0.02))

    def run(x):
        m = x.shape[0]
        return layout.untile_lanes(harness.mlp13(w1, w3, layout.lane_tiles(x), m), m)

    check_invariant(run, xs[2048], "gate+up", lambda m: m)


def test_qkv(gen, xs):
    D = 64
    wq = layout.pack_tiles(rand_bf16(gen, 2048, 2048, 0.02), layout.rope_rows(2048, D))
    wk = layout.pack_tiles(rand_bf16(gen, 512, 2048, 0.02), layout.rope_rows(512, D))
    wv = layout.pack_tiles(rand_bf16(gen, 512, 2048, 0.02), layout.rope_rows(512, D))
    from oracle.oracle import rope_table

    rope = torch.from_numpy(rope_table(D, 64)).to(DEV)
    pos_all = torch.from_numpy((np.arange(max(MS)) * 7 % 64).astype(np.int32)).to(DEV)

    def run(x, pos=None):
        m = x.shape[0]
        pos = pos_all[:m] if pos is None else pos
        kv = harness.PagedKv.create(m, 64, 8, D, layers=1, page_tokens=16, device=DEV, shuffle_seed=m)
        slots = torch.arange(m, dtype=torch.int32, device=DEV)
        q = harness.qkv(wq, wk, wv, layout.lane_tiles(x), m, D, rope, slots, pos, kv)
        kk = kv.gather(0, 0, range(min(m, 64)), pos[:64].tolist(), 8, D)
        return q, kk

    qref, kref = run(xs[2048])
    qh, kh = row_hashes(qref), row_hashes(kref)
    for m in MS:
        say("qkv M =", m)
        q, kk = run(xs[2048][:m])
        assert row_hashes(q[:m]) == qh[:m], f"qkv q rows differ at M={m}"
        assert row_hashes(kk) == kh[:min(m, 64)], f"qkv k rows differ at M={m}"
    p = _perm(1024, 5)
    q, _ = run(xs[2048][:1024][p], pos_all[:1024][p])
    assert row_hashes(q[:1024]) == [qh[i] for i in p.tolist()]


def test_lm_head_greedy_and_full(gen, xs):
    vocab = 128256
    w = layout.pack_tiles(rand_bf16(gen, vocab, 2048, 0.02))
    # 1024 rows take the 256 x 256 pipeline blocks that serve M > 384; 290 the
    # 128 x 256 ones; 64 and 128 the decode kernels
    msl = [1, 64, 128, 290, 1024]
    x = xs[2048][:max(msl)]
    ref = harness.lm_greedy(w, layout.lane_tiles(x), x.shape[0], vocab)
    for m in msl:
        say("lm_greedy M =", m)
        b = harness.lm_greedy(w, layout.lane_tiles(x[:m]), m, vocab)
        assert torch.equal(b.cpu(), ref[:m].cpu()), f"argmax/value bits differ at M={m}"
    p = _perm(128, 9)
    b = harness.lm_greedy(w, layout.lane_tiles(x[:128][p]), 128, vocab)
    assert torch.equal(b.cpu(), ref[:128][p].cpu())
    # full logits: row hashes across M, the reference from M = 1024 (the 16-row
    # tile of lanes is the unit of output)
    full_ref = layout.untile_logits(harness.lm_full(w, layout.lane_tiles(x[:1024]), 1024), 1024, vocab)
    ref_h = row_hashes(full_ref)
    for m in (1, 64, 128, 400):
        say("lm_full M =", m)
        f = layout.untile_logits(harness.lm_full(w, layout.lane_tiles(x[:m]), m), m, vocab)
        assert row_hashes(f) == ref_h[:m], f"lm_full rows differ at M={m}"
        del f
    # the argmax kernel and the full-logits kernel agree bit for bit on the max
    vals = full_ref[:1024].max(dim=1)
    bv, bi = harness.best_split(ref[:1024])
    assert torch.equal(vals.values.cpu(), bv)
