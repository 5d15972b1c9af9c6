"""Captured HIP graphs replay to the same bits as eager launches. The benchmark and
the engine both run the GEMMs from a graph; the cross-workgroup split combine
(arrival counters re-armed by the last workgroup, no memset node) and the greedy
LM head's candidate scratch must give the eager result on every replay, with other
eager work between replays. Each replay first restores its inputs with copy
kernels captured in the same graph."""
import hashlib

import pytest
import torch

from stride_amd import _lib, harness, layout

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


def say(*a):
    print(*a, flush=True)


def digest(t):
    return hashlib.sha256(t.cpu().numpy().tobytes()).hexdigest()


@pytest.fixture(scope="module")
def data():
    g = torch.Generator(device=DEV).manual_seed(91)

    def w(n, k):
        return layout.pack_tiles((torch.randn(n, k, generator=g, device=DEV) * 0.02).to(torch.bfloat16).view(torch.int16))

    W = dict(o=w(2048, 2048), down=w(512, 8192), w1=w(1024, 2048), w3=w(1024, 2048), lm=w(4000, 2048))
    rows = max(m for m, _ in CASES)
    x = {k: (torch.randn(rows, k, generator=g, device=DEV)).to(torch.bfloat16).view(torch.int16) for k in (2048, 8192)}
    h = torch.randn(rows, 2048, generator=g, device=DEV)
    return W, x, h


def launch_set(W, xt, xd, h_o0, h_d0, h_o, h_d, best, best0, z, m):
    h_o.copy_(h_o0)
    h_d.copy_(h_d0)
    best.copy_(best0)
    harness.gemm_residual(W["o"], xt, h_o, m)
    harness.gemm_residual(W["down"], xd, h_d, m)
    harness.mlp13(W["w1"], W["w3"], xt, m, out=z)
    harness.lm_greedy(W["lm"], xt, m, 3990, best=best)


# (M, forced configuration): the automatic choice, cross-workgroup split configurations
# of the streaming kernel (53) and of k_dec (1007), and the pipeline.
CASES = [(1, -1), (1, 53), (64, -1), (64, 1007), (128, -1), (290, -1)]


@pytest.mark.parametrize("m,cfg", CASES)
def test_graph_replays_match_eager(data, m, cfg):
    W, x, h = data
    say("graph replay M =", m, "config", cfg)
    assert x[2048].shape[0] >= m and h.shape[0] >= m, "activations must hold M rows"  # the kernels read M rows
    xt = layout.lane_tiles(x[2048][:m])
    xd = layout.lane_tiles(x[8192][:m])
    h_o0 = layout.lane_tiles(h[:m].clone())
    h_d0 = layout.lane_tiles(h[:m, :512].clone())
    h_o, h_d = torch.empty_like(h_o0), torch.empty_like(h_d0)
    best0 = harness.best_init(m, DEV)
    best = torch.empty_like(best0)
    z = torch.zeros(((m + 15) // 16, W["w1"].shape[0], 16, 16), dtype=torch.int16, device=DEV)
    _lib.set_stream_config(cfg)
    try:
        launch_set(W, xt, xd, h_o0, h_d0, h_o, h_d, best, best0, z, m)
        torch.cuda.synchronize()
        ref = [digest(t) for t in (h_o, h_d, z, best)]
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            launch_set(W, xt, xd, h_o0, h_d0, h_o, h_d, best, best0, z, m)  # warm-up on the capture stream
        torch.cuda.current_stream().wait_stream(side)
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            launch_set(W, xt, xd, h_o0, h_d0, h_o, h_d, best, best0, z, m)
        scratch_h = layout.lane_tiles(h[:m].clone())
        for rep in range(4):
            for t in (h_o, h_d, z, best):
                t.fill_(0)  # replays must rebuild every output
            graph.replay()
            torch.cuda.synchronize()
            got = [digest(t) for t in (h_o, h_d, z, best)]
            assert got == ref, f"replay {rep} differs from eager (M={m}, config {cfg})"
            harness.gemm_residual(W["o"], xt, scratch_h, m)  # eager work between replays
            torch.cuda.synchronize()
        del graph
    finally:
        _lib.set_stream_config(-1)


def test_engine_step_graph_replays_match_eager():
    """One full decode step of the engine (every layer's norm, QKV + KV append,
    attention, O, gate/up, down, then the greedy LM head) captured as a graph, as
    the benchmark runs it: each replay returns the eager step's tokens and logit
    bits (the step rewrites the same KV entries with the same values)."""
    import numpy as np

    from stride_amd import engine

    cfg = engine.LlamaConfig()
    say("engine graph: building weights")
    w = engine.Weights(cfg, DEV, seed=7, max_positions=128)
    eng = engine.Engine(w, slots=4, max_ctx=96, max_rows=96, page_tokens=16, shuffle_seed=2)
    rng = np.random.default_rng(1)
    seqs = [engine.Sequence(i, rng.integers(0, cfg.vocab, 70).tolist()) for i in range(4)]
    eng.prefill(seqs)
    rows = [(s.slot, len(s.prompt), s.tokens[-1]) for s in seqs]
    slot, pos, tok, items = eng.device_rows(rows)
    best = torch.empty((len(rows), 2), dtype=torch.int32, device=DEV)
    eng.launch(len(rows), slot, pos, tok, items, best=best)
    torch.cuda.synchronize()
    ref = digest(best)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        eng.launch(len(rows), slot, pos, tok, items, best=best)
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        eng.launch(len(rows), slot, pos, tok, items, best=best)
    for rep in range(3):
        best.fill_(0)
        graph.replay()
        torch.cuda.synchronize()
        assert digest(best) == ref, f"engine step replay {rep} differs from eager"
        eng.launch(len(rows), slot, pos, tok, items)  # eager work between replays (no LM head)
        torch.cuda.synchronize()
    del graph


@pytest.mark.parametrize("m,cfg", [(1, 53), (64, -1), (64, 1007)])
def test_two_streams_at_once(data, m, cfg):
    """Launches that use the device scratch (cross-workgroup split partials and
    counters, the greedy LM head's candidates) on two streams at the same time,
    eight rounds each with no synchronisation in between: every stream gets the
    results of its inputs run alone (each stream is given its own scratch set)."""
    W, x, h = data
    say("two streams M =", m, "config", cfg)
    g = torch.Generator(device=DEV).manual_seed(m + 7)
    xs = [x[2048][:m], (torch.randn(m, 2048, generator=g, device=DEV)).to(torch.bfloat16).view(torch.int16)]
    xds = [x[8192][:m], (torch.randn(m, 8192, generator=g, device=DEV)).to(torch.bfloat16).view(torch.int16)]
    sets = []
    for xi, xdi in zip(xs, xds):
        xt, xd = layout.lane_tiles(xi), layout.lane_tiles(xdi)
        h_o0 = layout.lane_tiles(h[:m].clone())
        h_d0 = layout.lane_tiles(h[:m, :512].clone())
        best0 = harness.best_init(m, DEV)
        z = torch.zeros(((m + 15) // 16, W["w1"].shape[0], 16, 16), dtype=torch.int16, device=DEV)
        sets.append([xt, xd, h_o0, h_d0, torch.empty_like(h_o0), torch.empty_like(h_d0), torch.empty_like(best0),
                     best0, z])
    _lib.set_stream_config(cfg)
    try:
        refs = []
        for xt, xd, h_o0, h_d0, h_o, h_d, best, best0, z in sets:
            launch_set(W, xt, xd, h_o0, h_d0, h_o, h_d, best, best0, z, m)
            torch.cuda.synchronize()
            refs.append([digest(t) for t in (h_o, h_d, z, best)])
        assert refs[0] != refs[1]
        streams = [torch.cuda.Stream(), torch.cuda.Stream()]
        for s in streams:
            s.wait_stream(torch.cuda.current_stream())
        for _ in range(8):
            for s, (xt, xd, h_o0, h_d0, h_o, h_d, best, best0, z) in zip(streams, sets):
                with torch.cuda.stream(s):
                    launch_set(W, xt, xd, h_o0, h_d0, h_o, h_d, best, best0, z, m)
        torch.cuda.synchronize()
        for ref, (xt, xd, h_o0, h_d0, h_o, h_d, best, best0, z) in zip(refs, sets):
            assert [digest(t) for t in (h_o, h_d, z, best)] == ref
    finally:
        _lib.set_stream_config(-1)
