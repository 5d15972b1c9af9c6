"""The allocation-free entry point stride_tc_gemm_f32x_noalloc, through the C
ABI: on two calls in a row (the second with fewer rows and another K, so the
shared device scratch holds the first call's hi/lo tiles when the second starts)
its output equals stride_tc_gemm_f32x's (caller workspace) bit for bit; calls
beyond the scratch, or that pass a workspace, are rejected before any launch."""
import numpy as np
import pytest
import torch

from stride_amd import _lib, harness, layout, tc

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


def say(*a):
    print(*a, flush=True)


def case(seed, n, k, m):
    g = torch.Generator(device=DEV).manual_seed(seed)
    w = layout.pack_tiles((torch.randn(n, k, generator=g, device=DEV) * 0.02).to(torch.bfloat16).view(torch.int16))
    x = torch.randn(m, k, generator=g, device=DEV)
    return w, x


def test_noalloc_under_graph_capture():
    """The entry point's first call in the process happens inside a HIP graph
    capture (it resolves the scratch address there); each replay, with eager
    launches of the workspace entry point and synchronizations in between, gives
    the eager bits."""
    n, k, m = 2048, 2048, 40
    say("f32x noalloc under capture: n", n, "k", k, "m", m)
    w, x = case(4, n, k, m)
    want = harness.gemm_f32x(w, x, m)
    torch.cuda.synchronize()
    got = torch.full_like(want, float("nan"))
    g = torch.cuda.CUDAGraph()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        with torch.cuda.graph(g):
            harness.gemm_f32x_noalloc(w, x, m, got)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    for i in range(3):
        got.fill_(float("nan"))
        w2, x2 = case(10 + i, 1024, 4096, 17 + i)
        harness.gemm_f32x(w2, x2, 17 + i)  # eager work on the scratch sets between replays
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(layout.untile_lanes(got, m).view(torch.int32), layout.untile_lanes(want, m).view(torch.int32)), i


def test_noalloc_matches_workspace_entry_point_twice():
    for seed, n, k, m in ((1, 2048, 8192, 200), (2, 3072, 2048, 37)):
        say("f32x noalloc: n", n, "k", k, "m", m)
        w, x = case(seed, n, k, m)
        want = harness.gemm_f32x(w, x, m)
        got = torch.full_like(want, float("nan"))
        harness.gemm_f32x_noalloc(w, x, m, got)
        torch.cuda.synchronize()
        assert torch.equal(layout.untile_lanes(got, m).view(torch.int32), layout.untile_lanes(want, m).view(torch.int32))


def test_noalloc_rejects_oversize_and_workspace():
    lib = _lib.load()
    cap = lib.stride_tc_f32x_scratch_elems()
    k = 8192
    m = cap // (2 * k) + 16  # one lane tile more than fits
    w, x = case(3, 64, k, 1)
    p = tc.TcGemmF32xParams(harness.lanes(m), harness.ptr(x), harness.mat(w), harness.ptr(x), None)
    with pytest.raises(_lib.StrideTcError, match="exceeds the scratch"):
        tc.tc_gemm_f32x_noalloc(p)
    ws = torch.empty(16, dtype=torch.int16, device=DEV)
    p = tc.TcGemmF32xParams(harness.lanes(1), harness.ptr(x), harness.mat(w), harness.ptr(x), harness.ptr(ws))
    with pytest.raises(_lib.StrideTcError, match="workspace must be null"):
        tc.tc_gemm_f32x_noalloc(p)
