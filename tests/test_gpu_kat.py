"""Hardware known-answer tests on the GPU (kernels in tests/kat/mfma_kat.hip).

MFMA position invariance (the gfx950 counterpart of the reference's tc_probe Q1,
tools/tc_probe.cu:106-139, reports/g3/tc_probe.txt:1): permuting the rows of A
(weights) and the lanes of B (activations) inside a tile, with C permuted the same
way, must permute the v_mfma_f32_16x16x32_bf16 output element for element, bit for
bit. This is the hardware fact the whole batch-invariance design rests on: an
output element's bits depend only on its own row, lane and K chunk, never on where
in the tile that row or lane sits.
"""
import os
import sys

import pytest
import torch

sys.path.insert(0, os.path.join(os.path.dirname(os.path.abspath(__file__)), "kat"))
import kat  # noqa: E402

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


def stream():
    return torch.cuda.current_stream().cuda_stream


def test_mfma_position_invariance():
    tiles = 4096
    g = torch.Generator(device=DEV).manual_seed(3)
    # A chunk: [t][2 col tiles][16 rows][16 cols]; B chunk: [t][2][16 lanes][16 cols]; C: [t][16 lanes][16 rows]
    a = torch.randn(tiles, 2, 16, 16, generator=g, device=DEV).to(torch.bfloat16)
    b = torch.randn(tiles, 2, 16, 16, generator=g, device=DEV).to(torch.bfloat16)
    c = torch.randn(tiles, 16, 16, generator=g, device=DEV)
    out = torch.empty_like(c)
    kat.mfma_tiles(a.view(torch.int16), b.view(torch.int16), c, out, stream())
    # float64 reference: out[t][n][m] = c[t][n][m] + sum_k A[t][m][k] B[t][n][k]
    A = a.double().permute(0, 2, 1, 3).reshape(tiles, 16, 32)
    B = b.double().permute(0, 2, 1, 3).reshape(tiles, 16, 32)
    ref = c.double() + torch.einsum("tmk,tnk->tnm", A, B)
    assert torch.allclose(out.double(), ref, atol=1e-5, rtol=1e-5)
    rp = torch.stack([torch.randperm(16, generator=g, device=DEV) for _ in range(tiles)])
    lp = torch.stack([torch.randperm(16, generator=g, device=DEV) for _ in range(tiles)])
    t = torch.arange(tiles, device=DEV)[:, None]
    ap = a[t, :, rp].permute(0, 2, 1, 3).contiguous()          # rows permuted
    bp = b[t, :, lp].permute(0, 2, 1, 3).contiguous()          # lanes permuted
    cp = c[t, lp][t[:, :, None], torch.arange(16, device=DEV)[None, :, None], rp[:, None, :]].contiguous()
    outp = torch.empty_like(c)
    kat.mfma_tiles(ap.view(torch.int16), bp.view(torch.int16), cp, outp, stream())
    expect = out[t, lp][t[:, :, None], torch.arange(16, device=DEV)[None, :, None], rp[:, None, :]]
    same = int((outp.view(torch.int32) == expect.contiguous().view(torch.int32)).sum())
    print(f"MFMA row/lane permutation: {same} / {outp.numel()} elements bit-identical", flush=True)
    assert same == outp.numel()


def test_mfma_shapes_equivalent():
    """One v_mfma_f32_16x16x32_bf16 per 32-column chunk and two chained
    v_mfma_f32_32x32x16_bf16 (columns 0-15, then 16-31) give the same bits on
    gfx950, for chains of up to 64 chunks and operands spread over 20 binary
    orders of magnitude. Either shape may therefore implement the chunk step of
    the batch-invariance contract; this pins that fact for the build's kernels."""
    g = torch.Generator(device=DEV).manual_seed(5)
    for chunks in (1, 2, 64):
        cases = 512
        a = torch.randn(cases, 32, 32 * chunks, generator=g, device=DEV)
        b = torch.randn(cases, 32, 32 * chunks, generator=g, device=DEV)
        a = a * torch.exp2(torch.randint(-10, 10, a.shape, generator=g, device=DEV).float())
        b = b * torch.exp2(torch.randint(-10, 10, b.shape, generator=g, device=DEV).float())
        a, b = a.to(torch.bfloat16), b.to(torch.bfloat16)
        c0 = torch.randn(cases, 32, 32, generator=g, device=DEV)
        o16, o32 = torch.empty_like(c0), torch.empty_like(c0)
        kat.mfma_equiv(a.view(torch.int16), b.view(torch.int16), c0, o16, o32, chunks, stream())
        torch.cuda.synchronize()
        ref = c0.double() + torch.einsum("tmk,tnk->tmn", a.double(), b.double())
        assert torch.allclose(o16.double(), ref, rtol=1e-3, atol=1e-3 * ref.abs().max().item())
        assert torch.equal(o16.view(torch.int32), o32.view(torch.int32)), f"shapes differ at chunks={chunks}"
