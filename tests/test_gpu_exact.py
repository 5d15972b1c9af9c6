"""GPU exact path (include/stride_exact.h, stride_amd/csrc/exact.hip) against the
reference's own CPU exact path (src/kernels.cu compiled as C++ into
oracle/_ref/libstride_ref.so by oracle/Makefile), bit for bit: the same
operands go through the reference's k_* on the CPU and stride_k_* on the GPU,
and every output word must be identical - the reference's CPU == GPU claim on
MI355X. Shapes: one row (J = 1) and ragged batches (J = 4, rows not a multiple
of four), Llama-3.2-1B widths and small odd ones."""
import numpy as np
import pytest
import torch

from oracle import oracle as O
from stride_amd import exact, tc, weights
from stride_amd._lib import (CompactParams, EmbedParams, GemmResidualParams, LmFullParams, LmGreedyParams, Mlp13Params,
                             NormParams, QkvParams, AttentionParams, KvRef)

pytestmark = [pytest.mark.gpu, pytest.mark.skipif(not O.ref_available(), reason="oracle/_ref not built")]
DEV = "cuda:0"


def say(*a):
    print(*a, flush=True)


@pytest.fixture(scope="module")
def ref():
    return O.Ref()


def bf16(rng, *shape, std=1.0):
    return (np.ascontiguousarray(rng.standard_normal(shape) * std, np.float32).view(np.uint32) >> 16).astype(np.uint16)


def dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).to(DEV)


def groups_dev(w, order=None):
    return dev(exact.pack_groups(w.view(np.int16), order))


def x_dev(x):
    J, g, stride = exact.lane_shape(x.shape[0])
    return dev(exact.dim_major(x.astype(np.float32), stride)), J


def back(t, rows, n):
    """dim-major [n][stride] device tensor -> row-major [rows][n] numpy."""
    return t.cpu().numpy()[:n, :rows].T.copy()


# K a multiple of 256 runs the sliced four-lane kernel (eight weight groups per
# workgroup: 25 groups leave dead blocks); K = 264 the streaming one.
SHAPES = [(1, 2048, 2048), (7, 256, 512), (37, 512, 2048), (64, 2048, 8192), (9, 100, 512), (6, 256, 264)]


@pytest.mark.parametrize("m,n,k", SHAPES)
def test_lm_full_and_residual(ref, m, n, k):
    say("exact lm_full/residual", m, n, k)
    rng = np.random.default_rng(m + n)
    w = bf16(rng, n, k, std=0.02)
    x = rng.standard_normal((m, k)).astype(np.float32)
    h = rng.standard_normal((m, n)).astype(np.float32)
    wd = groups_dev(w)
    xd, J = x_dev(x)
    stride = exact.lane_shape(m)[2]
    logits = torch.zeros((wd.shape[0] * 4, stride), dtype=torch.float32, device=DEV)
    exact.k_lm_full(LmFullParams(exact.lanes(m), tc.ptr(xd), exact.mat(wd, k), tc.ptr(logits)), J)
    hd = dev(exact.dim_major(h, stride))
    exact.k_gemm_residual(GemmResidualParams(exact.lanes(m), tc.ptr(xd), exact.mat(wd, k), tc.ptr(hd)), J)
    torch.cuda.synchronize()
    assert np.array_equal(back(logits, m, n).view(np.uint32), ref.gemm(w, x).view(np.uint32))
    assert np.array_equal(back(hd, m, n).view(np.uint32), ref.gemm_residual(w, x, h).view(np.uint32))


@pytest.mark.parametrize("m,n,k", [(1, 512, 2048), (5, 256, 256), (33, 1024, 2048)])
def test_mlp13(ref, m, n, k):
    say("exact mlp13", m, n, k)
    rng = np.random.default_rng(3 * m + n)
    w1, w3 = bf16(rng, n, k, std=0.05), bf16(rng, n, k, std=0.05)
    x = rng.standard_normal((m, k)).astype(np.float32)
    xd, J = x_dev(x)
    stride = exact.lane_shape(m)[2]
    z = torch.zeros((n, stride), dtype=torch.float32, device=DEV)
    g1, g3 = groups_dev(w1), groups_dev(w3)  # kept alive: the structs hold raw device pointers
    exact.k_mlp13(Mlp13Params(exact.lanes(m), tc.ptr(xd), exact.mat(g1, k), exact.mat(g3, k), tc.ptr(z)), J)
    torch.cuda.synchronize()
    assert np.array_equal(back(z, m, n).view(np.uint32), ref.mlp13(w1, w3, x).view(np.uint32))


@pytest.mark.parametrize("m,vocab", [(1, 1000), (6, 4001), (17, 1000)])
def test_lm_greedy(ref, m, vocab):
    say("exact lm_greedy", m, vocab)
    rng = np.random.default_rng(vocab + m)
    k = 256
    n = (vocab + 3) // 4 * 4
    w = bf16(rng, n, k, std=0.05)
    w[vocab:] = 0
    w[77] = w[21]  # an exact tie between rows 21 and 77: the smaller index wins
    x = rng.standard_normal((m, k)).astype(np.float32)
    xd, J = x_dev(x)
    best = torch.zeros((m, 2), dtype=torch.int32, device=DEV)
    best[:, 0] = torch.tensor(np.float32(-np.inf)).view(torch.int32)
    best[:, 1] = -1
    wg = groups_dev(w)
    exact.k_lm_greedy(LmGreedyParams(exact.lanes(m), tc.ptr(xd), exact.mat(wg, k), vocab, tc.ptr(best)), J)
    torch.cuda.synchronize()
    b = best.cpu().numpy()
    rv, ri = ref.lm_greedy(w, vocab, x)
    assert np.array_equal(b[:, 0].view(np.uint32), rv.view(np.uint32)) and np.array_equal(b[:, 1], ri)


@pytest.mark.parametrize("m,hd", [(1, 64), (9, 64), (6, 32), (5, 128)])
def test_qkv(ref, m, hd):
    say("exact qkv", m, hd)
    rng = np.random.default_rng(m * hd)
    nkv, k = 2 * hd, 512
    nq = 4 * nkv
    wq, wk, wv = bf16(rng, nq, k, std=0.05), bf16(rng, nkv, k, std=0.05), bf16(rng, nkv, k, std=0.05)
    x = rng.standard_normal((m, k)).astype(np.float32)
    pos = rng.integers(0, 200, m).astype(np.int32)
    pos[0] = 130
    cfg = weights.ModelConfig(head_dim=hd)
    rope = weights.build_rope_table(cfg, 256)
    rq, rk, rv = ref.qkv(wq, wk, wv, x, hd, rope, pos)
    xd, J = x_dev(x)
    order_q, order_kv = exact.rope_group_rows(nq, hd), exact.rope_group_rows(nkv, hd)
    kv_heads, tokens = nkv // hd, 64
    max_blocks = 4
    group = tokens * hd
    which = group * kv_heads
    block = which * 2
    table = dev(np.random.default_rng(1).permutation(m * max_blocks).astype(np.int32).reshape(m, max_blocks))
    arena = torch.zeros(m * max_blocks * block, dtype=torch.float32, device=DEV)
    kv = KvRef(tc.ptr(arena), tc.ptr(table), block, block, which, group, max_blocks, hd)
    q = torch.zeros((m, nq), dtype=torch.float32, device=DEV)
    slots = dev(np.arange(m, dtype=np.int32))
    posd = dev(pos)
    ropd = dev(rope)
    gq, gk, gv = groups_dev(wq, order_q), groups_dev(wk, order_kv), groups_dev(wv, order_kv)
    exact.k_qkv(QkvParams(exact.lanes(m), tc.ptr(xd), exact.mat(gq, k), exact.mat(gk, k), exact.mat(gv, k), tc.ptr(q), nq,
                          kv, tc.ptr(ropd), tc.ptr(slots), tc.ptr(posd), 0, hd), J)
    torch.cuda.synchronize()
    assert np.array_equal(q.cpu().numpy().view(np.uint32), rq.view(np.uint32))
    a, t = arena.cpu().numpy(), table.cpu().numpy()
    for j in range(m):
        b = t[j, pos[j] // tokens]
        for g in range(kv_heads):
            base = b * block + g * group + (pos[j] % tokens) * hd
            assert np.array_equal(a[base:base + hd].view(np.uint32), rk[j, g * hd:(g + 1) * hd].view(np.uint32))
            assert np.array_equal(a[base + which:base + which + hd].view(np.uint32),
                                  rv[j, g * hd:(g + 1) * hd].view(np.uint32))


@pytest.mark.parametrize("m,dim", [(1, 2048), (7, 2048), (13, 512), (6, 2052), (3, 4096), (1, 16384), (5, 8192),
                                   (1, 20480)])
def test_embed_norm_compact(ref, m, dim):
    """Up to 4096 sixteen-byte items per lane group (dim for four-lane groups,
    dim / 4 for one row) the norm stages its inputs in LDS; beyond, it streams them."""
    say("exact embed/norm/compact", m, dim)
    rng = np.random.default_rng(m + dim)
    vocab = 301
    emb = bf16(rng, vocab, dim)
    tokens = rng.integers(0, vocab, m).astype(np.int32)
    J, g, stride = exact.lane_shape(m)
    h = torch.zeros((dim, stride), dtype=torch.float32, device=DEV)
    eg, td = groups_dev(emb), dev(tokens)
    exact.k_embed(EmbedParams(exact.lanes(m), tc.ptr(eg), tc.ptr(td), tc.ptr(h), dim))
    torch.cuda.synchronize()
    assert np.array_equal(back(h, m, dim), ref.embed(emb, tokens))
    hv = (rng.standard_normal((m, dim)) * 3).astype(np.float32)
    wgain = rng.standard_normal(dim).astype(np.float32)
    hd = dev(exact.dim_major(hv, stride))
    out = torch.zeros_like(hd)
    gd = dev(wgain)
    exact.k_norm(NormParams(exact.lanes(m), tc.ptr(hd), tc.ptr(out), tc.ptr(gd), dim, 1e-5), J)
    rows = np.array([m - 1, 0, m // 2], np.int32)
    comp = torch.zeros((dim, 4), dtype=torch.float32, device=DEV)
    rd = dev(rows)
    exact.k_compact(CompactParams(exact.lanes(m), tc.ptr(out), tc.ptr(comp), tc.ptr(rd), 3, 4, dim))
    torch.cuda.synchronize()
    want = ref.norm(hv, wgain, 1e-5)
    assert np.array_equal(back(out, m, dim).view(np.uint32), want.view(np.uint32))
    assert np.array_equal(comp.cpu().numpy()[:, :3].T.view(np.uint32), want[rows].view(np.uint32))


@pytest.mark.parametrize("m,n_kv,hd,cap,split", [(1, 2, 64, 300, False), (7, 8, 64, 200, False), (5, 1, 128, 700, False),
                                                 (6, 2, 32, 130, False), (7, 8, 64, 200, True), (3, 2, 128, 2048, False)])
def test_attention(ref, m, n_kv, hd, cap, split):
    """The item list the reference's engine builds (every page of every row) runs
    the one-kernel form; split = True lists each row's pages but its last in a
    first call and the last pages in a second, whose combine takes the first
    call's records from scratch; cap = 2048 (the reference's longest context,
    src/kernels.h:18) at head_dim 128 is too long for the one kernel's LDS and
    runs the page + combine pair."""
    say("exact attention", m, n_kv, hd, cap, split)
    rng = np.random.default_rng(m + hd + cap)
    slots_n = 3
    q = rng.standard_normal((m, n_kv * 4 * hd)).astype(np.float32)
    kb, vb = bf16(rng, slots_n, n_kv, cap, hd), bf16(rng, slots_n, n_kv, cap, hd)
    row_slot = rng.integers(0, slots_n, m).astype(np.int32)
    row_pos = rng.integers(0, cap, m).astype(np.int32)
    row_pos[0] = cap - 1
    want = ref.attention(q.reshape(m, n_kv * 4, hd), kb, vb, row_slot, row_pos, hd ** -0.5)
    # fp32 arena [block][layer=1][K|V][group][64 tokens][hd], blocks of a slot shuffled
    tokens = 64
    max_blocks = (cap + tokens - 1) // tokens
    group = tokens * hd
    which = group * n_kv
    block = which * 2
    perm = np.random.default_rng(2).permutation(slots_n * max_blocks).astype(np.int32)
    table = perm.reshape(slots_n, max_blocks)
    arena = np.zeros(slots_n * max_blocks * block, np.float32)
    kf = (kb.astype(np.uint32) << 16).view(np.float32)
    vf = (vb.astype(np.uint32) << 16).view(np.float32)
    for s in range(slots_n):
        for p in range(cap):
            b = table[s, p // tokens]
            for g in range(n_kv):
                base = b * block + g * group + (p % tokens) * hd
                arena[base:base + hd] = kf[s, g, p]
                arena[base + which:base + which + hd] = vf[s, g, p]
    arena_d, table_d = dev(arena), dev(table)
    max_pages = (cap + 63) // 64
    items = np.array([[j, pg] for j in range(m) for pg in range(row_pos[j] // 64 + 1)], np.int32).reshape(-1)
    rec = 8 + 4 * hd
    scratch = torch.zeros(m * n_kv * max_pages * rec, dtype=torch.float32, device=DEV)
    J, g_, stride = exact.lane_shape(m)
    out = torch.zeros((n_kv * 4 * hd, stride), dtype=torch.float32, device=DEV)
    qd, items_d, rs, rp = dev(q), dev(items), dev(row_slot), dev(row_pos)
    p = AttentionParams()
    p.l = exact.lanes(m)
    p.q, p.q_stride, p.out, p.out_cols = tc.ptr(qd), q.shape[1], tc.ptr(out), q.shape[1]
    p.kv = KvRef(tc.ptr(arena_d), tc.ptr(table_d), block, block, which, group, max_blocks, hd)
    p.row_slot, p.row_pos, p.items, p.item_count = tc.ptr(rs), tc.ptr(rp), tc.ptr(items_d), items.size // 2
    p.scratch, p.max_pages, p.rec_floats, p.layer = tc.ptr(scratch), max_pages, rec, 0
    p.n_kv, p.n_q, p.head_dim, p.scale = n_kv, 4, hd, hd ** -0.5
    if split:
        first = np.array([[j, pg] for j in range(m) for pg in range(row_pos[j] // 64)], np.int32).reshape(-1)
        second = np.array([[j, row_pos[j] // 64] for j in range(m)], np.int32).reshape(-1)
        first_d, second_d = dev(first), dev(second)
        p.items, p.item_count = tc.ptr(first_d), first.size // 2
        exact.k_attention(p)
        p.items, p.item_count = tc.ptr(second_d), second.size // 2
    exact.k_attention(p)
    torch.cuda.synchronize()
    got = back(out, m, n_kv * 4 * hd)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), f"{(got != want).sum()} mismatches"


def test_rejects_bad_lanes():
    w = torch.zeros((2, 32, 4), dtype=torch.int16, device=DEV)
    p = GemmResidualParams(exact.lanes(6), 1, exact.mat(w, 32), 1)
    p.l.stride = 6  # not a multiple of four
    from stride_amd._lib import StrideTcError
    with pytest.raises(StrideTcError, match="J = 4"):
        exact.k_gemm_residual(p, 4)
