"""GPU parity of the non-GEMM tensor-core operators (tc_embed, tc_norm,
tc_attention, tc_compact) against the oracle, bit for bit, through the C ABI.
Shapes follow the Llama-3.2-1B decode step (hidden 2048, 8 KV heads of 64 dims,
four query heads per KV head); batches are ragged (not multiples of 16) and
positions straddle the 64-position attention pages and the 16-token KV pages."""
import numpy as np
import pytest
import torch

from stride_amd import harness, layout

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


def say(*a):
    print(*a, flush=True)


def bf16_bits(a):
    return (np.ascontiguousarray(a, np.float32).view(np.uint32) >> 16).astype(np.uint16)


def test_embed():
    say("tc_embed M=37")
    rng = np.random.default_rng(1)
    vocab, dim, m = 4096, 2048, 37
    emb = bf16_bits(rng.standard_normal((vocab, dim)) * 0.02)
    tokens = rng.integers(0, vocab, m).astype(np.int32)
    tiles = layout.pack_tiles(torch.from_numpy(emb.view(np.int16)).to(DEV))
    h = harness.embed(tiles, torch.from_numpy(tokens).to(DEV), m, dim)
    got = layout.untile_lanes(h, m).cpu().numpy()
    assert np.array_equal(got.view(np.uint32), emb[tokens].astype(np.uint32) << 16)


@pytest.mark.parametrize("per_lane,dim", [(True, 2048), (False, 2048), (True, 768), (False, 512)])
def test_norm(exact, per_lane, dim):
    say("tc_norm M=37 per_lane", per_lane, "dim", dim)
    rng = np.random.default_rng(2)
    m = 37
    h = (rng.standard_normal((m, dim)) * 2).astype(np.float32)
    w = rng.standard_normal(dim).astype(np.float32)
    ht = layout.lane_tiles(torch.from_numpy(h).to(DEV))
    x = harness.norm(ht, m, torch.from_numpy(w).to(DEV), 1e-5, per_lane=per_lane)
    torch.cuda.synchronize()
    xs = x.cpu()
    got = layout.untile_lanes(xs, m).numpy().view(np.uint16)
    assert np.array_equal(got, exact.tc_norm(h, w, 1e-5))
    pad = layout.untile_lanes(xs, 48).numpy().view(np.uint16)[m:]
    assert np.all(pad == (0x7FFF if per_lane else 0)), "padding lanes: untouched per lane, zeroed per tile"


def test_norm_rows_are_batch_invariant(exact):
    say("tc_norm invariance")
    rng = np.random.default_rng(3)
    h = rng.standard_normal((64, 2048)).astype(np.float32)
    w = rng.standard_normal(2048).astype(np.float32)
    wt = torch.from_numpy(w).to(DEV)
    full = layout.untile_lanes(harness.norm(layout.lane_tiles(torch.from_numpy(h).to(DEV)), 64, wt, 1e-5), 64).cpu()
    perm = rng.permutation(64)[:5]
    part = layout.untile_lanes(harness.norm(layout.lane_tiles(torch.from_numpy(h[perm]).to(DEV)), 5, wt, 1e-5), 5).cpu()
    assert torch.equal(part, full[perm])


@pytest.mark.parametrize("per_lane", [True, False])
def test_norm_tree_pinned_rows(exact, per_lane):
    """Rows whose fp32 sum depends on the summation tree (tests/norm_tree.py):
    the GPU output equals the oracle's, which equals the closed form of the
    reference tree's sum, for each row at lane 0 and at lane 21 of a 23-row batch."""
    import norm_tree

    say("tc_norm pinned tree rows, per_lane", per_lane)
    h, g, want, _ = norm_tree.pinned_inputs()
    rng = np.random.default_rng(9)
    for i in range(h.shape[0]):
        batch = (rng.standard_normal((23, norm_tree.DIM)) * 3).astype(np.float32)
        batch[0] = h[i]
        batch[21] = h[i]
        ht = layout.lane_tiles(torch.from_numpy(batch).to(DEV))
        x = harness.norm(ht, 23, torch.from_numpy(g[i]).to(DEV), float(norm_tree.EPS), per_lane=per_lane)
        got = layout.untile_lanes(x.cpu(), 23).numpy().view(np.uint16)
        assert np.array_equal(got[0], want[i]) and np.array_equal(got[21], want[i]), f"row {i}"
        assert np.array_equal(got, exact.tc_norm(batch, g[i], float(norm_tree.EPS)))


def test_compact():
    say("tc_compact")
    rng = np.random.default_rng(4)
    m, dim = 70, 2048
    x = bf16_bits(rng.standard_normal((m, dim)))
    rows = np.array([3, 69, 0, 17, 17, 42], np.int32)
    xt = layout.lane_tiles(torch.from_numpy(x.view(np.int16)).to(DEV))
    out = harness.compact(xt, torch.from_numpy(rows).to(DEV))
    got = layout.untile_lanes(out, rows.size).cpu().numpy().view(np.uint16)
    assert np.array_equal(got, x[rows])


@pytest.mark.parametrize("page_tokens,n_kv,hd,cap,m", [(16, 8, 64, 320, 21), (64, 8, 64, 320, 21),
                                                        (16, 2, 128, 2048, 3), (32, 1, 32, 200, 9),
                                                        (16, 8, 64, 512, 130), (16, 1, 64, 7360, 2),
                                                        (16, 1, 128, 2816, 2),
                                                        # past 512 rows item lists run the page + combine pair
                                                        (16, 2, 64, 200, 600)])
def test_attention(exact, page_tokens, n_kv, hd, cap, m):
    say("tc_attention page_tokens", page_tokens, "n_kv", n_kv, "hd", hd, "cap", cap, "m", m)
    rng = np.random.default_rng(5 + page_tokens + hd)
    slots = 6
    q = rng.standard_normal((m, n_kv * 4, hd)).astype(np.float32)
    k = bf16_bits(rng.standard_normal((slots, n_kv, cap, hd)))
    v = bf16_bits(rng.standard_normal((slots, n_kv, cap, hd)))
    slot = rng.permutation(slots)[rng.integers(0, slots, m)].astype(np.int32)
    pos = rng.integers(0, cap, m).astype(np.int32)
    pos[:min(m, 7)] = np.array([cap - 1, 0, 15, 16, 63, 64, 65])[:min(m, 7)]
    kv = harness.PagedKv.create(slots, cap, n_kv, hd, 2, page_tokens, DEV, shuffle_seed=9)
    kv.fill_dense(1, 0, torch.from_numpy(k.view(np.int16)))
    kv.fill_dense(1, 1, torch.from_numpy(v.view(np.int16)))
    scale = hd ** -0.5
    out = harness.attention(torch.from_numpy(q.reshape(m, -1)).to(DEV), kv, torch.from_numpy(slot).to(DEV),
                            torch.from_numpy(pos).to(DEV), n_kv, hd, scale, layer=1, max_pages=(cap + 63) // 64)
    got = layout.untile_lanes(out, m).cpu().numpy().view(np.uint16)
    want = exact.tc_attention(q, k, v, slot, pos, scale)
    assert np.array_equal(got, want), f"{(got != want).sum()} mismatches"
    # the one-kernel form (item_count = -1: every page of every row) gives the same bits
    say("tc_attention one kernel")
    one = harness.attention(torch.from_numpy(q.reshape(m, -1)).to(DEV), kv, torch.from_numpy(slot).to(DEV),
                            torch.from_numpy(pos).to(DEV), n_kv, hd, scale, layer=1, max_pages=(cap + 63) // 64,
                            one_kernel=True)
    got1 = layout.untile_lanes(one, m).cpu().numpy().view(np.uint16)
    assert np.array_equal(got1, want), f"one kernel: {(got1 != want).sum()} mismatches"


def test_attention_item_lists(exact):
    """The item-list semantics of the page + combine pair (src/engine.cpp:93-103,
    src/kernels_tc.cu:668-679) hold for any list: the engine's own list (checked on
    the device, one kernel), the same items shuffled, and partial lists whose
    unlisted pages are combined from the records left in scratch. The one-kernel
    form (max_pages 44 fits its LDS at head_dim 128) and the pair (max_pages 60
    does not) agree bit for bit on a partial list."""
    n_kv, hd, cap, m, page_tokens = 2, 128, 2816, 5, 16
    rng = np.random.default_rng(21)
    slots = 5
    q = rng.standard_normal((m, n_kv * 4, hd)).astype(np.float32)
    k = bf16_bits(rng.standard_normal((slots, n_kv, cap, hd)))
    v = bf16_bits(rng.standard_normal((slots, n_kv, cap, hd)))
    slot = rng.permutation(slots).astype(np.int32)
    pos = np.array([cap - 1, 0, 700, 64, 1500], np.int32)
    kv = harness.PagedKv.create(slots, cap, n_kv, hd, 1, page_tokens, DEV, shuffle_seed=4)
    kv.fill_dense(0, 0, torch.from_numpy(k.view(np.int16)))
    kv.fill_dense(0, 1, torch.from_numpy(v.view(np.int16)))
    scale = hd ** -0.5
    want = exact.tc_attention(q, k, v, slot, pos, scale)
    qd, sd, pd = torch.from_numpy(q.reshape(m, -1)).to(DEV), torch.from_numpy(slot).to(DEV), torch.from_numpy(pos).to(DEV)
    full = [(j, pg) for j in range(m) for pg in range((int(pos[j]) >> 6) + 1)]

    def run(items, max_pages, scratch):
        it = torch.tensor(items, dtype=torch.int32, device=DEV).reshape(-1)
        out = harness.attention(qd, kv, sd, pd, n_kv, hd, scale, layer=0, max_pages=max_pages, items=it,
                                scratch=scratch)
        return layout.untile_lanes(out, m).cpu().numpy().view(np.uint16)

    rec = 4 * hd + 8
    scratch = lambda mp: torch.zeros(m * n_kv * mp * rec, dtype=torch.float32, device=DEV)
    s44 = scratch(44)
    say("tc_attention item list: engine order")
    assert np.array_equal(run(full, 44, s44), want)
    assert int(torch.count_nonzero(s44)) == 0  # whole rows keep their records in LDS
    say("tc_attention item list: shuffled")
    shuffled = [full[i] for i in rng.permutation(len(full))]
    assert np.array_equal(run(shuffled, 44, s44), want)
    say("tc_attention item list: last pages only, earlier records from scratch")
    last = [(j, int(pos[j]) >> 6) for j in range(m)]
    assert np.array_equal(run(last, 44, s44), want)
    say("tc_attention item list: partial list over empty scratch, one kernel vs pair")
    got44 = run(last[::2], 44, scratch(44))
    got60 = run(last[::2], 60, scratch(60))
    assert np.array_equal(got44, got60)
    multi = [j for j in range(m) if pos[j] >= 64]
    assert not np.array_equal(got44[multi], want[multi])


def test_attention_rejects_bad_arguments():
    say("tc_attention rejects")
    kv = harness.PagedKv.create(1, 64, 1, 64, 1, 16, DEV)
    q = torch.zeros((1, 4 * 64), device=DEV)
    z = torch.zeros(1, dtype=torch.int32, device=DEV)
    from stride_amd import _lib, tc
    p = tc.AttentionParams()
    p.l = tc.lanes(1)
    p.q, p.q_stride, p.out, p.out_cols = tc.ptr(q), 256, tc.ptr(q), 256
    p.kv = kv.ref
    p.row_slot = p.row_pos = p.items = tc.ptr(z)
    p.item_count, p.scratch, p.max_pages, p.rec_floats = 1, tc.ptr(q), 1, 264
    p.n_kv, p.n_q, p.head_dim, p.scale = 1, 2, 64, 0.125
    with pytest.raises(_lib.StrideTcError, match="four query heads"):
        tc.tc_attention(p)
