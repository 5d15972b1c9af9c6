"""Tile layout helpers (CPU): packing round trips and the RoPE row order."""
import numpy as np
import torch

from stride_amd import layout, synth


def test_pack_roundtrip_numpy_and_torch():
    w = synth.bf16_normal(0, 1, 48, 64)
    t = layout.pack_tiles(w)
    assert t.shape == (3, 4, 16, 16)
    # tile (rt, ct) slot s column c is W[16 rt + s][16 ct + c]
    assert t[2, 1, 5, 7] == w[2 * 16 + 5, 16 + 7]
    assert np.array_equal(layout.unpack_rows(t), w)
    tt = layout.pack_tiles(torch.from_numpy(w.view(np.int16)))
    assert np.array_equal(tt.numpy().view(np.uint16), t)


def test_lane_tiles_pad_and_roundtrip():
    x = synth.f32_normal(0, 2, 19, 32)
    t = layout.lane_tiles(x)
    assert t.shape == (2, 2, 16, 16)
    assert np.all(t[1, :, 3:, :] == 0)  # lanes past rows are zero
    assert t[1, 1, 2, 5] == x[18, 21]
    assert np.array_equal(layout.untile_lanes(t, 19), x)


def test_rope_rows_is_the_reference_pair_order():
    D, n = 64, 256
    rows = layout.rope_rows(n, D)
    assert sorted(rows.tolist()) == list(range(n))
    # packed row 16*rt + slot: slot < 8 -> d0 + slot, else d0 + D/2 + slot - 8
    for rt in range(n // 16):
        head, d0 = rt // (D // 16), (rt % (D // 16)) * 8
        for slot in range(16):
            d = d0 + slot if slot < 8 else d0 + D // 2 + slot - 8
            assert rows[rt * 16 + slot] == head * D + d
    # each row tile's slot i and slot i+8 are a RoPE pair (d, d + D/2)
    r = rows.reshape(-1, 16)
    assert np.all(r[:, 8:] - r[:, :8] == D // 2)


def test_untile_logits():
    rt, T = 3, 2
    t = np.arange(rt * T * 256, dtype=np.float32).reshape(rt, T, 16, 16)
    a = layout.untile_logits(t, 20, 40)
    assert a.shape == (20, 40)
    assert a[17, 35] == t[35 // 16, 17 // 16, 35 % 16, 17 % 16]
