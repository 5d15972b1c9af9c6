"""Inputs that pin the tensor-core RMSNorm's summation tree (src/kernels_tc.cu:205-271).

The reference sums v*v of a row into 32 partials: partial t chains fmaf over the
16 columns of every column tile ct == t (mod 32), tiles ascending, columns
ascending; the partials are then added left to right, p0 + p1 + ... + p31.

Each row below is built from values 2^12 (square 2^24) and 1 (square 1), so
every partial sum is a small integer or 2^24 plus one, and a round-to-nearest-
even step decides whether a 1 survives next to 2^24 (ulp 2, 2^24 + 1 is a tie
and rounds back to 2^24) or next to 2^28 (ulp 32). The sum each row gives under
the reference's tree is stated in closed form, and so is the sum under a
plausible wrong tree; the two differ by 2^-20 of the sum or more, so a gain can
be found for some column that turns the difference into a different bf16 output.

dim = 2048 (128 column tiles); column index = 16 * tile + column.
"""
import numpy as np

DIM = 2048
EPS = np.float32(1e-5)
BIG = np.float32(4096.0)  # square 2^24


def _row():
    return np.zeros(DIM, np.float32)


def cases():
    """[(name, row, closed-form sum under the reference tree, [(wrong tree, its sum)])]."""
    out = []
    # Fold order of the partials: p0 = 2^24 (tile 0), p1..p31 = 1 (col 0 of tiles
    # 1..31). Left to right every +1 is a tie next to 2^24 and is lost: 2^24.
    # Right to left the ones sum to 31 first and 2^24 + 31 rounds to 2^24 + 32;
    # a pairwise tree or a 16-partial grouping keeps 30 of them.
    r = _row()
    r[0] = BIG
    for t in range(1, 32):
        r[16 * t] = 1.0
    out.append(("fold", r, 2.0 ** 24, [("right-to-left fold", 2.0 ** 24 + 32), ("pairwise fold", 2.0 ** 24 + 30)]))
    # Column order inside a tile: tile 0 holds 1 in columns 0..14 and 2^12 in column
    # 15. Ascending: 15, then 2^24 + 15 is a tie, rounded to even: 2^24 + 16.
    # Descending: 2^24 first, then every 1 is lost: 2^24.
    r = _row()
    r[0:15] = 1.0
    r[15] = BIG
    out.append(("columns", r, 2.0 ** 24 + 16, [("columns descending", 2.0 ** 24)]))
    # Tile order inside a partial: 1 in the 16 columns of tile 0, 2^12 in column 0 of
    # tile 32 (both partial 0). Tiles ascending: 16, then 2^24 + 16 exactly.
    # Descending: 2^24, then the ones are lost: 2^24.
    r = _row()
    r[0:16] = 1.0
    r[16 * 32] = BIG
    out.append(("tiles", r, 2.0 ** 24 + 16, [("tiles descending", 2.0 ** 24)]))
    # Partial membership (ct mod 32): 2^12 in column 0 of tiles 0..15 (partials
    # 0..15 = 2^24 each, summing exactly to 2^28) and 1 in all 16 columns of tiles
    # 16..31 and 48..63 (partials 16..31 = 32 each, exact). Folded after 2^28
    # (ulp 32) each +32 is exact: 2^28 + 16 * 32. With ct mod 16 partials, tiles
    # 16+t and 48+t join tile t's 2^24 and every 1 is lost: 2^28.
    r = _row()
    for t in range(16):
        r[16 * t] = BIG
    for t in list(range(16, 32)) + list(range(48, 64)):
        r[16 * t:16 * t + 16] = 1.0
    out.append(("membership", r, 2.0 ** 28 + 512, [("ct mod 16 partials", 2.0 ** 28)]))
    return out


def bf16_rne(a):
    u = np.ascontiguousarray(a, np.float32).view(np.uint32).astype(np.uint64)
    return ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)


def norm_from_sum(row, gains, s):
    """bf16(g * (v * r)) with r = 1 / sqrtf(s / dim + eps), all in fp32."""
    r = np.float32(1.0) / np.sqrt(np.float32(s) / np.float32(DIM) + EPS)
    return bf16_rne(gains * (row * r))


def gains_for(row, s, wrong, seed):
    """Gains (fp32) under which the bf16 output of sum s differs from that of
    every wrong sum in at least one column. Columns holding 0 get gain 1."""
    rng = np.random.default_rng(seed)
    g = np.ones(DIM, np.float32)
    cols = np.flatnonzero(row)
    r = np.float32(1.0) / np.sqrt(np.float32(s) / np.float32(DIM) + EPS)
    for i, (_, sw) in enumerate(wrong):
        rw = np.float32(1.0) / np.sqrt(np.float32(sw) / np.float32(DIM) + EPS)
        assert rw != r, "wrong sum too close to separate"
        c = cols[i % cols.size]
        cand = rng.uniform(0.5, 2.0, 1 << 18).astype(np.float32)
        v = row[c]
        hit = np.flatnonzero(bf16_rne(cand * (v * r)) != bf16_rne(cand * (v * rw)))
        assert hit.size, "no separating gain found"
        g[c] = cand[hit[0]]
    return g


def pinned_inputs():
    """(h [rows][dim], gains per row [rows][dim], expected bf16 [rows][dim], wrong
    outputs per row [(name, bf16 row)]). The reference tree's output is the closed
    form of norm_from_sum at the stated sum."""
    hs, gs, want, wrong_out = [], [], [], []
    for i, (name, row, s, wrong) in enumerate(cases()):
        g = gains_for(row, s, wrong, seed=100 + i)
        hs.append(row)
        gs.append(g)
        want.append(norm_from_sum(row, g, s))
        wrong_out.append([(w, norm_from_sum(row, g, sw)) for w, sw in wrong])
    return np.stack(hs), np.stack(gs), np.stack(want), wrong_out
