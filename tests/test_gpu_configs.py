"""Every decode-regime kernel configuration (in-workgroup split, cross-workgroup
split, x staged in LDS or not, any register blocking, weights streamed to
registers with activations in an LDS ring) must produce bit-identical outputs:
the configuration is a speed choice, never a numerical one."""
import hashlib

import pytest
import torch

from stride_amd import _lib, harness, layout

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


def say(*a):
    print(*a, flush=True)


def digest(t):
    torch.cuda.synchronize()
    return hashlib.sha256(t.cpu().numpy().tobytes()).hexdigest()


@pytest.fixture(scope="module")
def setup():
    g = torch.Generator(device=DEV).manual_seed(77)

    def w(n, k, rows=None):
        return layout.pack_tiles((torch.randn(n, k, generator=g, device=DEV) * 0.02).to(torch.bfloat16).view(torch.int16), rows)

    W = dict(o=w(2048, 2048), o_odd=w(592, 2048), down=w(512, 8192), w1=w(1024, 2048), w3=w(1024, 2048), w1b=w(8192, 2048), w3b=w(8192, 2048), lm=w(4000, 2048), lm1=w(16400, 2048),
             q=w(512, 2048, layout.rope_rows(512, 64)), k=w(128, 2048, layout.rope_rows(128, 64)),
             v=w(128, 2048, layout.rope_rows(128, 64)),
             # 20 + 4 + 4 row tiles: three-tile flat blocks straddle the Q/K boundary
             # and the last block is partial
             q5=w(320, 2048, layout.rope_rows(320, 64)), k1=w(64, 2048, layout.rope_rows(64, 64)),
             v1=w(64, 2048, layout.rope_rows(64, 64)))
    x = {k: (torch.randn(128, k, generator=g, device=DEV)).to(torch.bfloat16).view(torch.int16) for k in (2048, 8192)}
    h = torch.randn(128, 2048, generator=g, device=DEV)
    W["rope"] = torch.rand(17, 32, 2, generator=g, device=DEV)
    return W, x, h


def run_all(W, x, h, m):
    out = {}
    xt = layout.lane_tiles(x[2048][:m])
    ht = layout.lane_tiles(h[:m].clone())
    harness.gemm_residual(W["o"], xt, ht, m)
    out["o"] = digest(ht)
    # 37 row tiles: every row blocking leaves a partial last block, whose missing
    # tiles the cross-workgroup split fold must skip
    ho = layout.lane_tiles(h[:m, :592].clone())
    harness.gemm_residual(W["o_odd"], xt, ho, m)
    out["o_odd"] = digest(ho)
    hd = layout.lane_tiles(h[:m, :512].clone())
    harness.gemm_residual(W["down"], layout.lane_tiles(x[8192][:m]), hd, m)
    out["down"] = digest(hd)
    out["gate_up"] = digest(harness.mlp13(W["w1"], W["w3"], xt, m))
    out["gate_up1"] = digest(harness.mlp13(W["w1b"], W["w3b"], xt, m))  # Llama-3.2-1B shape: a single split
    out["lm"] = digest(harness.lm_greedy(W["lm"], xt, m, 3990))
    out["lm1"] = digest(harness.lm_greedy(W["lm1"], xt, m, 16390))  # a single split
    out["lm1_full"] = digest(harness.lm_full(W["lm1"], xt, m))
    kv = harness.PagedKv.create(m, 16, 2, 64, 1, 16, DEV)
    rope = W["rope"]
    q = harness.qkv(W["q"], W["k"], W["v"], xt, m, 64, rope, torch.arange(m, dtype=torch.int32, device=DEV),
                    torch.full((m,), 5, dtype=torch.int32, device=DEV), kv)
    out["qkv"] = digest(q) + digest(kv.arena)
    kv1 = harness.PagedKv.create(m, 16, 1, 64, 1, 16, DEV)
    q1 = harness.qkv(W["q5"], W["k1"], W["v1"], xt, m, 64, rope, torch.arange(m, dtype=torch.int32, device=DEV),
                     torch.full((m,), 5, dtype=torch.int32, device=DEV), kv1)
    out["qkv_odd"] = digest(q1) + digest(kv1.arena)
    return out


@pytest.mark.parametrize("m", [1, 20, 64, 128])
def test_all_configs_identical(setup, m):
    W, x, h = setup
    cfgs = _lib.stream_configs()
    _lib.set_stream_config(-1)
    ref = run_all(W, x, h, m)
    try:
        for i in range(len(cfgs)):
            say("config", i, cfgs[i], "M =", m)
            _lib.set_stream_config(i)
            got = run_all(W, x, h, m)
            for k in ref:
                assert got[k] == ref[k], f"config {i} {cfgs[i]} changes {k} bits at M={m}"
    finally:
        _lib.set_stream_config(-1)


@pytest.mark.parametrize("m", [20, 128, 150, 290, 1024])
def test_all_prefill_configs_identical(setup, m):
    """The same for the prefill (LDS-pipelined) kernel configurations; their
    outputs must also match the decode kernels row for row."""
    W, x, h = setup
    xx = {k: torch.cat([v] * 9)[:m] for k, v in x.items()}
    hh = torch.cat([h] * 9)[:m]
    _lib.set_stream_config(-1)
    ref = run_all(W, xx, hh, m)
    try:
        for i in range(_lib.pipe_config_count()):
            say("prefill config", i, "M =", m)
            _lib.set_stream_config(-3 - i)
            got = run_all(W, xx, hh, m)
            for k in ref:
                assert got[k] == ref[k], f"prefill config {i} changes {k} bits at M={m}"
    finally:
        _lib.set_stream_config(-1)


@pytest.mark.parametrize("m", [1, 20, 64, 128])
def test_all_dec_configs_identical(setup, m):
    W, x, h = setup
    _lib.set_stream_config(-1)
    ref = run_all(W, x, h, m)
    try:
        for i in range(_lib.dec_config_count()):
            say("dec config", i, "M =", m)
            _lib.set_stream_config(_lib.DEC_CONFIG_BASE + i)
            got = run_all(W, x, h, m)
            for k in ref:
                assert got[k] == ref[k], f"dec config {i} changes {k} bits at M={m}"
    finally:
        _lib.set_stream_config(-1)
