"""The exact-path engine (stride_amd.exact_engine) on the CPU, through the
reference's own exact-path operators (tests/exact_cpu.py: src/kernels.cu
compiled as C++): the step sequence of src/engine.cpp:144-297 checked without
a GPU.

* Batch invariance of the whole decode: each sequence's tokens and logit bits
  are identical alone (one row per step, the J = 1 kernels) and in a batch with
  others (lane groups of four, J = 4), with shuffled KV blocks and prompts split
  across prefill steps of a ragged row budget.
* A tiny safetensors Llama (llama3 RoPE, GQA 4:1, non-unit gains, tied and
  untied heads) loaded by ExactModel.load: every greedy token's logit is the
  float64 forward's within 1e-4 of the logit scale (the exact path keeps fp32
  everywhere), and the token is the float64 argmax unless the top two are that
  close.
"""
import numpy as np
import pytest

from oracle import oracle as O
from stride_amd import exact_engine as E
from stride_amd.weights import ModelConfig

pytestmark = pytest.mark.skipif(not O.ref_available(), reason="oracle/_ref not built (reference tree absent)")

TINY = ModelConfig(hidden=256, mlp=512, layers=2, heads=8, kv_heads=2, head_dim=32, vocab=1000,
                   rope_theta=10000.0, rope_llama3=False)


@pytest.fixture(scope="module")
def cpu():
    import exact_cpu

    return exact_cpu.CpuBackend(threads=8)


def test_exact_decode_batch_equals_alone(cpu):
    model = E.ExactModel.random(TINY, seed=3, max_positions=128)
    rng = np.random.default_rng(4)
    prompts = [rng.integers(0, TINY.vocab, n).tolist() for n in (5, 19, 33)]
    eng = E.ExactEngine(model, cpu, slots=5, max_ctx=64, max_rows=16, shuffle_seed=7)
    toks, vals, _ = E.decode(eng, prompts, 6, slots=[4, 0, 2], chunk=16)
    for i, p in enumerate(prompts):
        solo = E.ExactEngine(model, cpu, slots=1, max_ctx=64, max_rows=48)
        t1, v1, _ = E.decode(solo, [p], 6)
        assert t1[0] == toks[i] and v1[0] == vals[i], f"sequence {i}"
    assert len({tuple(t) for t in toks}) > 1


@pytest.mark.parametrize("tied", [True, False])
def test_exact_engine_matches_float64_forward(cpu, tmp_path, tied):
    import llama_tiny

    t, c = llama_tiny.write(str(tmp_path), seed=11, tied=tied)
    model = E.ExactModel.load(str(tmp_path), max_positions=64)
    rng = np.random.default_rng(12)
    prompts = [rng.integers(0, c["vocab_size"], n).tolist() for n in (5, 19)]
    eng = E.ExactEngine(model, cpu, slots=2, max_ctx=48, max_rows=16, shuffle_seed=2)
    toks, vals, _ = E.decode(eng, prompts, 4, chunk=16)
    for p, ts, vs in zip(prompts, toks, vals):
        seq = list(p)
        for tok, vbits in zip(ts, vs):
            ref = llama_tiny.forward_last_logits(t, c, seq, model.rope, round_bf16=False)
            tol = 1e-4 * np.abs(ref).max()
            val = float(np.uint32(vbits).view(np.float32))
            assert abs(val - ref[tok]) <= tol, (val, ref[tok])
            assert ref[tok] >= ref.max() - 2 * tol
            seq.append(tok)
