"""Config 5 at its stated size: a greedy decode of a random-init Llama-3.2-1B
(16 layers, hidden 2048, 32/8 heads of 64, FFN 8192, vocab 128256, RMSNorm eps
1e-5, RoPE theta 500000 with llama3 scaling, bf16 KV in 16-token pages) with
256-token prompts of uniform random ids and 256 generated tokens per sequence, at
batch 64 and at batch 128.

Batch runs put the sequences in shuffled KV slots, shuffle the KV pages, split
prompts across prefill steps of a ragged row budget and permute the lanes every
decode step. For each sequence checked, the generated tokens, the fp32 bits of
their logits and the scheduler fingerprint (src/scheduler.cpp:15-24, 280) must
equal those of the same sequence decoded alone (batch 1: its prompt as one
256-row chunk, then 255 single-row steps), and the 64 sequences the two batches
share must agree between the batches. Step order follows the reference's
Engine::step_tensor_core (src/engine.cpp:300-462) and its scheduler's chunked
prefill (src/scheduler.cpp:127-191)."""
import numpy as np
import pytest
import torch

from stride_amd import engine

pytestmark = pytest.mark.gpu
DEV = "cuda:0"
PLEN, NEW = 256, 256


def say(*a):
    print(*a, flush=True)


@pytest.fixture(scope="module")
def model():
    cfg = engine.LlamaConfig()
    say("config5 full size: building weights")
    w = engine.Weights(cfg, DEV, seed=21, max_positions=PLEN + NEW)
    rng = np.random.default_rng(22)
    prompts = [rng.integers(0, cfg.vocab, PLEN).tolist() for _ in range(128)]
    return w, prompts


def batch_run(w, prompts, max_rows, seed):
    b = len(prompts)
    rng = np.random.default_rng(seed)
    slots = rng.permutation(b + 3)[:b]
    eng = engine.Engine(w, slots=b + 3, max_ctx=PLEN + NEW, max_rows=max_rows, page_tokens=16, shuffle_seed=seed)
    seqs = [engine.Sequence(int(slots[i]), p) for i, p in enumerate(prompts)]
    order = rng.permutation(b * PLEN)
    say(f"config5 batch {b}: prefill {b * PLEN} rows in chunks of {max_rows}")
    eng.prefill(seqs, order=order)
    say(f"config5 batch {b}: decode {NEW - 1} steps")
    eng.decode(seqs, NEW - 1, perm_seed=seed + 1)
    torch.cuda.synchronize()
    return seqs


def solo_run(w, prompt):
    eng = engine.Engine(w, slots=1, max_ctx=PLEN + NEW, max_rows=PLEN, page_tokens=16)
    s = engine.Sequence(0, prompt)
    eng.prefill([s])
    eng.decode([s], NEW - 1)
    torch.cuda.synchronize()
    return s


def same(a, b):
    return a.tokens == b.tokens and a.values == b.values and a.fingerprint == b.fingerprint


def test_config5_batch64_and_batch128_equal_alone(model):
    w, prompts = model
    b128 = batch_run(w, prompts, max_rows=1000, seed=31)
    b64 = batch_run(w, prompts[:64], max_rows=3000, seed=41)
    for s in b128:
        assert len(s.tokens) == NEW
    mismatch = [i for i in range(64) if not same(b64[i], b128[i])]
    assert not mismatch, f"sequences differ between batch 64 and batch 128: {mismatch[:8]}"
    for i in (0, 17, 63, 100, 127):
        say("config5: sequence", i, "alone")
        s = solo_run(w, prompts[i])
        assert s.tokens == b128[i].tokens, f"sequence {i}: tokens differ from batch 128"
        assert s.values == b128[i].values, f"sequence {i}: logit bits differ from batch 128"
        assert s.fingerprint == b128[i].fingerprint
        if i < 64:
            assert same(s, b64[i]), f"sequence {i}: differs from batch 64"
    # random weights still give distinct continuations
    assert len(set(tuple(s.tokens) for s in b128)) > 1
