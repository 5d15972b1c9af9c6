"""BASELINE config 5 on one GPU: a greedy decode of a random-init
Llama-3.2-1B-shaped model (16 layers, hidden 2048, 32/8 heads, FFN 8192,
vocab 128256, 16-token KV pages) through every tensor-core operator. Each
sequence's generated tokens, the fp32 bits of their logits and the scheduler
fingerprint (src/scheduler.cpp:15-24, 280) must be identical when the sequence
runs alone (batch 1, its prompt as one chunk) and when it runs in a batch with
other sequences, other KV slots, shuffled KV pages, shuffled lanes every step
and a prompt chunking that splits its prompt across steps."""
import numpy as np
import pytest
import torch

from stride_amd import engine

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


def say(*a):
    print(*a, flush=True)


def test_config5_batch_equals_alone():
    cfg = engine.LlamaConfig()
    say("config5: building weights")
    w = engine.Weights(cfg, DEV, seed=3, max_positions=256)
    rng = np.random.default_rng(4)
    batch, plen, new = 6, 70, 12
    prompts = [rng.integers(0, cfg.vocab, plen).tolist() for _ in range(batch)]
    say("config5: batch run")
    eng = engine.Engine(w, slots=batch + 2, max_ctx=plen + new, max_rows=160, page_tokens=16, shuffle_seed=5)
    slots = rng.permutation(batch + 2)[:batch]
    seqs = [engine.Sequence(int(slots[i]), p) for i, p in enumerate(prompts)]
    eng.prefill(seqs)  # 420 prompt rows in chunks of 160: prompts split across steps
    eng.decode(seqs, new - 1, perm_seed=8)
    for i in (0, 3, 5):
        say("config5: alone", i)
        solo = engine.Engine(w, slots=1, max_ctx=plen + new, max_rows=plen, page_tokens=16)
        s = engine.Sequence(0, prompts[i])
        solo.prefill([s])
        solo.decode([s], new - 1)
        assert s.tokens == seqs[i].tokens, f"sequence {i}: tokens differ"
        assert s.values == seqs[i].values, f"sequence {i}: logit bits differ"
        assert s.fingerprint == seqs[i].fingerprint
    assert len(set(tuple(s.tokens) for s in seqs)) > 1
    torch.cuda.synchronize()
