"""The full greedy decode on one GPU: a greedy decode of a random-init
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


@pytest.mark.parametrize("tied", [True, False])
def test_loaded_checkpoint_matches_float64_forward(tmp_path, tied):
    """A tiny Llama checkpoint (llama3 RoPE, GQA 4:1, non-unit norm gains) loaded
    by stride_amd.weights and decoded by the engine: every greedy token's logit
    (fp32 bits returned by the LM head) must equal a float64 forward of the same
    model that rounds to bf16 where the path stores bf16, within 2e-3 of the
    largest logit magnitude, and the token must be the float64 argmax unless the
    top two are within that margin. Then batch vs alone must agree bit for bit."""
    from stride_amd import weights
    import llama_tiny

    t, c = llama_tiny.write(str(tmp_path), seed=11, tied=tied)
    say("loaded checkpoint: tied", tied)
    w = weights.Weights.load(str(tmp_path), DEV, max_positions=64)
    rope = w.rope.cpu().numpy()
    rng = np.random.default_rng(12)
    prompts = [rng.integers(0, c["vocab_size"], n).tolist() for n in (5, 19, 33)]
    eng = engine.Engine(w, slots=3, max_ctx=48, max_rows=64, page_tokens=16, shuffle_seed=2)
    seqs = [engine.Sequence(i, p) for i, p in enumerate(prompts)]
    eng.prefill(seqs)
    eng.decode(seqs, 3, perm_seed=3)
    for s in seqs:
        toks = list(s.prompt)
        for tok, vbits in zip(s.tokens, s.values):
            ref = llama_tiny.forward_last_logits(t, c, toks, rope)
            tol = 2e-3 * np.abs(ref).max()
            val = float(np.uint32(vbits).view(np.float32))
            assert abs(val - ref[tok]) <= tol, (val, ref[tok])
            assert ref[tok] >= ref.max() - 2 * tol
            toks.append(tok)
    solo = engine.Engine(w, slots=1, max_ctx=48, max_rows=64, page_tokens=16)
    s1 = engine.Sequence(0, prompts[2])
    solo.prefill([s1])
    solo.decode([s1], 3)
    assert s1.tokens == seqs[2].tokens and s1.values == seqs[2].values and s1.fingerprint == seqs[2].fingerprint


@pytest.mark.parametrize("path", ["tc", "exact"])
def test_ledger_identical_across_scheduling(tmp_path, path):
    """stride_amd.cli on a tiny checkpoint: the JSONL ledger (tokens, logit bits,
    fingerprints) must be byte-identical whether sequences run one at a time or
    three at a time with a 16-row budget (prompts split across steps), shuffled
    rows and shuffled KV pages."""
    import json
    from stride_amd import cli
    import llama_tiny

    llama_tiny.write(str(tmp_path / "m"), seed=5)
    rng = np.random.default_rng(6)
    with open(tmp_path / "p.jsonl", "w") as f:
        for i, n in enumerate((3, 17, 9, 30, 1)):
            f.write(json.dumps({"id": 10 + i, "tokens": rng.integers(0, 1000, n).tolist()}) + "\n")
    say("ledger: sequential")
    assert cli.main(["--model", str(tmp_path / "m"), "--input", str(tmp_path / "p.jsonl"), "--output",
                     str(tmp_path / "a.jsonl"), "--max-new", "6", "--path", path]) == 0
    say("ledger: batched")
    assert cli.main(["--model", str(tmp_path / "m"), "--input", str(tmp_path / "p.jsonl"), "--output",
                     str(tmp_path / "b.jsonl"), "--max-new", "6", "--concurrency", "3", "--max-rows", "16",
                     "--row-shuffle", "5", "--kv-shuffle", "7", "--path", path]) == 0
    a, b = (tmp_path / "a.jsonl").read_text(), (tmp_path / "b.jsonl").read_text()
    assert a == b
    recs = [json.loads(line) for line in a.splitlines()]
    assert [r["id"] for r in recs] == [10, 11, 12, 13, 14] and all(len(r["tokens"]) == 6 for r in recs)
    assert all(cli.hex64(cli.fingerprint(r["tokens"], [int(v, 16) for v in r["values"]])) == r["fingerprint"]
               for r in recs)
