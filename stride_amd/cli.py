"""Greedy batch driver with a run ledger, the counterpart of the reference's
tools/stride_cli.cpp:

    python -m stride_amd.cli --model DIR --input prompts.jsonl --output out.jsonl
        [--path tc|exact] [--max-new N] [--concurrency C] [--max-rows R]
        [--page-tokens P] [--kv-shuffle S] [--row-shuffle S] [--use-eos]

--path tc (default) runs the tensor-core operators (bf16 tiles, bf16 KV in
--page-tokens pages); --path exact runs the exact FP32 path
(stride_amd.exact_engine: fp32 activations and KV in 64-token blocks), whose
ledger is the reference's exact-path ledger bit for bit on the same weights.

Input lines: {"id": 0, "tokens": [1, 2, 3]}. Output lines (one per prompt, in
input order): {"id": 0, "tokens": [...], "values": ["3f800000", ...],
"fingerprint": "...", "finish": "length" | "stop"} - each generated token, the
fp32 bits of its logit in hex, and the FNV-1a chain over both
(src/scheduler.cpp:15-24, 280; tools/stride_cli.cpp:102-127). --model may be
"random:SEED" for random-init Llama-3.2-1B-shaped weights.

Scheduling: up to C sequences are active; each step packs the next prompt chunk
of every prefilling sequence and one decode row of every generating sequence, at
most R rows, in an order permuted by --row-shuffle; KV pages are placed in an
order permuted by --kv-shuffle. None of this may change any output bit: two runs
with different C, R, shuffles or arrival order must write identical ledgers.
"""
from __future__ import annotations

import argparse
import collections
import json
import struct
import sys

import numpy as np

from . import engine


def hex32(bits: int) -> str:
    return f"{bits & 0xFFFFFFFF:08x}"


def hex64(v: int) -> str:
    return f"{v & 0xFFFFFFFFFFFFFFFF:016x}"


def fingerprint(tokens, values) -> int:
    """The scheduler's chain over (token id, fp32 logit bits) pairs."""
    h = engine.FNV_OFFSET
    for t, v in zip(tokens, values):
        h = engine.fnv_mix(engine.fnv_mix(h, t), v)
    return h


class _ExactSlots:
    def __init__(self, slots, capacity):
        self.slots, self.capacity = slots, capacity


class ExactCliEngine:
    """The exact-path engine behind the Scheduler's interface (step(rows, greedy)
    -> [(index, value bits)], kv.slots, kv.capacity, max_rows)."""

    def __init__(self, model, slots: int, max_ctx: int, max_rows: int, shuffle_seed: int, device: str):
        from . import exact_engine

        self.inner = exact_engine.ExactEngine(model, exact_engine.GpuBackend(device), slots, max_ctx, max_rows,
                                              shuffle_seed)
        self.kv = _ExactSlots(slots, max_ctx)
        self.max_rows = max_rows

    def step(self, rows, greedy):
        return self.inner.step(rows, greedy=greedy)[0]


class Scheduler:
    """Continuous greedy batching over one Engine (src/scheduler.cpp:127-191 in
    spirit: admission up to `concurrency`, chunked prefill within `max_rows`)."""

    def __init__(self, eng: engine.Engine, concurrency: int, max_new: int, eos=(), row_shuffle: int = 0):
        self.eng, self.concurrency, self.max_new, self.eos = eng, concurrency, max_new, set(eos)
        self.rng = np.random.default_rng(row_shuffle) if row_shuffle else None

    def run(self, prompts):
        """prompts: list of (id, tokens). Returns {id: (Sequence, finish)}."""
        eng = self.eng
        pending = collections.deque(prompts)
        free = list(range(eng.kv.slots))
        active, done = [], {}
        while pending or active:
            while pending and len(active) < self.concurrency and free:
                pid, toks = pending.popleft()
                if not toks or len(toks) + self.max_new > eng.kv.capacity:
                    raise ValueError(f"prompt {pid}: empty or longer than the KV capacity")
                s = engine.Sequence(free.pop(0), list(toks))
                s.pid, s.next_prompt = pid, 0
                active.append(s)
            order = self.rng.permutation(len(active)) if self.rng is not None else range(len(active))
            rows, owners, greedy = [], [], []
            budget = eng.max_rows
            for i in order:
                s = active[i]
                if budget == 0:
                    break
                if s.next_prompt < len(s.prompt):
                    n = min(len(s.prompt) - s.next_prompt, budget)
                    for p in range(s.next_prompt, s.next_prompt + n):
                        rows.append((s.slot, p, s.prompt[p]))
                    s.next_prompt += n
                    budget -= n
                    if s.next_prompt == len(s.prompt):
                        greedy.append(len(rows) - 1)
                        owners.append(s)
                else:
                    rows.append((s.slot, s.length - 1, s.tokens[-1]))
                    greedy.append(len(rows) - 1)
                    owners.append(s)
                    budget -= 1
            for s, (idx, val) in zip(owners, eng.step(rows, greedy)):
                s.tokens.append(idx)
                s.values.append(val)
                s.fingerprint = engine.fnv_mix(engine.fnv_mix(s.fingerprint, idx & 0xFFFFFFFF), val)
            for s in list(active):
                fin = None
                if s.tokens and s.tokens[-1] in self.eos:
                    fin = "stop"
                elif len(s.tokens) >= self.max_new:
                    fin = "length"
                if fin:
                    done[s.pid] = (s, fin)
                    active.remove(s)
                    free.append(s.slot)
        return done


def ledger_lines(prompts, done):
    for pid, _ in prompts:
        s, fin = done[pid]
        yield json.dumps({"id": pid, "tokens": s.tokens, "values": [hex32(v) for v in s.values],
                          "fingerprint": hex64(s.fingerprint), "finish": fin})


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(description=__doc__.split("\n\n")[0])
    ap.add_argument("--model", required=True)
    ap.add_argument("--input", required=True)
    ap.add_argument("--output", required=True)
    ap.add_argument("--max-new", type=int, default=16)
    ap.add_argument("--concurrency", type=int, default=1)
    ap.add_argument("--max-rows", type=int, default=256)
    ap.add_argument("--page-tokens", type=int, default=16)
    ap.add_argument("--kv-shuffle", type=int, default=0)
    ap.add_argument("--row-shuffle", type=int, default=0)
    ap.add_argument("--use-eos", action="store_true")
    ap.add_argument("--device", default="cuda:0")
    ap.add_argument("--path", choices=("tc", "exact"), default="tc")
    a = ap.parse_args(argv)

    import torch
    from . import weights

    if not torch.cuda.is_available():
        print("stride_amd.cli needs a GPU", file=sys.stderr)
        return 2
    with open(a.input) as f:
        prompts = [(int(j["id"]), [int(t) for t in j["tokens"]]) for j in map(json.loads, filter(str.strip, f))]
    longest = max(len(t) for _, t in prompts) + a.max_new
    if a.path == "exact":
        from . import exact_engine

        if a.model.startswith("random:"):
            model = exact_engine.ExactModel.random(weights.ModelConfig(), int(a.model.split(":", 1)[1]), longest + 1)
        else:
            model = exact_engine.ExactModel.load(a.model, max_positions=longest + 1)
        eng = ExactCliEngine(model, a.concurrency, longest, a.max_rows, a.kv_shuffle, a.device)
        cfg = model.cfg
    else:
        if a.model.startswith("random:"):
            w = weights.Weights.random(weights.ModelConfig(), a.device, int(a.model.split(":", 1)[1]), longest + 1)
        else:
            w = weights.Weights.load(a.model, a.device, max_positions=longest + 1)
        eng = engine.Engine(w, slots=a.concurrency, max_ctx=longest, max_rows=a.max_rows, page_tokens=a.page_tokens,
                            shuffle_seed=a.kv_shuffle)
        cfg = w.cfg
    eos = cfg.eos_tokens if a.use_eos else ()
    done = Scheduler(eng, a.concurrency, a.max_new, eos, a.row_shuffle).run(prompts)
    with open(a.output, "w") as f:
        for line in ledger_lines(prompts, done):
            f.write(line + "\n")
    print(json.dumps({"sequences": len(prompts), "generated": sum(len(s.tokens) for s, _ in done.values())}))
    return 0


if __name__ == "__main__":
    sys.exit(main())
