"""The exact path end to end on the GPU: stride_amd.exact_engine driving the
MI355X exact-path kernels (stride_k_*) against the same engine driving the
reference's own exact-path operators on the CPU (tests/exact_cpu.py: its
src/kernels.cu compiled as C++). Same weights, prompts, KV block shuffle and
prefill chunking; every generated token, the fp32 bits of every greedy logit and
the full logits of the last step must be identical: the reference's claim of
byte-identical exact-path logits across devices (README.md:57) for a whole model
(src/engine.cpp:144-297)."""
import numpy as np
import pytest

from oracle import oracle as O
from stride_amd import exact_engine as E
from stride_amd.weights import ModelConfig

pytestmark = [pytest.mark.gpu, pytest.mark.skipif(not O.ref_available(), reason="oracle/_ref not built")]


def say(*a):
    print(*a, flush=True)


@pytest.fixture(scope="module")
def backends():
    import exact_cpu

    return exact_cpu.CpuBackend(threads=16), E.GpuBackend("cuda:0")


def run_both(backends, model, prompts, new, max_ctx, max_rows, chunk, slots, shuffle):
    out = []
    for be in backends:
        eng = E.ExactEngine(model, be, slots=max(slots) + 1, max_ctx=max_ctx, max_rows=max_rows, shuffle_seed=shuffle)
        out.append(E.decode(eng, prompts, new, slots=slots, chunk=chunk, full_last=True))
        del eng
    return out


def test_exact_engine_gpu_equals_cpu_tiny(backends):
    cfg = ModelConfig(hidden=256, mlp=512, layers=2, heads=8, kv_heads=2, head_dim=32, vocab=1000,
                      rope_theta=10000.0, rope_llama3=False)
    model = E.ExactModel.random(cfg, seed=5, max_positions=128)
    rng = np.random.default_rng(6)
    prompts = [rng.integers(0, cfg.vocab, n).tolist() for n in (1, 7, 30, 12)]
    say("exact engine tiny: CPU and GPU")
    (tc, vc, fc), (tg, vg, fg) = run_both(backends, model, prompts, 8, 64, 16, 13, [3, 0, 5, 1], 9)
    assert tg == tc and vg == vc
    for a, b in zip(fg, fc):
        assert np.array_equal(a.view(np.uint32), b.view(np.uint32))


def test_exact_engine_gpu_equals_cpu_llama_1b(backends):
    cfg = ModelConfig()
    say("exact engine Llama-3.2-1B: random weights")
    model = E.ExactModel.random(cfg, seed=7, max_positions=64)
    rng = np.random.default_rng(8)
    prompts = [rng.integers(0, cfg.vocab, n).tolist() for n in (6, 9)]
    say("exact engine Llama-3.2-1B: CPU and GPU")
    (tc, vc, fc), (tg, vg, fg) = run_both(backends, model, prompts, 3, 32, 16, 8, [1, 0], 3)
    assert tg == tc and vg == vc
    for a, b in zip(fg, fc):
        assert np.array_equal(a.view(np.uint32), b.view(np.uint32))


def test_exact_ledger_gpu_equals_cpu(backends, tmp_path):
    """The scheduler's ledger (tokens, logit bits, fingerprints; continuous
    batching of 5 prompts, 3 at a time, 16-row budget, shuffled rows and KV
    blocks) on the exact path: GPU kernels and the reference's CPU operators
    write byte-identical ledgers for a loaded checkpoint."""
    from stride_amd import cli
    import llama_tiny

    llama_tiny.write(str(tmp_path / "m"), seed=5)
    model = E.ExactModel.load(str(tmp_path / "m"), max_positions=64)
    rng = np.random.default_rng(6)
    prompts = [(10 + i, rng.integers(0, 1000, n).tolist()) for i, n in enumerate((3, 17, 9, 30, 1))]

    class Adapter:
        def __init__(self, be):
            self.inner = E.ExactEngine(model, be, slots=3, max_ctx=40, max_rows=16, shuffle_seed=7)
            self.kv = type("Kv", (), {"slots": 3, "capacity": 40})()
            self.max_rows = 16

        def step(self, rows, greedy):
            return self.inner.step(rows, greedy=greedy)[0]

    ledgers = []
    for be in backends:
        say("exact ledger on", type(be).__name__)
        done = cli.Scheduler(Adapter(be), 3, 6, (), row_shuffle=5).run(prompts)
        ledgers.append("\n".join(cli.ledger_lines(prompts, done)))
    assert ledgers[0] == ledgers[1]
