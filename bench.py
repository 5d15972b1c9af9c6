"""Benchmark: the Llama-3.2-1B decode-step GEMM set on one MI355X.

A "step" is one decode step's worth of linear layers for a batch of M rows
(the decode GEMM set and the LM head): for each of 16 layers, fused QKV (N=3072, K=2048,
RoPE + bf16 KV append), O + residual (2048 x 2048), gate+up + SiLU (2 x 8192 x
2048) and down + residual (2048 x 8192), then the LM head with greedy argmax
(128256 x 2048). Weights are random-init bf16 ~N(0, 0.02) in the reference tile
layout, 16 distinct layers (2.47 GB per step, far above the 256 MB MALL), so the
weights stream from HBM as in a real decode. Inputs are resident in HBM before
the timed region. Attention, norms and embedding are not GEMMs and are not in the
step; their activation buffers hold fixed synthetic tiles.

value = decode tokens/s of the GEMM path = M * steps / time, the steps launched from
the host on one stream as the reference engine launches them (the same step as a
HIP-graph replay is reported beside it).

Printed as one JSON line with a per-GEMM table (GB/s, TFLOP/s, fraction of the
HBM roofline at decode, of the MFMA roofline at prefill), the roofline object of
the dominant kernel measured live with HIP events on the launch stream, and a CPU
baseline: the reference's exact path (oracle/_ref) timed on this host's cores.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0
MFMA_BF16_PEAK_TFLOPS = 2500.0

LAYERS, HIDDEN, FFN, HEADS, KV_HEADS, HEAD_DIM, VOCAB = 16, 2048, 8192, 32, 8, 64, 128256


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--m", type=int, default=128, help="decode batch (activation rows)")
    ap.add_argument("--table", type=int, default=1, help="per-GEMM table over M (0 to skip)")
    ap.add_argument("--cpu-seconds", type=float, default=15.0, help="CPU baseline budget (0 to skip)")
    ap.add_argument("--cpu-threads", type=int, default=0,
                    help="threads for the CPU baseline (0: the cores this process may use, at most 16)")
    ap.add_argument("--library", type=int, default=1,
                    help="also time torch.matmul (hipBLASLt) bf16 on the five shapes at M=128, 2048, 4096 as context "
                    "(0 to skip)")
    ap.add_argument("--op", default="", help="time only this GEMM (qkv, o, gate_up, down, lm_head) at --m and print "
                    "its JSON (for kernel-level profiles)")
    ap.add_argument("--engine-only", type=int, default=0,
                    help="run only the full decode step (for kernel profiles of it) and print its JSON")
    ap.add_argument("--engine", type=int, default=1,
                    help="also time one full decode step of the engine (0 to skip)")
    ap.add_argument("--step-only", type=int, default=0,
                    help="run only the measured steps (host-launched, no graph, no per-op timing; for kernel "
                    "profiles of the step as it is measured) and print its time")
    ap.add_argument("--exact-step", type=int, default=0,
                    help="time the exact FP32 path's whole decode step (random-init Llama-3.2-1B, bf16 weights, "
                    "batch 1 and 32, position 100) and print its JSON")
    ap.add_argument("--summarize-trace", default="",
                    help="print per-kernel launch counts and durations from a rocprofv3 kernel_trace.csv and exit")
    ap.add_argument("--summarize-counters", default="",
                    help="print the average value per dispatch of each counter per kernel from a rocprofv3 "
                    "counter_collection.csv and exit")
    ap.add_argument("--traffic-from", default="",
                    help="FETCH_CSV,WRITE_CSV: print the HBM bytes per launch of each kernel from a rocprofv3 "
                    "FETCH_SIZE run and a WRITE_SIZE run of this benchmark with --copy-calib-mib 512 (the JSON "
                    "the roofline's traffic field reads) and exit")
    ap.add_argument("--copy-calib-mib", type=int, default=0,
                    help="also run one plain device copy of this size (calibrates FETCH_SIZE/WRITE_SIZE counters)")
    return ap.parse_args()


class Model:
    """Random-init Llama-3.2-1B-shaped weights in tile layout, on the GPU."""

    def __init__(self, torch, dev):
        from stride_amd import layout

        g = torch.Generator(device=dev).manual_seed(0)

        def w(n, k, rows=None):
            t = (torch.randn(n, k, generator=g, device=dev) * 0.02).to(torch.bfloat16).view(torch.int16)
            return layout.pack_tiles(t, rows)

        self.layers = []
        for _ in range(LAYERS):
            self.layers.append(dict(
                q=w(HEADS * HEAD_DIM, HIDDEN, layout.rope_rows(HEADS * HEAD_DIM, HEAD_DIM)),
                k=w(KV_HEADS * HEAD_DIM, HIDDEN, layout.rope_rows(KV_HEADS * HEAD_DIM, HEAD_DIM)),
                v=w(KV_HEADS * HEAD_DIM, HIDDEN, layout.rope_rows(KV_HEADS * HEAD_DIM, HEAD_DIM)),
                o=w(HIDDEN, HEADS * HEAD_DIM), w1=w(FFN, HIDDEN), w3=w(FFN, HIDDEN), w2=w(HIDDEN, FFN)))
        self.lm = w(VOCAB, HIDDEN)
        self._torch = torch
        self._rot = {}
        torch.cuda.synchronize()

    def rotation(self, name):
        """Distinct weight sets for timing `name` alone: the 16 layers, extended
        with copies (distinct memory) until one pass over them reads at least
        ROTATION_BYTES, so the 256 MB MALL cannot serve a repeat. The LM head is
        one matrix; two copies of it are rotated."""
        if name not in self._rot:
            keys = OP_WEIGHTS[name]
            if name == "lm_head":
                sets = [{"lm": self.lm}, {"lm": self.lm.clone()}]
            else:
                sets = [{k: L[k] for k in keys} for L in self.layers]
                per = sum(sets[0][k].numel() * 2 for k in keys)
                i = 0
                while len(sets) * per < ROTATION_BYTES:
                    sets.append({k: self.layers[i % LAYERS][k].clone() for k in keys})
                    i += 1
            self._torch.cuda.synchronize()
            self._rot[name] = sets
        return self._rot[name]


class Buffers:
    def __init__(self, torch, dev, m):
        from stride_amd import harness, layout
        from stride_amd.harness import PagedKv

        g = torch.Generator(device=dev).manual_seed(1)
        T = (m + 15) // 16
        self.m = m

        def act(k):
            x = (torch.randn(m, k, generator=g, device=dev)).to(torch.bfloat16).view(torch.int16)
            return layout.lane_tiles(x, T)

        self.x = act(HIDDEN)
        self.attn = act(HEADS * HEAD_DIM)
        self.h = layout.lane_tiles(torch.randn(m, HIDDEN, generator=g, device=dev), T)
        self.z = torch.zeros((T, FFN // 16, 16, 16), dtype=torch.int16, device=dev)
        self.q = torch.zeros((m, HEADS * HEAD_DIM), dtype=torch.float32, device=dev)
        self.kv = PagedKv.create(m, 16, KV_HEADS, HEAD_DIM, LAYERS, 16, dev, shuffle_seed=3)
        half = HEAD_DIM // 2
        pos = torch.arange(17, dtype=torch.float64, device=dev)[:, None]
        inv = 1.0 / (500000.0 ** (torch.arange(half, dtype=torch.float64, device=dev) * 2 / HEAD_DIM))
        ang = pos * inv
        self.rope = torch.stack([ang.cos(), ang.sin()], dim=-1).float().contiguous()
        self.slots = torch.arange(m, dtype=torch.int32, device=dev)
        self.pos = torch.full((m,), 10, dtype=torch.int32, device=dev)
        self.best = harness.best_init(m, dev)


# Weights each op reads, and the least bytes one pass of a per-op timing graph reads.
OP_WEIGHTS = {"qkv": ("q", "k", "v"), "o": ("o",), "gate_up": ("w1", "w3"), "down": ("w2",), "lm_head": ("lm",)}
ROTATION_BYTES = 512 << 20


def op_launch(name, W, b, li=0):
    """One launch of op `name` over weight set W (a dict holding OP_WEIGHTS[name])."""
    from stride_amd import harness

    m = b.m
    if name == "qkv":
        return lambda: harness.qkv(W["q"], W["k"], W["v"], b.x, m, HEAD_DIM, b.rope, b.slots, b.pos, b.kv,
                                   layer=li % LAYERS, q_out=b.q)
    if name == "o":
        return lambda: harness.gemm_residual(W["o"], b.attn, b.h, m)
    if name == "gate_up":
        return lambda: harness.mlp13(W["w1"], W["w3"], b.x, m, out=b.z)
    if name == "down":
        return lambda: harness.gemm_residual(W["w2"], b.z, b.h, m)
    # best is re-initialised before every argmax, as the engine uploads {-inf, -1}
    # each step (reference src/engine.cpp:423-424); the reset is part of the op.
    return lambda: (harness.best_reset(b.best), harness.lm_greedy(W["lm"], b.x, m, VOCAB, best=b.best))


def rotated_ops(model, b, names):
    """(name, launch) pairs for per-op timing: each op over its rotation set."""
    return [(n, op_launch(n, W, b, li)) for n in names for li, W in enumerate(model.rotation(n))]


def step_ops(model, b):
    """The launches of one decode step, as (name, callable) pairs."""
    ops = []
    for li, L in enumerate(model.layers):
        for n in ("qkv", "o", "gate_up", "down"):
            ops.append((n, op_launch(n, L, b, li)))
    ops.append(("lm_head", op_launch("lm_head", {"lm": model.lm}, b)))
    return ops


# Algorithmic work per launch: FLOPs = 2 M N K; bytes = weights + activations in +
# outputs (fp32 h read+write for residual GEMMs; bf16 z; fp32 q + bf16 k, v; 8 B
# per row for the argmax).
def work(name, m):
    if name == "qkv":
        n, k = (HEADS + 2 * KV_HEADS) * HEAD_DIM, HIDDEN
        out = 4 * m * HEADS * HEAD_DIM + 2 * m * 2 * KV_HEADS * HEAD_DIM
    elif name == "o":
        n, k = HIDDEN, HEADS * HEAD_DIM
        out = 8 * m * n
    elif name == "gate_up":
        n, k = 2 * FFN, HIDDEN
        out = 2 * m * FFN
    elif name == "down":
        n, k = HIDDEN, FFN
        out = 8 * m * n
    else:
        n, k = VOCAB, HIDDEN
        out = 8 * m
    return 2.0 * m * n * k, 2.0 * n * k + 2.0 * m * k + out


def rotated_bytes(model, name):
    """Weight bytes one pass over op `name`'s rotation set reads."""
    return int(sum(t.numel() * 2 for W in model.rotation(name) for t in W.values()))


def capture(torch, fns, reps=1):
    """A HIP graph of `reps` passes over the launches in `fns` (the C-ABI entry
    points launch on torch's current stream, which is the capture stream here)."""
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for f in fns:
            f()
    torch.cuda.current_stream().wait_stream(side)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        for _ in range(reps):
            for f in fns:
                f()
    g.replay()
    torch.cuda.synchronize()
    return g


def time_ops(torch, ops, reps, replays=5):
    """Device time per launch of each op name: a HIP graph of `reps` passes over
    that op's launches (one per weight set of its rotation, so weights stream from
    HBM), replayed `replays` times, each replay between HIP events recorded on the
    replay stream. Returns {name: (median, min, max)} seconds per launch over the
    replays."""
    names = sorted({n for n, _ in ops})
    res = {}
    for name in names:
        sel = [f for n, f in ops if n == name]
        g = capture(torch, sel, reps)
        stream = torch.cuda.current_stream()
        per = []
        for _ in range(replays):
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record(stream)
            g.replay()
            e1.record(stream)
            e1.synchronize()
            per.append(e0.elapsed_time(e1) / 1e3 / (reps * len(sel)))
        per.sort()
        res[name] = (per[len(per) // 2], per[0], per[-1])
        del g
    return res


# Epilogue of the kernel serving each op (the name rocprofv3 records).
OP_EPILOGUE = {"gate_up": "EpiGateUp", "qkv": "EpiQkv", "lm_head": "EpiArgmax"}


def measured_traffic(op, m):
    """HBM bytes per launch of `op` from the committed counter profile of this
    benchmark (FETCH_SIZE and WRITE_SIZE runs, each scaled by what the counter
    reads for a plain copy of known size), or None when no profile covers it."""
    path = os.path.join(ROOT, "profiles", f"decode_gemm_set_m{m}_traffic.json")
    epi = OP_EPILOGUE.get(op)
    if not epi or not os.path.exists(path):
        return None
    with open(path) as f:
        prof = json.load(f)
    hits = [v["hbm_bytes"] for k, v in prof["kernels"].items() if epi in k]
    return int(hits[0]) if len(hits) == 1 else None


def short_kernel(name):
    """Kernel name without namespaces, argument list or a leading `void`."""
    import re

    name = name.replace("stride_tc::", "")
    name = re.sub(r"\(Geometry.*$", "", name)
    return re.sub(r"^void ", "", name)[:140]


def summarize_trace(path):
    """calls / average / min / max / total duration (us) per kernel of a rocprofv3
    kernel trace, largest total first."""
    import csv
    from collections import defaultdict

    rows = defaultdict(list)
    with open(path) as f:
        for r in csv.DictReader(f):
            rows[short_kernel(r["Kernel_Name"])].append((int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1e3)
    lines = [f"{'kernel':<90} {'calls':>6} {'avg_us':>9} {'min_us':>9} {'max_us':>9} {'total_us':>11}"]
    for n, d in sorted(rows.items(), key=lambda kv: -sum(kv[1])):
        lines.append(f"{n[:90]:<90} {len(d):>6} {sum(d) / len(d):>9.2f} {min(d):>9.2f} {max(d):>9.2f} {sum(d):>11.1f}")
    return "\n".join(lines)


def summarize_counters(path):
    """Average value per dispatch of each counter, per kernel (FETCH_SIZE and
    WRITE_SIZE in KiB), from a rocprofv3 counter collection."""
    import csv
    from collections import defaultdict

    vals = defaultdict(lambda: defaultdict(float))
    disp = defaultdict(lambda: defaultdict(set))
    with open(path) as f:
        for r in csv.DictReader(f):
            n = short_kernel(r["Kernel_Name"])
            vals[n][r["Counter_Name"]] += float(r["Counter_Value"])
            disp[n][r["Counter_Name"]].add(r["Dispatch_Id"])
    lines = [f"{'kernel':<90} {'counter':>28} {'dispatches':>10} {'avg_per_dispatch':>18}"]
    for n in sorted(vals):
        for c in sorted(vals[n]):
            k = len(disp[n][c])
            lines.append(f"{n[:90]:<90} {c:>28} {k:>10} {vals[n][c] / k:>18.1f}")
    return "\n".join(lines)


def traffic_from(fetch_csv, write_csv, calib_bytes=512 << 20):
    """HBM bytes per launch by kernel: FETCH_SIZE and WRITE_SIZE (KiB per
    dispatch, averaged over dispatches), each scaled by what the counter reads
    for the plain copy (torch neg) of calib_bytes each way in the same run."""
    import csv
    from collections import defaultdict

    def per_dispatch(path, counter):
        vals, disp = defaultdict(float), defaultdict(set)
        with open(path) as f:
            for r in csv.DictReader(f):
                if r["Counter_Name"] == counter:
                    n = short_kernel(r["Kernel_Name"])
                    vals[n] += float(r["Counter_Value"])
                    disp[n].add(r["Dispatch_Id"])
        return {n: vals[n] / len(disp[n]) for n in vals}

    fetch, write = per_dispatch(fetch_csv, "FETCH_SIZE"), per_dispatch(write_csv, "WRITE_SIZE")
    cal = [n for n in fetch if "neg_kernel" in n]
    if len(cal) != 1 or cal[0] not in write:
        raise SystemExit(f"bench.py: need exactly one calibration copy kernel in both runs, found {cal}")
    fs, ws = calib_bytes / (fetch[cal[0]] * 1024.0), calib_bytes / (write[cal[0]] * 1024.0)
    out = {"source": "rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE --kernel-trace, one run each",
           "calibration": {"kernel": cal[0], "bytes_each_way": calib_bytes, "fetch_scale": round(fs, 4),
                           "write_scale": round(ws, 4)},
           "kernels": {}}
    for n in sorted(fetch):
        if n != cal[0] and n in write and n.startswith("k_"):
            fb, wb = fetch[n] * 1024.0 * fs, write[n] * 1024.0 * ws
            out["kernels"][n] = {"fetch_bytes": int(fb), "write_bytes": int(wb), "hbm_bytes": int(fb + wb)}
    return out


def host_info():
    """Host cores (as os.cpu_count() reports them), the cores this process may run
    on, and the CPU model string."""
    model = ""
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    return {"host_cores": os.cpu_count(), "affinity_cores": len(os.sched_getaffinity(0)), "cpu_model": model}


def cpu_threads_default():
    """Threads for the CPU baseline: every core this process may use, capped at
    the 16-core share a one-GPU job is given on the GPU hosts (OMP_NUM_THREADS
    there holds that share)."""
    share = int(os.environ.get("OMP_NUM_THREADS", "0") or 0) or 16
    return max(1, min(len(os.sched_getaffinity(0)), share))


def cpu_baseline(seconds, threads, batches=(128, 1), prefill=(290, 1024)):
    """The reference's exact path (oracle/_ref: its src/kernels.cu compiled as C++)
    on this host: one decode step's GEMM set at each batch in `batches`, sampled
    as one layer's QKV, O, gate+up and down GEMMs plus the LM head (the config-2
    and config-3 shapes), with the layer time scaled to 16 layers; the same five
    GEMMs once each at the prefill row counts in `prefill` (config 4); and config 1
    (one projection, M = 1, N = K = 2048). `value` is the first batch's (the
    benchmark's M = 128) tok/s."""
    import ctypes as C

    import numpy as np

    os.environ.setdefault("STRIDE_CPU_THREADS", str(threads))
    from oracle import oracle as orc

    kind = "reference" if orc.ref_available() else "port"
    rng = np.random.default_rng(0)

    def wts(n, k):
        return (rng.standard_normal((n, k), dtype=np.float32) * 0.02).view(np.uint32).__rshift__(16).astype(np.uint16)

    dims = [("qkv", 3072, HIDDEN), ("o", HIDDEN, HIDDEN), ("gate_up", 2 * FFN, HIDDEN), ("down", HIDDEN, FFN),
            ("lm_head", VOCAB, HIDDEN)]
    lib = None
    if kind == "reference":
        lib = C.CDLL(orc.REF_PATH)
        lib.ref_bench_gemm.restype = C.c_double
        lib.ref_bench_gemm.argtypes = [np.ctypeslib.ndpointer(np.uint16, flags="C_CONTIGUOUS"), C.c_int, C.c_int,
                                       np.ctypeslib.ndpointer(np.float32, flags="C_CONTIGUOUS"), C.c_int, C.c_int]
    else:
        ex = orc.Exact(threads=threads)
    res = {}
    budget = seconds / (len(dims) * len(batches))
    for name, n, k in dims:
        w = wts(n, k)
        for m in batches:
            x = rng.standard_normal((m, k), dtype=np.float32)
            if lib is not None:
                one = lib.ref_bench_gemm(w, n, k, x, m, 1)
                reps = max(1, min(50, int(budget / max(one, 1e-6))))
                sec = lib.ref_bench_gemm(w, n, k, x, m, reps) / reps if reps > 1 else one
            else:
                t0 = time.perf_counter()
                ex.gemm(w, x)
                sec = time.perf_counter() - t0
            res.setdefault(m, {})[name] = sec
        del w
    per_batch = {}
    for m in batches:
        t = res[m]
        step = LAYERS * (t["qkv"] + t["o"] + t["gate_up"] + t["down"]) + t["lm_head"]
        per_batch[m] = {
            "tok_s": round(m / step, 3), "seconds_per_step": round(step, 4),
            "per_gemm_ms": {k: round(v * 1e3, 3) for k, v in t.items()},
            "per_gemm_GB/s": {nm: round((2 * n * k + 4 * m * (k + n)) / t[nm] / 1e9, 2) for nm, n, k in dims},
            "per_gemm_GFLOP/s": {nm: round(2 * m * n * k / t[nm] / 1e9, 2) for nm, n, k in dims}}
    def once(w, n, k, m):
        x = rng.standard_normal((m, k), dtype=np.float32)
        if lib is not None:
            return lib.ref_bench_gemm(w, n, k, x, m, 1)
        t0 = time.perf_counter()
        ex.gemm(w, x)
        return time.perf_counter() - t0

    w1 = wts(HIDDEN, HIDDEN)
    sec1 = min(once(w1, HIDDEN, HIDDEN, 1) for _ in range(5))
    config1 = {"M": 1, "N": HIDDEN, "K": HIDDEN, "ms": round(sec1 * 1e3, 4),
               "GB/s": round((2 * HIDDEN * HIDDEN + 4 * (2 * HIDDEN)) / sec1 / 1e9, 2),
               "GFLOP/s": round(2 * HIDDEN * HIDDEN / sec1 / 1e9, 2), "repetitions": 5, "statistic": "min"}
    pre = {}
    for name, n, k in dims:
        w = wts(n, k)
        for m in prefill:
            sec = once(w, n, k, m)
            pre.setdefault(str(m), {})[name] = {"ms": round(sec * 1e3, 2),
                                                "GFLOP/s": round(2 * m * n * k / sec / 1e9, 1)}
        del w
    m0 = batches[0]
    out = {"value": per_batch[m0]["tok_s"], "unit": "tok/s", "cores": threads, "kind": kind,
           "sample": f"exact path (k_lm_full order, all fmaf chains) at batch {m0}: one layer's QKV/O/gate+up/down "
                     "GEMMs + the LM head timed, layer time x16 + LM head; STRIDE_CPU_THREADS="
                     f"{threads}", "seconds_per_step": per_batch[m0]["seconds_per_step"]}
    out.update(host_info())
    out["batches"] = {str(m): v for m, v in per_batch.items()}
    out["config1"] = config1
    out["prefill"] = {"repetitions": 1, "per_gemm": pre}
    return out


def cpu_baseline_single_core(seconds):
    """The same sample on one core at batch 1. The reference's thread pool reads
    its size once per process, so this runs in a child process with
    STRIDE_CPU_THREADS=1."""
    import subprocess

    env = dict(os.environ, STRIDE_CPU_THREADS="1")
    code = f"import json, bench; print(json.dumps(bench.cpu_baseline({seconds!r}, 1, (1,), ())))"
    try:
        r = subprocess.run([sys.executable, "-c", code], cwd=ROOT, env=env, capture_output=True, text=True,
                           timeout=120 + 4 * seconds)
    except subprocess.TimeoutExpired:
        return None
    if r.returncode != 0 or not r.stdout.strip():
        return None
    one = json.loads(r.stdout.strip().splitlines()[-1])
    return {k: one[k] for k in ("value", "unit", "cores", "seconds_per_step", "batches")}


def engine_step(torch, dev, m, steps, warmup, position=383):
    """The full greedy decode step at batch m: the whole step of
    stride_amd.engine (embedding, per layer RMSNorm, QKV + RoPE + KV append,
    paged attention over `position` + 1 positions, O, RMSNorm, gate/up, down;
    final RMSNorm and the greedy LM head), every row at `position` (the middle of
    a 256-token prompt + 256-token generation), captured as one HIP graph and
    replayed. Random-init weights; KV contents do not change the work."""
    from stride_amd import engine

    w = engine.Weights(engine.LlamaConfig(), dev, seed=1, max_positions=512)
    eng = engine.Engine(w, slots=m, max_ctx=512, max_rows=m, page_tokens=16, shuffle_seed=3)
    rows = [(j, position, (j * 7919) % w.cfg.vocab) for j in range(m)]
    slot, pos, tok, items = eng.device_rows(rows)
    best = torch.empty((m, 2), dtype=torch.int32, device=dev)
    g = capture(torch, [lambda: eng.launch(m, slot, pos, tok, items, best=best)])
    for _ in range(warmup):
        g.replay()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        g.replay()
    torch.cuda.synchronize()
    dt = time.perf_counter() - t0
    del g, eng, w
    torch.cuda.empty_cache()
    return {"batch": m, "position": position, "page_tokens": 16, "ms_per_step": round(dt / steps * 1e3, 4),
            "tok_s": round(m * steps / dt, 1), "launch": "HIP graph of one full step, replayed",
            "ops": "tc_embed, 16 x (tc_norm, tc_qkv, tc_attention, tc_gemm_residual, tc_norm, tc_mlp13, "
                   "tc_gemm_residual), tc_norm, tc_lm_greedy"}


def exact_step(torch, batches=(1, 32), steps=5):
    """The exact FP32 path end to end on the GPU (stride_amd.exact_engine over the
    stride_k_* kernels, bit-identical to the reference's CPU exact path): one greedy
    decode step of random-init Llama-3.2-1B (bf16 weights widened to fp32 in the
    kernels, 2.47 GB read per step), every row at position 100: host-launched from
    Python with the rows' upload and the argmax read-back (ms_per_step), and the
    device part of the same step (its ~130 launches and the argmax re-arm) as one
    HIP graph, replayed (graph_ms_per_step)."""
    from stride_amd import exact_engine as E
    from stride_amd.weights import ModelConfig

    cfg = ModelConfig()
    model = E.ExactModel.random(cfg, seed=7, max_positions=512)
    be = E.GpuBackend("cuda:0")
    out = {}
    for m in batches:
        eng = E.ExactEngine(model, be, slots=m, max_ctx=512, max_rows=m)
        rows = [(j, 100, 7 + j) for j in range(m)]
        eng.step(rows, greedy=list(range(m)))
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(steps):
            eng.step(rows, greedy=list(range(m)))
        torch.cuda.synchronize()
        dt = (time.perf_counter() - t0) / steps
        items = eng.upload(rows)
        best = eng.best.view(-1, 2)[:m]

        def device_step():
            best[:, 0].fill_(-8388608)  # 0xFF800000: -inf
            best[:, 1].fill_(-1)
            eng.launch_layers(m, items)
            eng.launch_lm_greedy_all(m)

        g = capture(torch, [device_step])
        for _ in range(2):
            g.replay()
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(steps * 4):
            g.replay()
        torch.cuda.synchronize()
        dg = (time.perf_counter() - t0) / (steps * 4)
        out[str(m)] = {"ms_per_step": round(dt * 1e3, 3), "tok_s": round(m / dt, 1),
                       "graph_ms_per_step": round(dg * 1e3, 3), "graph_tok_s": round(m / dg, 1)}
        del g, eng
    return out


def library_gemm(torch, dev, ms=(128, 2048, 4096)):
    """Context for both rooflines: the vendor library (torch.matmul, which calls
    hipBLASLt) on the same shapes in bf16 (gate+up as one 16384-row matmul, no
    SiLU), weights rotated past the MALL (at least ROTATION_BYTES per pass, as
    the per-op table), HIP-graph timing. It has no batch-invariance contract and
    no fused epilogue, so it is a reference point, not a parity target."""
    res = {}
    shapes = {"qkv": (3072, HIDDEN), "o": (HIDDEN, HIDDEN), "gate_up": (2 * FFN, HIDDEN), "down": (HIDDEN, FFN),
              "lm_head": (VOCAB, HIDDEN)}
    for m in ms:
        row = {}
        for name, (n, k) in shapes.items():
            a = torch.randn(m, k, device=dev, dtype=torch.bfloat16)
            copies = max(2, -(-ROTATION_BYTES // (2 * n * k)))
            ws = [torch.randn(n, k, device=dev, dtype=torch.bfloat16) for _ in range(copies)]
            g = capture(torch, [lambda w=w: torch.matmul(a, w.t()) for w in ws])
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record()
            g.replay()
            g.replay()
            e1.record()
            e1.synchronize()
            sec = e0.elapsed_time(e1) / 1e3 / (2 * len(ws))
            f, byt = 2.0 * m * n * k, 2.0 * n * k + 2.0 * m * k + 2.0 * m * n
            gbs, tfl = byt / sec / 1e9, f / sec / 1e12
            frac = gbs / HBM_PEAK_GBS if m <= 128 else tfl / MFMA_BF16_PEAK_TFLOPS
            row[name] = {"us": round(sec * 1e6, 2), "GB/s": round(gbs, 1), "TFLOP/s": round(tfl, 1),
                         "frac": round(frac, 4), "bound": "hbm" if m <= 128 else "mfma"}
            del g, ws, a
            torch.cuda.empty_cache()
        res[str(m)] = row
    return res


def main():
    a = parse()
    if a.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py: this build runs on one GPU only (the GEMM path has no multi-GPU part); "
              "use --gpus 1", file=sys.stderr)
        sys.exit(2)
    import torch

    from stride_amd import _lib

    if a.summarize_trace:
        print(summarize_trace(a.summarize_trace))
        return
    if a.summarize_counters:
        print(summarize_counters(a.summarize_counters))
        return
    if a.traffic_from:
        fetch_csv, write_csv = a.traffic_from.split(",")
        print(json.dumps(traffic_from(fetch_csv, write_csv), indent=1))
        return
    _lib.load()  # fail loudly without the HIP library
    dev = "cuda:0"
    torch.cuda.set_device(0)
    if a.exact_step:
        print(json.dumps({"exact_decode_step": exact_step(torch)}), flush=True)
        return
    if a.engine_only:
        print(json.dumps({"full_decode_step": engine_step(torch, dev, a.m, a.steps, a.warmup)}), flush=True)
        return
    if a.copy_calib_mib:
        src = torch.ones(a.copy_calib_mib << 18, dtype=torch.float32, device=dev)
        dst = torch.empty_like(src)
        torch.neg(src, out=dst)  # a plain streaming kernel: reads and writes exactly N bytes
        torch.cuda.synchronize()
        del src, dst

    model = Model(torch, dev)
    b = Buffers(torch, dev, a.m)
    ops = step_ops(model, b)
    if a.op:
        if a.op not in OP_WEIGHTS:
            print(f"bench.py: unknown --op {a.op}", file=sys.stderr)
            sys.exit(2)
        sel = rotated_ops(model, b, [a.op])
        sec, lo, hi = time_ops(torch, sel, max(1, a.steps // len(sel)))[a.op]
        f, byt = work(a.op, a.m)
        print(json.dumps({"op": a.op, "M": a.m, "us": round(sec * 1e6, 2), "spread_us": [round(lo * 1e6, 2), round(hi * 1e6, 2)],
                          "GB/s": round(byt / sec / 1e9, 1), "TFLOP/s": round(f / sec / 1e12, 1)}), flush=True)
        return

    from stride_amd import harness

    step = [f for _, f in ops]

    if a.step_only:
        for _ in range(a.warmup):
            for f in step:
                f()
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(a.steps):
            for f in step:
                f()
        torch.cuda.synchronize()
        dt = time.perf_counter() - t0
        print(json.dumps({"step_only": True, "M": a.m, "steps": a.steps, "ms_per_step": round(dt / a.steps * 1e3, 4)}),
              flush=True)
        return

    # The measured path: K decode steps launched from the host on one stream, the
    # way the reference's engine launches its kernels (no graph), bracketed by
    # device synchronizations. The same step captured once as a HIP graph and
    # replayed is timed beside it: on this ROCm the graph's kernels each run a few
    # percent slower (same kernels, same bits; see the design notes).
    for _ in range(a.warmup):
        for f in step:
            f()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(a.steps):
        for f in step:
            f()
    torch.cuda.synchronize()
    dt = time.perf_counter() - t0
    ms_step = dt / a.steps * 1e3
    value = a.m * a.steps / dt

    graph = capture(torch, step)
    for _ in range(a.warmup):
        graph.replay()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(a.steps):
        graph.replay()
    torch.cuda.synchronize()
    graph_ms = (time.perf_counter() - t0) / a.steps * 1e3
    del graph

    # Per-kernel times at the bench M (dominant kernel -> roofline object): the
    # median over graph replays, with the fastest and slowest replay beside it.
    spread = time_ops(torch, rotated_ops(model, b, list(OP_WEIGHTS)), 3)
    per = {n: v[0] for n, v in spread.items()}
    share = {n: per[n] * sum(1 for o, _ in ops if o == n) for n in per}
    dom = max(share, key=share.get)
    fl, by = work(dom, a.m)
    ach = by / per[dom] / 1e9
    roof = {"kernel": dom, "bound": "hbm", "achieved": round(ach, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
            "frac": round(ach / HBM_PEAK_GBS, 4), "traffic": measured_traffic(dom, a.m),
            "avg_launch_us": round(per[dom] * 1e6, 2),
            "launch_us_spread": [round(spread[dom][1] * 1e6, 2), round(spread[dom][2] * 1e6, 2)],
            "algorithmic_bytes": int(by), "rotated_bytes": rotated_bytes(model, dom)}
    weight_bytes = sum(work(n, 0)[1] for n, _ in ops)

    table = []
    if a.table:
        for m in (1, 8, 32, 64, 128, 290, 1024, 2048, 4096):
            bm = b if m == a.m else Buffers(torch, dev, m)
            t = time_ops(torch, rotated_ops(model, bm, list(OP_WEIGHTS)), 2 if m >= 1024 else 3)
            row = {"M": m}
            for n, (sec, lo, hi) in sorted(t.items()):
                f, byt = work(n, m)
                gbs, tfl = byt / sec / 1e9, f / sec / 1e12
                bound = "hbm" if m <= 128 else "mfma"
                frac = gbs / HBM_PEAK_GBS if bound == "hbm" else tfl / MFMA_BF16_PEAK_TFLOPS
                row[n] = {"us": round(sec * 1e6, 2), "spread_us": [round(lo * 1e6, 2), round(hi * 1e6, 2)],
                          "GB/s": round(gbs, 1), "TFLOP/s": round(tfl, 2), "frac": round(frac, 4), "bound": bound,
                          "rotated_bytes": rotated_bytes(model, n)}
            table.append(row)
            del bm
            torch.cuda.empty_cache()

    full = engine_step(torch, dev, a.m, a.steps, a.warmup) if a.engine else None
    library = library_gemm(torch, dev) if a.library else None
    if library:
        for row in table:  # vendor time / our time, same shape and M
            lib = library.get(str(row["M"]))
            if lib:
                for n, v in row.items():
                    if n in lib:
                        v["library_us"] = lib[n]["us"]
                        v["speedup_vs_library"] = round(lib[n]["us"] / v["us"], 3)
    threads = a.cpu_threads or cpu_threads_default()
    cpu = cpu_baseline(a.cpu_seconds, threads) if a.cpu_seconds > 0 else None
    if cpu is not None and threads != 1:
        cpu["single_core"] = cpu_baseline_single_core(a.cpu_seconds / 2)
    out = {
        "metric": "Llama-3.2-1B GEMM GB/s & TFLOP/s (% roofline) at M=1..4096; decode tok/s",
        "value": round(value, 1), "unit": "tok/s", "n_gpus": 1, "steps": a.steps, "warmup": a.warmup,
        "ms_per_step": round(ms_step, 4), "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "bf16", "data": "synthetic (random-init bf16 weights ~N(0,0.02), activations ~N(0,1))",
        "config": {"workload": f"decode-step GEMM set, Llama-3.2-1B shapes, 16 layers + LM head greedy, M={a.m}",
                   "M": a.m, "layers": LAYERS, "weight_bytes_per_step": int(weight_bytes),
                   "step_GB/s": round(weight_bytes / (ms_step / 1e3) / 1e9, 1), "parallelism": "single-gpu",
                   "launch": "host-launched on one stream (as the reference engine launches)",
                   "graph_ms_per_step": round(graph_ms, 4)},
        "roofline": roof, "cpu_baseline": cpu, "full_decode_step": full, "gemm_table": table,
        "library_gemm": library,
    }
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
