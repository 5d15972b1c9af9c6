"""Builds libstride_tc.so in-tree for gfx950 with hipcc (no JIT cache).

Flags: -ffp-contract=off so that no a*b+c in the epilogues is fused on the
compiler's initiative (every kernel variant must produce the same bits), and the
packed-fp32 feature switched off for the device code.

Each source is compiled to its own object in parallel, then linked.
``python -m stride_amd.build --incremental`` skips objects newer than every
source and header (a development shortcut; build() always recompiles).
"""
from __future__ import annotations

import glob
import os
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
OBJ = os.path.join(HERE, "_obj")
SOURCES = [os.path.join(CSRC, f) for f in ("tc_gemm.hip", "tc_gemm_mlp13.hip", "tc_gemm_qkv.hip", "tc_gemm_lm_full.hip",
                                            "tc_gemm_lm_greedy.hip", "tc_aux.hip", "exact.hip")]
OUT = os.path.join(HERE, "libstride_tc.so")
PROBE_SOURCES = [os.path.join(CSRC, "probe.hip")]
PROBE_OUT = os.path.join(HERE, "libstride_probe.so")
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
FLAGS = [
    "-O3", "--offload-arch=gfx950", "-std=c++17", "-fPIC",
    "-ffp-contract=off", "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
]


def _run(cmd, what: str, verbose: bool) -> None:
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        sys.stderr.write(res.stdout + res.stderr)
        raise RuntimeError(f"hipcc failed building {what}")
    if verbose:
        print(" ".join(cmd))


def _deps_mtime(src: str) -> float:
    """Newest of the source, the shared headers and the public C headers."""
    files = [src] + glob.glob(os.path.join(CSRC, "*.hpp")) + glob.glob(os.path.join(os.path.dirname(HERE), "include", "*.h"))
    return max(os.path.getmtime(f) for f in files)


def _link(out: str, sources, verbose: bool, incremental: bool) -> None:
    os.makedirs(OBJ, exist_ok=True)
    objs = [os.path.join(OBJ, os.path.basename(s) + ".o") for s in sources]
    def compile_one(src_obj):
        src, obj = src_obj
        if incremental and os.path.exists(obj) and os.path.getmtime(obj) > _deps_mtime(src):
            return
        _run([HIPCC, *FLAGS, "-c", "-o", obj, src], os.path.basename(src), verbose)

    with ThreadPoolExecutor(max_workers=len(sources)) as ex:
        list(ex.map(compile_one, zip(sources, objs)))
    _run([HIPCC, "--offload-arch=gfx950", "-shared", "-fPIC", "-o", out, *objs], os.path.basename(out), verbose)


def build(verbose: bool = False, incremental: bool = False) -> str:
    """Builds libstride_tc.so (the GEMM library) and libstride_probe.so (the
    methodology probes)."""
    _link(OUT, SOURCES, verbose, incremental)
    _link(PROBE_OUT, PROBE_SOURCES, verbose, incremental)
    return OUT


if __name__ == "__main__":
    print(build(verbose=True, incremental="--incremental" in sys.argv))
