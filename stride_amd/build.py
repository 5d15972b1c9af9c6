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
# (source, object name, extra flags): the entry points, then each epilogue's
# configuration table of each kernel family in an object of its own.
UNITS = [(s, os.path.basename(s) + ".o", []) for s in SOURCES] + [
    (os.path.join(CSRC, "tc_gemm_inst.hip"), f"inst_{epi}_{fam}.o", [f"-DSTRIDE_TC_EPI={epi}", f"-DSTRIDE_TC_FAMILY={fam}"])
    for epi in ("EpiResidual", "EpiLogits", "EpiGateUp", "EpiArgmax", "EpiQkv") for fam in (0, 1, 2)]
OUT = os.path.join(HERE, "libstride_tc.so")
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


def _link(out: str, units, verbose: bool, incremental: bool) -> None:
    os.makedirs(OBJ, exist_ok=True)
    objs = [os.path.join(OBJ, name) for _, name, _ in units]

    def compile_one(unit_obj):
        (src, _, extra), obj = unit_obj
        if incremental and os.path.exists(obj) and os.path.getmtime(obj) > _deps_mtime(src):
            return
        _run([HIPCC, *FLAGS, *extra, "-c", "-o", obj, src], os.path.basename(obj), verbose)

    workers = max(1, min(len(units), os.cpu_count() or 1))
    with ThreadPoolExecutor(max_workers=workers) as ex:
        list(ex.map(compile_one, zip(units, objs)))
    _run([HIPCC, "--offload-arch=gfx950", "-shared", "-fPIC", "-o", out, *objs], os.path.basename(out), verbose)


def build(verbose: bool = False, incremental: bool = False) -> str:
    """Builds libstride_tc.so (the GEMM library)."""
    _link(OUT, UNITS, verbose, incremental)
    return OUT


if __name__ == "__main__":
    print(build(verbose=True, incremental="--incremental" in sys.argv))
