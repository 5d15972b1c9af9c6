"""Builds libstride_tc.so in-tree for gfx950 with hipcc (no JIT cache).

Flags: -ffp-contract=off so that no a*b+c in the epilogues is fused on the
compiler's initiative (every kernel variant must produce the same bits), and the
packed-fp32 feature switched off for the device code.
"""
from __future__ import annotations

import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
SOURCES = [os.path.join(HERE, "csrc", "tc_gemm.hip"), os.path.join(HERE, "csrc", "tc_aux.hip")]
OUT = os.path.join(HERE, "libstride_tc.so")
PROBE_SOURCES = [os.path.join(HERE, "csrc", "probe.hip")]
PROBE_OUT = os.path.join(HERE, "libstride_probe.so")
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
FLAGS = [
    "-O3", "--offload-arch=gfx950", "-std=c++17", "-shared", "-fPIC",
    "-ffp-contract=off", "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
]


def _hipcc(out: str, sources, verbose: bool) -> None:
    cmd = [HIPCC, *FLAGS, "-o", out, *sources]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        sys.stderr.write(res.stdout + res.stderr)
        raise RuntimeError(f"hipcc failed building {os.path.basename(out)}")
    if verbose:
        print(" ".join(cmd))


def build(verbose: bool = False) -> str:
    """Builds libstride_tc.so (the GEMM library) and libstride_probe.so (the
    methodology probes)."""
    _hipcc(OUT, SOURCES, verbose)
    _hipcc(PROBE_OUT, PROBE_SOURCES, verbose)
    return OUT


if __name__ == "__main__":
    print(build(verbose=True))
