"""Builds tests/kat/libmfma_kat.so (the MFMA known-answer kernels the GPU tests
use; test infrastructure, not part of the product) with the library's flags."""
from __future__ import annotations

import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
SRC = os.path.join(HERE, "mfma_kat.hip")
OUT = os.path.join(HERE, "libmfma_kat.so")


def build(verbose: bool = False) -> str:
    sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))
    from stride_amd.build import FLAGS, HIPCC

    cmd = [HIPCC, *FLAGS, "-shared", "-o", OUT, SRC]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        sys.stderr.write(res.stdout + res.stderr)
        raise RuntimeError("hipcc failed building libmfma_kat.so")
    if verbose:
        print(" ".join(cmd))
    return OUT


if __name__ == "__main__":
    print(build(verbose=True))
