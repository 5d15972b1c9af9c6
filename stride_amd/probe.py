"""ctypes binding of libstride_probe.so (include/stride_probe.h): the MFMA
position-invariance probe and the HBM read-throughput probe."""
from __future__ import annotations

import ctypes as C
import os

HERE = os.path.dirname(os.path.abspath(__file__))
PATH = os.path.join(HERE, "libstride_probe.so")
_lib = None


def load():
    global _lib
    if _lib is None:
        if not os.path.exists(PATH):
            raise ImportError(f"{PATH} not built (python -m stride_amd.build)")
        lib = C.CDLL(PATH)
        vp = C.c_void_p
        lib.stride_probe_mfma_tiles.argtypes = [vp, vp, vp, vp, C.c_int32, vp]
        lib.stride_probe_mfma_tiles.restype = C.c_int
        lib.stride_probe_read.argtypes = [vp, C.c_int64, vp, C.c_int32, C.c_int32, vp]
        lib.stride_probe_read.restype = C.c_int
        lib.stride_probe_mfma_rate.argtypes = [vp, C.c_int32, C.c_int32, vp]
        lib.stride_probe_mfma_rate.restype = C.c_int
        lib.stride_probe_mfma_rate_variant.argtypes = [vp, C.c_int32, C.c_int32, C.c_int32, vp]
        lib.stride_probe_mfma_rate_variant.restype = C.c_int
        lib.stride_probe_mfma_equiv.argtypes = [vp, vp, vp, vp, vp, C.c_int32, C.c_int32, vp]
        lib.stride_probe_mfma_equiv.restype = C.c_int
        lib.stride_probe_strip_read.argtypes = [vp, C.c_int64, C.c_int64, C.c_int32, C.c_int32, C.c_int32, vp, vp]
        lib.stride_probe_strip_read.restype = C.c_int
        lib.stride_probe_decode_ceiling.argtypes = [vp, C.c_int32, C.c_int32, vp, C.c_int32, C.c_int32, vp, vp]
        lib.stride_probe_decode_ceiling.restype = C.c_int
        _lib = lib
    return _lib


def mfma_tiles(a, b, c, out, stream: int) -> None:
    rc = load().stride_probe_mfma_tiles(a.data_ptr(), b.data_ptr(), c.data_ptr(), out.data_ptr(), a.shape[0], stream)
    if rc:
        raise RuntimeError(f"stride_probe_mfma_tiles failed ({rc})")


def read(buf, out, blocks: int, unroll: int, stream: int) -> None:
    rc = load().stride_probe_read(buf.data_ptr(), buf.numel() * buf.element_size(), out.data_ptr(), blocks, unroll,
                                  stream)
    if rc:
        raise RuntimeError(f"stride_probe_read failed ({rc})")


def strip_read(buf, strip: int, out, blocks: int, unroll: int, rotate: int, stream: int) -> None:
    rc = load().stride_probe_strip_read(buf.data_ptr(), buf.numel() * buf.element_size(), strip, blocks, unroll,
                                        rotate, out.data_ptr(), stream)
    if rc:
        raise RuntimeError(f"stride_probe_strip_read failed ({rc})")


def mfma_rate(out, blocks: int, iters: int, stream: int) -> None:
    rc = load().stride_probe_mfma_rate(out.data_ptr(), blocks, iters, stream)
    if rc:
        raise RuntimeError(f"stride_probe_mfma_rate failed ({rc})")


def mfma_rate_variant(out, blocks: int, iters: int, variant: int, stream: int) -> None:
    rc = load().stride_probe_mfma_rate_variant(out.data_ptr(), blocks, iters, variant, stream)
    if rc:
        raise RuntimeError(f"stride_probe_mfma_rate_variant failed ({rc})")


def mfma_equiv(a, b, c0, o16, o32, chunks: int, stream: int) -> None:
    rc = load().stride_probe_mfma_equiv(a.data_ptr(), b.data_ptr(), c0.data_ptr(), o16.data_ptr(), o32.data_ptr(),
                                        c0.shape[0], chunks, stream)
    if rc:
        raise RuntimeError(f"stride_probe_mfma_equiv failed ({rc})")


def decode_ceiling(w, row_tiles: int, chunks: int, x, lane_tiles: int, mode: int, out, stream: int) -> None:
    rc = load().stride_probe_decode_ceiling(w.data_ptr(), row_tiles, chunks, x.data_ptr(), lane_tiles, mode,
                                            out.data_ptr(), stream)
    if rc:
        raise RuntimeError(f"stride_probe_decode_ceiling failed ({rc})")


def _graph_time(torch, fns, side):
    """Average seconds per call of fns (captured once in a HIP graph, replayed twice)."""
    g = torch.cuda.CUDAGraph()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for f in fns:
            f()
    torch.cuda.current_stream().wait_stream(side)
    with torch.cuda.graph(g):
        for f in fns:
            f()
    g.replay()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    g.replay()
    g.replay()
    e1.record()
    e1.synchronize()
    return e0.elapsed_time(e1) / 1e3 / (2 * len(fns))


def main(argv=None) -> None:
    """python -m stride_amd.probe [read] [strip] [mfma] [ceiling]: the floors the GEMM
    kernels are judged against, as markdown table rows. Buffers rotate over up to
    16 distinct copies in a 3 GiB pool, so the 256 MB MALL cannot serve repeats."""
    import sys

    import torch

    what = set((argv if argv is not None else sys.argv[1:]) or ["read", "strip", "mfma"])
    dev = "cuda:0"
    side = torch.cuda.Stream()
    out = torch.zeros(1 << 20, dtype=torch.int32, device=dev)
    stream = lambda: torch.cuda.current_stream().cuda_stream
    if what & {"read", "strip"}:
        pool = torch.empty(3 << 30, dtype=torch.uint8, device=dev).fill_(1)
    if "read" in what:
        print("| bytes | best time | GB/s | grid | loads in flight |\n|---|---|---|---|---|", flush=True)
        for mib in (8, 12, 32, 64, 128, 512):
            nb = mib << 20
            views = [pool[i * nb:(i + 1) * nb] for i in range(min(16, (3 << 30) // nb))]
            best = None
            for blocks in (256, 512, 1024, 2048, 4096, 0):
                for unroll in (4, 8, 16):
                    s = _graph_time(torch, [lambda v=v: read(v, out, blocks, unroll, stream()) for v in views], side)
                    if best is None or s < best[0]:
                        best = (s, blocks, unroll)
            grid = "1 WG / 64 KiB" if best[1] == 0 else str(best[1])
            print(f"| {mib} MiB | {best[0] * 1e6:.2f} us | {nb / best[0] / 1e9:.0f} | {grid} | {best[2]} |", flush=True)
    if "strip" in what:
        print("| bytes | strip | rotated starts | best time | GB/s |\n|---|---|---|---|---|", flush=True)
        for mib in (64, 512):
            nb = mib << 20
            views = [pool[i * nb:(i + 1) * nb] for i in range(min(16, (3 << 30) // nb))]
            for strip in (32768, 65536):
                for rot in (0, 1):
                    best = min(_graph_time(torch, [lambda v=v: strip_read(v, strip, out, blocks, unroll, rot, stream())
                                                   for v in views], side)
                               for blocks in (256, 512, 1024) for unroll in (8, 16))
                    print(f"| {mib} MiB | {strip // 1024} KiB | {'yes' if rot else 'no'} | {best * 1e6:.2f} us | "
                          f"{nb / best / 1e9:.0f} |", flush=True)
    if "ceiling" in what:
        # The gate/up shape at M = 64 and 128: 1024 strips of 64 chunks (64 MiB),
        # 16 copies rotated (1 GiB).
        print("| lane tiles (M) | activation fragments | time | GB/s of weights |\n|---|---|---|---|", flush=True)
        rt, ch = 1024, 64
        nb = rt * ch * 1024
        wpool = torch.empty(16 * nb, dtype=torch.uint8, device=dev).fill_(0x3c)
        xb = torch.empty(8 * ch * 1024, dtype=torch.uint8, device=dev).fill_(0x3c)
        fo = torch.zeros(rt * 64 * 4, dtype=torch.float32, device=dev)
        views = [wpool[i * nb:(i + 1) * nb] for i in range(16)]
        for lt in (4, 8):
            for mode, label in ((0, "registers (no LDS)"), (1, "static LDS slab"), (2, "LDS ring refilled by a copy wave")):
                s = _graph_time(torch, [lambda v=v: decode_ceiling(v, rt, ch, xb, lt, mode, fo, stream()) for v in views],
                                side)
                print(f"| {lt} ({16 * lt}) | {label} | {s * 1e6:.2f} us | {nb / s / 1e9:.0f} |", flush=True)
    if "mfma" in what:
        print("| form | waves per SIMD | TFLOP/s |\n|---|---|---|", flush=True)
        fo = torch.zeros(1 << 16, dtype=torch.float32, device=dev)
        iters = 4096
        for blocks, label in ((256, "1"), (2048, "8")):
            s = _graph_time(torch, [lambda: mfma_rate(fo, blocks, iters, stream())], side)
            print(f"| 16x16x32, 8 accumulators | {label} | {blocks * 4 * iters * 8 * 16384 / s / 1e12:.0f} |", flush=True)
            s = _graph_time(torch, [lambda: mfma_rate_variant(fo, blocks, iters, 1, stream())], side)
            print(f"| 16x16x32, 16 accumulators | {label} | {blocks * 4 * iters * 16 * 16384 / s / 1e12:.0f} |", flush=True)
            s = _graph_time(torch, [lambda: mfma_rate_variant(fo, blocks, iters, 2, stream())], side)
            print(f"| 32x32x16, 4 accumulators | {label} | {blocks * 4 * iters * 4 * 32768 / s / 1e12:.0f} |", flush=True)


if __name__ == "__main__":
    main()
