"""Machine-code checks on this repository's own gfx950 build (CPU only).

An MFMA ignores the EXEC mask: if one sits in a block that the compiler
entered by narrowing EXEC and chose not to branch around (it skips
`s_cbranch_execz` for short blocks on the assumption that masked lanes do
nothing), the MFMA accumulates even when no lane is meant to. That silently
adds a chunk twice. Every k-loop must therefore guard MFMAs with scalar
(wave-uniform) branches only; this test disassembles the built library and
fails if any MFMA is reachable, in straight-line order, after an EXEC
narrowing with no `s_cbranch_execz` in between.

Second check: every LDS-pipelined kernel (k_pipe, k_pipe32) must use exactly the LDS of
its staging ring, NS stages x (mats*WM*WRT + WN*WLT) tiles x KC chunks x 1 KiB.
Anything more is a private copy the compiler moved into LDS (a local struct
indexed at run time), which costs LDS capacity and an LDS round trip per use.
"""
import functools
import os
import re
import struct
import subprocess
import tempfile

import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
PKG = os.path.join(os.path.dirname(HERE), "stride_amd")
OBJDUMP = "/opt/rocm/llvm/bin/llvm-objdump"
MAGIC = b"__CLANG_OFFLOAD_BUNDLE__"


def code_objects(lib_path: str):
    """The gfx950 code objects of every offload bundle embedded in a hipcc-built
    .so (one per translation unit; bundle layout: magic, u64 count, then per
    entry u64 offset, u64 size, u64 triple length, triple)."""
    data = open(lib_path, "rb").read()
    out = []
    base = data.find(MAGIC)
    while base >= 0:
        (count,) = struct.unpack_from("<Q", data, base + len(MAGIC))
        p = base + len(MAGIC) + 8
        for _ in range(count):
            off, size, tlen = struct.unpack_from("<QQQ", data, p)
            p += 24
            triple = data[p:p + tlen].decode(errors="replace")
            p += tlen
            if "gfx950" in triple:
                out.append(data[base + off:base + off + size])
        base = data.find(MAGIC, base + len(MAGIC))
    assert out, "no gfx950 code object in " + lib_path
    return out


@functools.lru_cache(maxsize=None)
def disassemble(lib_path: str) -> str:
    """gfx950 disassembly of every code object in the library."""
    parts = []
    with tempfile.TemporaryDirectory() as d:
        for i, obj in enumerate(code_objects(lib_path)):
            co = os.path.join(d, f"k{i}.co")
            open(co, "wb").write(obj)
            parts.append(subprocess.run([OBJDUMP, "-d", "--mcpu=gfx950", co], capture_output=True, text=True,
                                        check=True).stdout)
    return "\n".join(parts)


def functions(disasm: str):
    """{function label: [instruction lines]} of a disassembly."""
    out, fn = {}, None
    for line in disasm.splitlines():
        s = line.strip()
        m = re.match(r"^[0-9a-f]+ <(.+)>:$", s)
        if m:
            fn = m.group(1)
            out[fn] = []
        elif fn and s:
            out[fn].append(s)
    return out


NARROW = ("s_and_saveexec", "s_andn2_saveexec", "s_or_saveexec", "s_xor_saveexec", "s_and_b64 exec",
          "s_andn2_b64 exec", "s_xor_b64 exec")
RESTORE = ("s_or_b64 exec", "s_mov_b64 exec", "s_cbranch_execz", "s_cbranch_execnz")


def masked_mfmas(disasm: str):
    """(function, instruction) pairs where an MFMA follows an EXEC narrowing
    with no branch-around or restore in between."""
    out, fn, masked = [], None, False
    for line in disasm.splitlines():
        s = line.strip()
        if s.endswith(">:"):
            fn, masked = s[s.find("<") + 1:-2], False
            continue
        ins = s.split("//")[0].strip()
        if not ins:
            continue
        if ins.startswith(NARROW):
            masked = True
        elif ins.startswith(RESTORE):
            masked = False
        elif ins.startswith("v_mfma") and masked:
            out.append((fn, ins))
    return out


def test_scanner_flags_unguarded_mfma():
    bad = """
<k>:
	s_and_saveexec_b64 s[2:3], s[0:1]
	v_mfma_f32_16x16x32_bf16 v[6:9], v[10:13], v[26:29], v[6:9]
	s_or_b64 exec, exec, s[2:3]
"""
    good = bad.replace("s_and_saveexec_b64 s[2:3], s[0:1]",
                       "s_and_saveexec_b64 s[2:3], s[0:1]\n\ts_cbranch_execz .LBB0_2")
    assert masked_mfmas(bad) and not masked_mfmas(good)


@pytest.mark.parametrize("lib", ["stride_amd/libstride_tc.so", "tests/kat/libmfma_kat.so"])
def test_no_mfma_under_exec_mask(lib):
    path = os.path.join(os.path.dirname(PKG), lib)
    if not os.path.exists(path):
        pytest.skip(lib + " not built")
    if not os.path.exists(OBJDUMP):
        pytest.skip("llvm-objdump not available")
    dis = disassemble(path)
    assert "v_mfma" in dis
    bad = masked_mfmas(dis)
    assert not bad, f"{len(bad)} MFMAs under an exec mask, first in {bad[0][0]}"


def kernel_lds(co_path: str):
    """(kernel name, group segment bytes) from the code object's metadata note."""
    notes = subprocess.run([OBJDUMP.replace("llvm-objdump", "llvm-readelf"), "--notes", co_path],
                           capture_output=True, text=True, check=True).stdout
    out, grp = [], None
    for line in notes.splitlines():
        line = line.strip()
        if line.startswith(".group_segment_fixed_size:"):
            grp = int(line.split()[-1])
        elif line.startswith(".name:"):
            out.append((line.split()[-1], grp))
    return out


def test_pipe_lds_is_exactly_the_ring():
    path = os.path.join(PKG, "libstride_tc.so")
    if not os.path.exists(path):
        pytest.skip("libstride_tc.so not built")
    if not os.path.exists(OBJDUMP):
        pytest.skip("llvm tools not available")
    kernels = []
    with tempfile.TemporaryDirectory() as d:
        for i, obj in enumerate(code_objects(path)):
            co = os.path.join(d, f"k{i}.co")
            open(co, "wb").write(obj)
            kernels += kernel_lds(co)
    seen = 0
    for name, grp in kernels:
        m = re.search(r"k_pipe(?:32)?INS_\d+(\w+?)ELi(\d+)ELi(\d+)ELi(\d+)ELi(\d+)ELi(\d+)ELi(\d+)ELi(\d+)ELb(\d)", name)
        if not m:
            continue
        wrt, wlt, wm, wn, kc, ns, _ = map(int, m.groups()[1:8])
        mats = 2 if m.group(1) == "EpiGateUp" else 1
        assert grp == ns * (mats * wm * wrt + wn * wlt) * kc * 1024, f"{name}: {grp} bytes of LDS"
        seen += 1
    assert seen > 0


def test_split_partials_travel_device_coherent():
    """The one-split-per-workgroup kernels publish split partials with 16-byte
    buffer stores and read them back with buffer loads, both with the sc1 cache
    policy (coherent at device scope across XCDs), and every such store has
    completed (s_waitcnt vmcnt(0)) before the workgroup's arrival atomic. The
    fixed-order fold relies on exactly this code; a compiler that emitted the
    accesses without sc1, or moved the atomic ahead of the wait, would break it
    silently, so the built machine code is checked here."""
    path = os.path.join(PKG, "libstride_tc.so")
    if not os.path.exists(path):
        pytest.skip("libstride_tc.so not built")
    if not os.path.exists(OBJDUMP):
        pytest.skip("llvm-objdump not available")
    seen = 0
    for name, ins in functions(disassemble(path)).items():
        stores = [i for i, s in enumerate(ins) if s.startswith("buffer_store_dwordx4")]
        if not stores:
            continue
        seen += 1
        for s in ins:
            if s.startswith(("buffer_store_dwordx4", "buffer_load_dwordx4")):
                assert " sc1" in s, f"{name}: {s}"
        atomics = [i for i, s in enumerate(ins) if s.startswith("global_atomic_add")]
        assert atomics, f"{name}: partial stores but no arrival atomic"
        for a in atomics:
            before = [i for i in stores if i < a]
            if before:
                waits = [s for s in ins[before[-1]:a] if s.startswith("s_waitcnt") and "vmcnt(0)" in s]
                assert waits, f"{name}: arrival atomic not after vmcnt(0)"
    assert seen > 0
