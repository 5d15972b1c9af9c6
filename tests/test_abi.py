"""C-ABI library checks that need no GPU: it loads, exports every symbol that
include/stride_tc.h and include/stride_exact.h declare, its structs are
byte-compatible with the reference's parameter blocks, the split rule, and
argument rejection before any launch."""
import ctypes as C
import os
import re
import subprocess

import pytest

from stride_amd import _lib
from stride_amd import tc

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "stride_tc.h")
EXACT_HEADER = os.path.join(ROOT, "include", "stride_exact.h")
REF_SRC = "/root/reference/src"


def test_exports_match_header():
    lib = _lib.load()
    declared = set(re.findall(r"\b(stride_tc_\w+)\s*\(", open(HEADER).read()))
    declared |= set(re.findall(r"\b(stride_k_\w+)\s*\(", open(EXACT_HEADER).read()))
    assert declared == set(_lib.EXPORTS)
    for name in declared:
        assert hasattr(lib, name), name
    assert b"gfx950" in lib.stride_tc_version()


def test_ctypes_layout():
    _lib.check_layout()


PROBE = r"""
#include <cstddef>
#include <cstdio>
#include HDR
int main() {
  printf("%zu %zu %zu %zu %zu %zu %zu %zu %zu %zu\n", sizeof(GM), sizeof(KV), sizeof(LN), sizeof(BE),
         sizeof(QKV), offsetof(QKV, kv), offsetof(QKV, head_dim), sizeof(RES), sizeof(MLP), sizeof(LMG));
  printf("%zu %zu %zu %zu %zu %zu %zu %zu %zu\n", sizeof(EMB), sizeof(NRM), offsetof(NRM, eps), sizeof(CMP),
         offsetof(CMP, col_tiles), sizeof(ATT), offsetof(ATT, kv), offsetof(ATT, items), offsetof(ATT, scale));
}
"""


def _probe(tmp_path, include, names, extra=()):
    src = tmp_path / "probe.cpp"
    defs = "".join(f"#define {k} {v}\n" for k, v in names.items())
    src.write_text(defs + PROBE.replace("HDR", f'"{include}"'))
    exe = tmp_path / "probe"
    subprocess.run(["g++", "-std=c++17", *extra, str(src), "-o", str(exe)], check=True)
    return subprocess.run([str(exe)], check=True, capture_output=True, text=True).stdout.split()


def test_struct_layout_matches_reference(tmp_path):
    ours = _probe(tmp_path, HEADER, dict(GM="StrideGemmMat", KV="StrideKvRef", LN="StrideLanes", BE="StrideBestEntry",
                                         QKV="StrideTcQkvParams", RES="StrideTcGemmResidualParams",
                                         MLP="StrideTcMlp13Params", LMG="StrideTcLmGreedyParams",
                                         EMB="StrideTcEmbedParams", NRM="StrideTcNormParams",
                                         CMP="StrideTcCompactParams", ATT="StrideAttentionParams"))
    assert ours == ["16", "56", "16", "8", "176", "88", "172", "48", "64", "56",
                    "48", "48", "44", "48", "44", "176", "48", "120", "168"]
    if not os.path.exists(os.path.join(REF_SRC, "kernels_tc.h")):
        pytest.skip("reference tree absent")
    theirs = _probe(tmp_path, os.path.join(REF_SRC, "kernels_tc.h"),
                    dict(GM="stride::GemmMat", KV="stride::KvRef", LN="stride::Lanes", BE="stride::BestEntry",
                         QKV="stride::TcQkvParams", RES="stride::TcGemmResidualParams", MLP="stride::TcMlp13Params",
                         LMG="stride::TcLmGreedyParams", EMB="stride::TcEmbedParams", NRM="stride::TcNormParams",
                         CMP="stride::TcCompactParams", ATT="stride::AttentionParams"))
    assert ours == theirs


EXACT_PROBE = r"""
#include <cstddef>
#include <cstdio>
#include HDR
int main() {
  printf("%zu %zu %zu %zu %zu %zu %zu %zu %zu %zu %zu %zu %zu %zu %zu\n", sizeof(EMB), offsetof(EMB, dim), sizeof(NRM),
         offsetof(NRM, eps), sizeof(QKV), offsetof(QKV, kv), offsetof(QKV, rope), offsetof(QKV, head_dim), sizeof(RES),
         sizeof(MLP), offsetof(MLP, z), sizeof(CMP), offsetof(CMP, dim), sizeof(LMG), sizeof(LMF));
}
"""


def test_exact_struct_layout_matches_reference(tmp_path):
    names = dict(EMB="EmbedParams", NRM="NormParams", QKV="QkvParams", RES="GemmResidualParams", MLP="Mlp13Params",
                 CMP="CompactParams", LMG="LmGreedyParams", LMF="LmFullParams")

    def probe(include, prefix):
        src = tmp_path / f"p{len(prefix)}.cpp"
        defs = "".join(f"#define {k} {prefix}{v}\n" for k, v in names.items())
        src.write_text(defs + EXACT_PROBE.replace("HDR", f'"{include}"'))
        exe = tmp_path / f"p{len(prefix)}"
        subprocess.run(["g++", "-std=c++17", str(src), "-o", str(exe)], check=True)
        return subprocess.run([str(exe)], check=True, capture_output=True, text=True).stdout.split()

    ours = probe(EXACT_HEADER, "Stride")
    assert ours == ["48", "40", "48", "44", "176", "88", "144", "172", "48", "64", "56", "56", "48", "56", "48"]
    if not os.path.exists(os.path.join(REF_SRC, "kernels.h")):
        pytest.skip("reference tree absent")
    assert probe(os.path.join(REF_SRC, "kernels.h"), "stride::") == ours


def test_split_rule():
    cases = {(2048, 2048): 4, (3072, 2048): 4, (512, 2048): 4, (2048, 8192): 4, (8192, 2048): 1, (4096, 2048): 4, (4112, 2048): 1,
             (128256, 2048): 1, (16, 64): 2, (16, 32): 1, (64, 96): 3, (64, 160): 1, (64, 192): 2, (64, 256): 4,
             # K = 16 (mod 32): whole chunks decide, the half chunk joins the last split
             (16, 48): 1, (16, 16): 1, (2048, 2064): 4, (8192, 2064): 1, (64, 112): 3}
    for (n, k), s in cases.items():
        assert tc.split_count(n, k) == s, (n, k)
    with pytest.raises(_lib.StrideTcError):
        tc.split_count(16, 24)


def test_split_rule_has_no_runtime_hook():
    """The split rule is a constant of the build: the library exports no call that
    changes it, so the bits depend on the weight shape only."""
    lib = _lib.load()
    assert not hasattr(lib, "stride_tc_set_split_rule")
    assert tc.split_count(2048, 2048) == 4


def test_rejects_bad_arguments_without_launch():
    lib = _lib.load()
    p = tc.TcGemmResidualParams(tc.Lanes(17, 1, 0, 0), 0x1000, tc.GemmMat(0x2000, 4, 64), 0x3000)
    assert lib.stride_tc_gemm_residual(C.byref(p), 1, 1, None) == _lib.EINVAL
    assert b"lane_groups" in lib.stride_tc_last_error()
    p = tc.TcGemmResidualParams(tc.Lanes(17, 2, 0, 0), 0x1000, tc.GemmMat(0x2000, 4, 40), 0x3000)
    assert lib.stride_tc_gemm_residual(C.byref(p), 1, 1, None) == _lib.EINVAL
    assert b"multiple of 16" in lib.stride_tc_last_error()
    g = tc.TcLmGreedyParams(tc.Lanes(1, 1, 0, 0), 0x1000, tc.GemmMat(0x2000, 4, 64), 65, 0x3000)
    with pytest.raises(tc.StrideTcError, match="vocab"):
        _lib.check(lib.stride_tc_lm_greedy(C.byref(g), 1, 1, None))
    q = tc.TcQkvParams()
    q.l = tc.Lanes(1, 1, 0, 0)
    q.x = 0x1000
    q.q = q.k = q.v = tc.GemmMat(0x2000, 4, 64)
    q.head_dim = 24
    assert lib.stride_tc_qkv(C.byref(q), None) == _lib.EINVAL
    assert lib.stride_tc_mlp13(None, 1, 1, None) == _lib.EINVAL
    # rows == 0 is a no-op, as the reference's launch<> with zero blocks
    z = tc.TcGemmResidualParams(tc.Lanes(0, 0, 0, 0), 0x1000, tc.GemmMat(0x2000, 4, 64), 0x3000)
    assert lib.stride_tc_gemm_residual(C.byref(z), 1, 1, None) == 0


def test_cpp_shim_compiles_against_reference_header(tmp_path):
    """include/stride_tc_shim.hpp defines stride::tc_* with the reference
    signatures over the C ABI; its static_asserts check the engine's PODs against
    the ABI structs. Compiled here against the reference's own kernels_tc.h."""
    if not os.path.exists(os.path.join(REF_SRC, "kernels_tc.h")):
        pytest.skip("reference tree absent")
    tu = tmp_path / "tc_gemm_hip.cpp"
    tu.write_text('#include "kernels_tc.h"\n#include "stride_tc_shim.hpp"\n'
                  'namespace stride { void* tc_stream() { return nullptr; } }\n')
    subprocess.run(["g++", "-std=c++17", "-Wall", "-Werror", "-c", f"-I{REF_SRC}", f"-I{os.path.join(ROOT, 'include')}",
                    str(tu), "-o", str(tmp_path / "tu.o")], check=True)
    syms = subprocess.run(["nm", "-C", str(tmp_path / "tu.o")], capture_output=True, text=True, check=True).stdout
    for name in ("stride::tc_qkv(stride::TcQkvParams const&)",
                 "stride::tc_gemm_residual(stride::TcGemmResidualParams const&, int, int)",
                 "stride::tc_mlp13(stride::TcMlp13Params const&, int, int)",
                 "stride::tc_lm_greedy(stride::TcLmGreedyParams const&, int, int)",
                 "stride::tc_lm_full(stride::TcLmFullParams const&, int)"):
        assert name in syms, name


def test_exact_shim_compiles_against_reference_header(tmp_path):
    """include/stride_exact_shim.hpp defines stride::k_* with the reference
    signatures (src/kernels.h:146-155) over the C ABI, compiled against the
    reference's own kernels.h together with the tensor-core shim."""
    if not os.path.exists(os.path.join(REF_SRC, "kernels.h")):
        pytest.skip("reference tree absent")
    tu = tmp_path / "exact_hip.cpp"
    tu.write_text('#include "kernels_tc.h"\n#include "stride_tc_shim.hpp"\n#include "stride_exact_shim.hpp"\n'
                  'namespace stride { void* tc_stream() { return nullptr; } }\n')
    subprocess.run(["g++", "-std=c++17", "-Wall", "-Werror", "-c", f"-I{REF_SRC}", f"-I{os.path.join(ROOT, 'include')}",
                    str(tu), "-o", str(tmp_path / "tu.o")], check=True)
    syms = subprocess.run(["nm", "-C", str(tmp_path / "tu.o")], capture_output=True, text=True, check=True).stdout
    for name in ("stride::k_embed(stride::EmbedParams const&)", "stride::k_norm(stride::NormParams const&, int)",
                 "stride::k_qkv(stride::QkvParams const&, int)", "stride::k_attention(stride::AttentionParams const&)",
                 "stride::k_gemm_residual(stride::GemmResidualParams const&, int)",
                 "stride::k_mlp13(stride::Mlp13Params const&, int)", "stride::k_compact(stride::CompactParams const&)",
                 "stride::k_lm_greedy(stride::LmGreedyParams const&, int)",
                 "stride::k_lm_full(stride::LmFullParams const&, int)"):
        assert name in syms, name
