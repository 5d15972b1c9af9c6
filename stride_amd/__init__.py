"""stride_amd: MI355X-native (gfx950) batch-invariant BF16 linear-layer GEMMs for
the stride inference engine, behind the C ABI of include/stride_tc.h.

    stride_amd.tc      the operator surface (tc_qkv, tc_gemm_residual, tc_mlp13,
                       tc_lm_greedy, tc_lm_full) mirroring src/kernels_tc.h
    stride_amd.layout  tile packing / unpacking of weights and activations
    stride_amd.synth   portable seeded synthetic inputs
    stride_amd.build   builds libstride_tc.so with hipcc for gfx950
"""
__version__ = "0.1.0"
