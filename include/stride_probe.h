/* Methodology probes for the MI355X GEMM design (libstride_probe.so), the gfx950
 * counterparts of the reference's tools/tc_probe.cu (Q1: mma position invariance,
 * tools/tc_probe.cu:25-35,106-139) and tools/bench_memread.cu (DRAM read pattern
 * throughput, tools/bench_memread.cu:20-83). Not part of the GEMM path. */
#ifndef STRIDE_PROBE_H
#define STRIDE_PROBE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* One v_mfma_f32_16x16x32_bf16 per tile t: out_t = A_t * B_t + C_t, where A_t is
 * a 16-row x 32-column bf16 chunk in the packed weight layout (two 16x16 tiles,
 * 1 KiB), B_t a 32-column chunk of 16 activation lanes in the x layout (1 KiB),
 * and C_t / out_t fp32 16x16 tiles in the h layout ([16 lanes][16 rows]). */
int stride_probe_mfma_tiles(const uint16_t* a, const uint16_t* b, const float* c, float* out, int32_t tiles,
                            void* stream);

/* Sustained MFMA issue rate: `blocks` workgroups of 4 waves each run `iters`
 * rounds of 8 independent v_mfma_f32_16x16x32_bf16 from registers (16384 flops
 * each); time it to get the achievable dense bf16 rate. */
int stride_probe_mfma_rate(float* out, int32_t blocks, int32_t iters, void* stream);
/* variant 1: 16 independent 16x16x32 accumulators per round; variant 2: 4
 * independent v_mfma_f32_32x32x16_bf16 (32768 flops each) per round. */
int stride_probe_mfma_rate_variant(float* out, int32_t blocks, int32_t iters, int32_t variant, void* stream);

/* Streams `bytes` (a multiple of 16) from `buf` with `blocks` workgroups of 256
 * threads, each thread keeping `unroll` (1, 4, 8 or 16) 16-byte loads in flight,
 * consecutive threads on consecutive 16-byte words; writes one xor-checksum word
 * per workgroup to out[blocks]. blocks = 0 picks one workgroup per 64 KiB. */
int stride_probe_read(const void* buf, int64_t bytes, uint32_t* out, int32_t blocks, int32_t unroll, void* stream);

/* Strip streaming, the decode GEMM pattern: `bytes / strip` strips of `strip`
 * bytes (a multiple of 1 KiB); wave w of the grid (4 waves per workgroup) reads
 * strips w, w + waves, ... in 1 KiB pieces (16 bytes per lane), `unroll` (4, 8,
 * 16) pieces in flight; `rotate` != 0 starts wave w at piece 7w mod pieces. */
int stride_probe_strip_read(const void* buf, int64_t bytes, int64_t strip, int32_t blocks, int32_t unroll,
                            int32_t rotate, uint32_t* out, void* stream);

/* Equivalence of the two bf16 MFMA shapes: for each of `cases` 32x32 output
 * blocks chained over `chunks` 32-column chunks from c0, o16 receives the result
 * of v_mfma_f32_16x16x32_bf16 (one per 16x16 sub-block and chunk) and o32 that of
 * v_mfma_f32_32x32x16_bf16 (two per chunk). a: [cases][32][32*chunks] bf16,
 * b: [cases][32][32*chunks] bf16, c0/o16/o32: [cases][32][32] fp32. */
int stride_probe_mfma_equiv(const uint16_t* a, const uint16_t* b, const float* c0, float* o16, float* o32,
                            int32_t cases, int32_t chunks, void* stream);

/* Decode-structure ceiling (measures the kernel structure, computes nothing
 * useful): row_tiles / 4 workgroups of 4 compute waves, each streaming one
 * weight strip of `chunks` 1 KiB chunks (a multiple of 16) from w into
 * registers 16 chunks ahead and issuing lane_tiles (4 or 8) 16x16x32 bf16 MFMAs
 * per chunk against activation fragments taken from registers (mode 0), from a
 * static LDS slab with a barrier every 4 chunks (mode 1), or from an LDS ring
 * that a fifth wave refills from x ([lane_tiles][chunks] 1 KiB chunks) with
 * global_load_lds (mode 2, what a real kernel must do). out: row_tiles * 64 f32x4. */
int stride_probe_decode_ceiling(const void* w, int32_t row_tiles, int32_t chunks, const void* x, int32_t lane_tiles,
                                int32_t mode, float* out, void* stream);

#ifdef __cplusplus
}
#endif

#endif
