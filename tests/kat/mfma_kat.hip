// Known-answer kernels for the hardware facts the batch-invariance design rests
// on (test infrastructure, built into tests/kat/libmfma_kat.so; not part of the
// product): one v_mfma_f32_16x16x32_bf16 per tile on the packed tile layout (the
// position-invariance test permutes rows and lanes inside a tile), and the
// equivalence of one 16x16x32 MFMA per 32-column chunk with two chained
// 32x32x16 MFMAs. The gfx950 counterpart of the reference's tc_probe Q1
// (tools/tc_probe.cu:25-35, 106-139).
#include <hip/hip_runtime.h>

#include "../../stride_amd/csrc/tc_common.hpp"

namespace {

using namespace stride_tc;

// out_t = A_t * B_t + C_t for tile t: A_t a 16-row x 32-column bf16 chunk in the
// packed weight layout (1 KiB), B_t a 32-column chunk of 16 activation lanes in
// the x layout (1 KiB), C_t / out_t fp32 16x16 tiles in the h layout.
__global__ __launch_bounds__(64) void k_mfma_tiles(const uint16_t* a, const uint16_t* b, const float* c, float* out) {
  const int t = blockIdx.x, lane = threadIdx.x;
  const int off = frag_offset(lane);
  const u32x4 av = load16(reinterpret_cast<const char*>(a) + static_cast<int64_t>(t) * kChunkBytes + off);
  const u32x4 bv = load16(reinterpret_cast<const char*>(b) + static_cast<int64_t>(t) * kChunkBytes + off);
  const int64_t base = static_cast<int64_t>(t) * kTileElems + (lane & 15) * 16 + (lane >> 4) * 4;
  const f32x4 cv = *reinterpret_cast<const f32x4*>(c + base);
  *reinterpret_cast<f32x4*>(out + base) = mfma(av, bv, cv);
}

// One 32x32 output block per workgroup chained over `chunks` 32-column chunks
// from c0: (a) four v_mfma_f32_16x16x32_bf16, one per 16x16 sub-block and chunk,
// into o16; (b) two v_mfma_f32_32x32x16_bf16 per chunk (columns 0-15, then
// 16-31) into o32. a: [32 rows][32*chunks] bf16 row-major, b: [32 lanes][32*chunks],
// c0 and the outputs [32 rows][32 lanes] fp32.
__global__ __launch_bounds__(64) void k_mfma_equiv(const uint16_t* a, const uint16_t* b, const float* c0, float* o16,
                                                   float* o32, int chunks) {
  const int lane = threadIdx.x;
  const int t = blockIdx.x;
  const int kk = 32 * chunks;
  a += static_cast<int64_t>(t) * 32 * kk;
  b += static_cast<int64_t>(t) * 32 * kk;
  c0 += t * 1024;
  o16 += t * 1024;
  o32 += t * 1024;
  auto frag = [&](const uint16_t* m, int row, int k) {
    u32x4 v;
    const uint32_t* p = reinterpret_cast<const uint32_t*>(m + static_cast<int64_t>(row) * kk + k);
    v[0] = p[0]; v[1] = p[1]; v[2] = p[2]; v[3] = p[3];
    return v;
  };
  // (a) C lane l holds lane column l%16, rows 4*(l/16)+i.
  for (int rb = 0; rb < 2; ++rb)
    for (int cb = 0; cb < 2; ++cb) {
      f32x4 acc;
      for (int i = 0; i < 4; ++i) acc[i] = c0[(rb * 16 + 4 * (lane / 16) + i) * 32 + cb * 16 + lane % 16];
      for (int c = 0; c < chunks; ++c) {
        const u32x4 fa = frag(a, rb * 16 + lane % 16, 32 * c + 8 * (lane / 16));
        const u32x4 fb = frag(b, cb * 16 + lane % 16, 32 * c + 8 * (lane / 16));
        acc = mfma(fa, fb, acc);
      }
      for (int i = 0; i < 4; ++i) o16[(rb * 16 + 4 * (lane / 16) + i) * 32 + cb * 16 + lane % 16] = acc[i];
    }
  // (b) C lane l holds lane column l%32, rows 8*(i/4) + 4*(l/32) + i%4.
  f32x16 acc;
  for (int i = 0; i < 16; ++i) acc[i] = c0[(8 * (i / 4) + 4 * (lane / 32) + i % 4) * 32 + lane % 32];
  for (int c = 0; c < chunks; ++c)
    for (int h = 0; h < 2; ++h) {
      const u32x4 fa = frag(a, lane % 32, 32 * c + 16 * h + 8 * (lane / 32));
      const u32x4 fb = frag(b, lane % 32, 32 * c + 16 * h + 8 * (lane / 32));
      acc = mfma32(fa, fb, acc);
    }
  for (int i = 0; i < 16; ++i) o32[(8 * (i / 4) + 4 * (lane / 32) + i % 4) * 32 + lane % 32] = acc[i];
}

}  // namespace

extern "C" int mfma_kat_tiles(const uint16_t* a, const uint16_t* b, const float* c, float* out, int32_t tiles,
                              void* stream) {
  if (!a || !b || !c || !out || tiles < 0) return 1;
  if (tiles == 0) return 0;
  hipLaunchKernelGGL(k_mfma_tiles, dim3(tiles), dim3(64), 0, static_cast<hipStream_t>(stream), a, b, c, out);
  return static_cast<int>(hipGetLastError());
}

extern "C" int mfma_kat_equiv(const uint16_t* a, const uint16_t* b, const float* c0, float* o16, float* o32,
                              int32_t cases, int32_t chunks, void* stream) {
  if (!a || !b || !c0 || !o16 || !o32 || cases <= 0 || chunks <= 0) return 1;
  hipLaunchKernelGGL(k_mfma_equiv, dim3(cases), dim3(64), 0, static_cast<hipStream_t>(stream), a, b, c0, o16, o32,
                     chunks);
  return static_cast<int>(hipGetLastError());
}
