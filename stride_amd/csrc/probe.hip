// Methodology probes (include/stride_probe.h): MFMA position invariance and HBM
// read throughput on gfx950. Not part of the GEMM path.
#include <hip/hip_runtime.h>

#include "../../include/stride_probe.h"
#include "tc_common.hpp"

namespace {

using namespace stride_tc;

__global__ __launch_bounds__(64) void k_mfma_tiles(const uint16_t* a, const uint16_t* b, const float* c, float* out) {
  const int t = blockIdx.x, lane = threadIdx.x;
  const int off = frag_offset(lane);
  const u32x4 av = load16(reinterpret_cast<const char*>(a) + static_cast<int64_t>(t) * kChunkBytes + off);
  const u32x4 bv = load16(reinterpret_cast<const char*>(b) + static_cast<int64_t>(t) * kChunkBytes + off);
  const int64_t base = static_cast<int64_t>(t) * kTileElems + (lane & 15) * 16 + (lane >> 4) * 4;
  const f32x4 cv = *reinterpret_cast<const f32x4*>(c + base);
  *reinterpret_cast<f32x4*>(out + base) = mfma(av, bv, cv);
}

template <int U>
__global__ __launch_bounds__(256) void k_read(const u32x4* buf, int64_t words, uint32_t* out) {
  const int64_t stride = static_cast<int64_t>(gridDim.x) * 256;
  uint32_t x = 0;
  int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  for (; i + (U - 1) * stride < words; i += U * stride) {
    u32x4 v[U];
#pragma unroll
    for (int u = 0; u < U; ++u) v[u] = buf[i + u * stride];
#pragma unroll
    for (int u = 0; u < U; ++u) x ^= v[u][0] ^ v[u][1] ^ v[u][2] ^ v[u][3];
  }
  for (; i < words; i += stride) {
    const u32x4 v = buf[i];
    x ^= v[0] ^ v[1] ^ v[2] ^ v[3];
  }
  __shared__ uint32_t red[256];
  red[threadIdx.x] = x;
  __syncthreads();
  if (threadIdx.x == 0) {
    uint32_t r = 0;
    for (int k = 0; k < 256; ++k) r ^= red[k];
    out[blockIdx.x] = r;
  }
}

}  // namespace

extern "C" int stride_probe_mfma_tiles(const uint16_t* a, const uint16_t* b, const float* c, float* out, int32_t tiles,
                                       void* stream) {
  if (!a || !b || !c || !out || tiles < 0) return 1;
  if (tiles == 0) return 0;
  hipLaunchKernelGGL(k_mfma_tiles, dim3(tiles), dim3(64), 0, static_cast<hipStream_t>(stream), a, b, c, out);
  return static_cast<int>(hipGetLastError());
}

extern "C" int stride_probe_read(const void* buf, int64_t bytes, uint32_t* out, int32_t blocks, int32_t unroll,
                                 void* stream) {
  if (!buf || !out || bytes <= 0 || bytes % 16 != 0) return 1;
  const int64_t words = bytes / 16;
  if (blocks <= 0) blocks = static_cast<int32_t>((bytes + 65535) / 65536);
  hipStream_t st = static_cast<hipStream_t>(stream);
  const u32x4* p = static_cast<const u32x4*>(buf);
  switch (unroll) {
    case 1: hipLaunchKernelGGL(k_read<1>, dim3(blocks), dim3(256), 0, st, p, words, out); break;
    case 4: hipLaunchKernelGGL(k_read<4>, dim3(blocks), dim3(256), 0, st, p, words, out); break;
    case 8: hipLaunchKernelGGL(k_read<8>, dim3(blocks), dim3(256), 0, st, p, words, out); break;
    case 16: hipLaunchKernelGGL(k_read<16>, dim3(blocks), dim3(256), 0, st, p, words, out); break;
    default: return 1;
  }
  return static_cast<int>(hipGetLastError());
}
