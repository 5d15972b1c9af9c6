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

// Back-to-back independent MFMAs from registers only: 8 accumulators per wave,
// `iters` rounds. Measures the sustained v_mfma_f32_16x16x32_bf16 issue rate.
__global__ __launch_bounds__(256) void k_mfma_rate(float* out, int iters) {
  const int lane = threadIdx.x & 63;
  u32x4 a = {static_cast<uint32_t>(lane) * 0x3f803f80u, 0x3f803f80u, 0x3f803f80u, 0x3f803f80u};
  u32x4 b = {0x3f803f80u, static_cast<uint32_t>(lane), 0x3f803f80u, 0x3f803f80u};
  f32x4 acc[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) acc[i] = f32x4{0.f, 0.f, 0.f, 0.f};
  for (int it = 0; it < iters; ++it) {
#pragma unroll
    for (int i = 0; i < 8; ++i) acc[i] = mfma(a, b, acc[i]);
  }
  f32x4 s = acc[0];
#pragma unroll
  for (int i = 1; i < 8; ++i) s = s + acc[i];
  if (s[0] == 12345.0f) out[threadIdx.x] = s[1];  // keeps the chain alive
}

typedef float f32x16 __attribute__((ext_vector_type(16)));

// Variants for comparison: 16 accumulators of 16x16x32, and 4 of 32x32x16
// (32768 flops each).
__global__ __launch_bounds__(256) void k_mfma_rate16(float* out, int iters) {
  const int lane = threadIdx.x & 63;
  u32x4 a = {static_cast<uint32_t>(lane) * 0x3f803f80u, 0x3f803f80u, 0x3f803f80u, 0x3f803f80u};
  u32x4 b = {0x3f803f80u, static_cast<uint32_t>(lane), 0x3f803f80u, 0x3f803f80u};
  f32x4 acc[16];
#pragma unroll
  for (int i = 0; i < 16; ++i) acc[i] = f32x4{0.f, 0.f, 0.f, 0.f};
  for (int it = 0; it < iters; ++it) {
#pragma unroll
    for (int i = 0; i < 16; ++i) acc[i] = mfma(a, b, acc[i]);
  }
  f32x4 s = acc[0];
#pragma unroll
  for (int i = 1; i < 16; ++i) s = s + acc[i];
  if (s[0] == 12345.0f) out[threadIdx.x] = s[1];
}

__global__ __launch_bounds__(256) void k_mfma_rate32(float* out, int iters) {
  const int lane = threadIdx.x & 63;
  u32x4 a = {static_cast<uint32_t>(lane) * 0x3f803f80u, 0x3f803f80u, 0x3f803f80u, 0x3f803f80u};
  u32x4 b = {0x3f803f80u, static_cast<uint32_t>(lane), 0x3f803f80u, 0x3f803f80u};
  f32x16 acc[4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 16; ++j) acc[i][j] = 0.f;
  for (int it = 0; it < iters; ++it) {
#pragma unroll
    for (int i = 0; i < 4; ++i)
      acc[i] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(as_bf16x8(a), as_bf16x8(b), acc[i], 0, 0, 0);
  }
  float s = 0.f;
#pragma unroll
  for (int i = 0; i < 4; ++i) s += acc[i][0] + acc[i][5];
  if (s == 12345.0f) out[threadIdx.x] = s;
}


// Strip streaming: wave w of the grid reads strips w, w + waves, ... of
// `strip` bytes each, one 1 KiB piece (16 bytes per lane) per load, U pieces in
// flight; the pattern of the decode GEMMs, where every wave streams one row
// tile's contiguous K strip. With `rotate`, wave w starts its strip at piece
// (w * 7) mod pieces and wraps, so that waves in lockstep touch different
// offsets at any moment.
template <int U>
__global__ __launch_bounds__(256) void k_strip_read(const char* buf, int64_t nstrips, int64_t strip, int rotate,
                                                    uint32_t* out) {
  const int lane = threadIdx.x & 63;
  const int64_t wave = static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6);
  const int64_t waves = static_cast<int64_t>(gridDim.x) * 4;
  const int pieces = static_cast<int>(strip / 1024);
  uint32_t x = 0;
  for (int64_t sidx = wave; sidx < nstrips; sidx += waves) {
    const char* base = buf + sidx * strip + lane * 16;
    const int r0 = rotate ? static_cast<int>((wave * 7) % pieces) : 0;
    for (int p = 0; p + U <= pieces; p += U) {
      u32x4 v[U];
#pragma unroll
      for (int u = 0; u < U; ++u) {
        int q = r0 + p + u;
        q = q >= pieces ? q - pieces : q;
        v[u] = load16(base + static_cast<int64_t>(q) * 1024);
      }
#pragma unroll
      for (int u = 0; u < U; ++u) x ^= v[u][0] ^ v[u][1] ^ v[u][2] ^ v[u][3];
    }
  }
  if (x == 0x12345678u) out[0] = x;
}


// Decode-structure ceiling (measurement of the kernel structure, not a GEMM):
// 4 compute waves per workgroup, one 16-row weight strip each (`chunks` 1 KiB
// chunks streamed HBM -> registers, U = 16 ahead), LT lane tiles of activation
// fragments per chunk, LT v_mfma_f32_16x16x32_bf16 per chunk. MODE 0: the
// fragments are constants in registers; MODE 1: read from a static LDS slab,
// one chunk ahead, with a barrier every 4 chunks; MODE 2: as 1 with a fifth
// wave refilling the LDS ring (slabs of 4 chunks, 3 slots) from x
// [LT][chunks] chunks by global_load_lds, as a real kernel must.
template <int LT, int MODE>
__global__ __launch_bounds__(320) void k_decode_ceiling(const u32x4* __restrict__ w, const u32x4* __restrict__ x,
                                                         int chunks, f32x4* out) {
  constexpr int U = 16, S = 4, NSLOT = 3, SLOT = S * LT * 64;
  __shared__ u32x4 ring[NSLOT * SLOT];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int nb = chunks / S;
  if (wave == 4) {  // copy wave (MODE 2 only; otherwise it only keeps the barrier count)
    auto issue = [&](int slab) {
      if constexpr (MODE == 2) {
        u32x4* dst = ring + (slab % NSLOT) * SLOT;
#pragma unroll
        for (int q = 0; q < S * LT; ++q) {
          const int c = min(slab * S + q / LT, chunks - 1);
          __builtin_amdgcn_global_load_lds(
              (const __attribute__((address_space(1))) void*)(x + (static_cast<int64_t>(q % LT) * chunks + c) * 64 + lane),
              (__attribute__((address_space(3))) void*)(dst + q * 64), 16, 0, 0);
        }
      }
    };
    for (int s = 0; s < NSLOT; ++s) issue(s);
    __builtin_amdgcn_s_waitcnt(0);
    __builtin_amdgcn_s_barrier();
    for (int j = 1; j <= nb; ++j) {
      constexpr int n = (NSLOT - 2) * S * LT;
      __builtin_amdgcn_s_waitcnt((n & 0xF) | ((n >> 4) << 14) | (0x7 << 4) | (0xF << 8));
      __builtin_amdgcn_s_barrier();
      issue(j + NSLOT - 1);
    }
    __builtin_amdgcn_s_waitcnt(0);
    return;
  }
  if (MODE != 2)
    for (int i = threadIdx.x; i < NSLOT * SLOT; i += 256) ring[i] = u32x4{static_cast<uint32_t>(i) * 0x10001u, 0x3f803f80u, 0x3f803f80u, 0x3f803f80u};
  const u32x4* wp = w + static_cast<int64_t>(blockIdx.x * 4 + wave) * chunks * 64 + lane;
  f32x4 acc[LT];
#pragma unroll
  for (int l = 0; l < LT; ++l) acc[l] = f32x4{0.f, 0.f, 0.f, 0.f};
  u32x4 buf[U];
#pragma unroll
  for (int u = 0; u < U; ++u) buf[u] = wp[static_cast<int64_t>(u) * 64];
  u32x4 xf[2][LT];
  __builtin_amdgcn_s_waitcnt(0xc07f);
  __builtin_amdgcn_s_barrier();
#pragma unroll
  for (int l = 0; l < LT; ++l) xf[0][l] = MODE == 0 ? u32x4{0x3f803f80u, static_cast<uint32_t>(l), 0u, 0u} : ring[l * 64 + lane];
  const int nbody = __builtin_amdgcn_readfirstlane(chunks / U);
  for (int k = 0; k < nbody; ++k) {
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int c = k * U + u;
      if ((u + 1) % S == 0) {
        __builtin_amdgcn_s_waitcnt(0xc07f);
        __builtin_amdgcn_s_barrier();
      }
      const u32x4 a = buf[u];
      buf[u] = wp[static_cast<int64_t>(min(c + U, chunks - 1)) * 64];
      if constexpr (MODE != 0) {
        const int cn = c + 1;
#pragma unroll
        for (int l = 0; l < LT; ++l) xf[(u + 1) & 1][l] = ring[((cn / S) % NSLOT) * SLOT + ((cn % S) * LT + l) * 64 + lane];
      }
#pragma unroll
      for (int l = 0; l < LT; ++l) acc[l] = mfma(a, xf[MODE == 0 ? 0 : (u & 1)][l], acc[l]);
    }
  }
  f32x4 r = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int l = 0; l < LT; ++l) r = r + acc[l];
  out[(blockIdx.x * 4 + wave) * 64 + lane] = r;
}

}  // namespace

extern "C" int stride_probe_mfma_rate_variant(float* out, int32_t blocks, int32_t iters, int32_t variant, void* stream) {
  if (!out || blocks <= 0 || iters <= 0) return 1;
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (variant == 1) hipLaunchKernelGGL(k_mfma_rate16, dim3(blocks), dim3(256), 0, st, out, iters);
  else if (variant == 2) hipLaunchKernelGGL(k_mfma_rate32, dim3(blocks), dim3(256), 0, st, out, iters);
  else return 1;
  return static_cast<int>(hipGetLastError());
}

extern "C" int stride_probe_mfma_rate(float* out, int32_t blocks, int32_t iters, void* stream) {
  if (!out || blocks <= 0 || iters <= 0) return 1;
  hipLaunchKernelGGL(k_mfma_rate, dim3(blocks), dim3(256), 0, static_cast<hipStream_t>(stream), out, iters);
  return static_cast<int>(hipGetLastError());
}

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

// Equivalence of the two bf16 MFMA shapes on one 32x32 output block chained
// over `chunks` 32-column chunks from the initial value c0: (a) four
// v_mfma_f32_16x16x32_bf16, one per 16x16 sub-block and chunk; (b) two
// v_mfma_f32_32x32x16_bf16 per chunk (columns 0-15, then 16-31). a is
// [32 rows][32*chunks] bf16 row-major, b is [32 lanes][32*chunks], c0 and both
// outputs [32 rows][32 lanes] fp32. One block of 64 threads per test case.
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
  // (a) 16x16x32: C lane l holds lane column l%16, rows 4*(l/16)+i.
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
  // (b) 32x32x16: C lane l holds lane column l%32, rows 8*(i/4) + 4*(l/32) + i%4.
  f32x16 acc;
  for (int i = 0; i < 16; ++i) acc[i] = c0[(8 * (i / 4) + 4 * (lane / 32) + i % 4) * 32 + lane % 32];
  for (int c = 0; c < chunks; ++c)
    for (int h = 0; h < 2; ++h) {
      const u32x4 fa = frag(a, lane % 32, 32 * c + 16 * h + 8 * (lane / 32));
      const u32x4 fb = frag(b, lane % 32, 32 * c + 16 * h + 8 * (lane / 32));
      acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(as_bf16x8(fa), as_bf16x8(fb), acc, 0, 0, 0);
    }
  for (int i = 0; i < 16; ++i) o32[(8 * (i / 4) + 4 * (lane / 32) + i % 4) * 32 + lane % 32] = acc[i];
}

extern "C" int stride_probe_mfma_equiv(const uint16_t* a, const uint16_t* b, const float* c0, float* o16, float* o32,
                                       int32_t cases, int32_t chunks, void* stream) {
  if (cases <= 0 || chunks <= 0) return 1;
  hipLaunchKernelGGL(k_mfma_equiv, dim3(cases), dim3(64), 0, static_cast<hipStream_t>(stream), a, b, c0, o16, o32, chunks);
  return static_cast<int>(hipGetLastError());
}

extern "C" int stride_probe_strip_read(const void* buf, int64_t bytes, int64_t strip, int32_t blocks, int32_t unroll,
                                       int32_t rotate, uint32_t* out, void* stream) {
  if (!buf || !out || strip < 1024 || strip % 1024 != 0 || bytes < strip || blocks <= 0) return 1;
  const int64_t nstrips = bytes / strip;
  hipStream_t st = static_cast<hipStream_t>(stream);
  const char* p = static_cast<const char*>(buf);
  switch (unroll) {
    case 4: hipLaunchKernelGGL(k_strip_read<4>, dim3(blocks), dim3(256), 0, st, p, nstrips, strip, rotate, out); break;
    case 8: hipLaunchKernelGGL(k_strip_read<8>, dim3(blocks), dim3(256), 0, st, p, nstrips, strip, rotate, out); break;
    case 16: hipLaunchKernelGGL(k_strip_read<16>, dim3(blocks), dim3(256), 0, st, p, nstrips, strip, rotate, out); break;
    default: return 1;
  }
  return static_cast<int>(hipGetLastError());
}

extern "C" int stride_probe_decode_ceiling(const void* w, int32_t row_tiles, int32_t chunks, const void* x,
                                           int32_t lane_tiles, int32_t mode, float* out, void* stream) {
  if (!w || !out || row_tiles <= 0 || row_tiles % 4 != 0 || chunks <= 0 || chunks % 16 != 0 || mode < 0 || mode > 2 ||
      (lane_tiles != 4 && lane_tiles != 8) || (mode == 2 && !x))
    return 1;
  const dim3 grid(row_tiles / 4), block(320);
  hipStream_t st = static_cast<hipStream_t>(stream);
  const u32x4* wv = static_cast<const u32x4*>(w);
  const u32x4* xv = static_cast<const u32x4*>(x);
  f32x4* o = reinterpret_cast<f32x4*>(out);
  if (lane_tiles == 8) {
    if (mode == 0) hipLaunchKernelGGL((k_decode_ceiling<8, 0>), grid, block, 0, st, wv, xv, chunks, o);
    else if (mode == 1) hipLaunchKernelGGL((k_decode_ceiling<8, 1>), grid, block, 0, st, wv, xv, chunks, o);
    else hipLaunchKernelGGL((k_decode_ceiling<8, 2>), grid, block, 0, st, wv, xv, chunks, o);
  } else {
    if (mode == 0) hipLaunchKernelGGL((k_decode_ceiling<4, 0>), grid, block, 0, st, wv, xv, chunks, o);
    else if (mode == 1) hipLaunchKernelGGL((k_decode_ceiling<4, 1>), grid, block, 0, st, wv, xv, chunks, o);
    else hipLaunchKernelGGL((k_decode_ceiling<4, 2>), grid, block, 0, st, wv, xv, chunks, o);
  }
  return static_cast<int>(hipGetLastError());
}
