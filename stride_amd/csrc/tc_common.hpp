// Device-side building blocks shared by every GEMM kernel of libstride_tc:
// MFMA fragment addressing on the reference tile layout, the deterministic
// epilogue numerics, and the order-independent argmax update.
//
// Fragment geometry (v_mfma_f32_16x16x32_bf16, one wavefront of 64 lanes):
//   A (weights, 16 rows x 32 k):  lane l holds row l%16, k = 8*(l/16) .. +7
//   B (x, 32 k x 16 lanes):       lane l holds lane l%16, k = 8*(l/16) .. +7
//   C/D (16 rows x 16 lanes fp32): lane l holds lane l%16, rows 4*(l/16) .. +3
// A 32-column chunk of a row tile is two adjacent 16x16 tiles (1 KiB, contiguous
// in the packed layout), and k-group g = l/16 of a lane lives in tile g/2, column
// half g%2. So lane l reads 16 contiguous bytes at
//   (g/2)*512 + (l%16)*32 + (g%2)*16
// and one wavefront load instruction covers the 1 KiB chunk exactly once.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <type_traits>

#include "../../include/stride_tc.h"

namespace stride_tc {

// Compile-time loop: calls f(std::integral_constant<int, i>) for i = 0 .. N-1.
// Used where register arrays must be indexed with constants and `#pragma unroll`
// may give up on a large body (a partially rolled loop would index the array at
// run time and move it to scratch memory).
template <int I, int N, class F>
__device__ __forceinline__ void unroll_impl(F& f) {
  if constexpr (I < N) {
    f(std::integral_constant<int, I>{});
    unroll_impl<I + 1, N>(f);
  }
}
template <int N, class F>
__device__ __forceinline__ void unroll(F f) {
  unroll_impl<0, N>(f);
}

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

constexpr int kTileElems = 256;     // one 16x16 tile
constexpr int kChunkBytes = 1024;   // 32 columns of one row/lane tile (two tiles)
constexpr int kChunkCols = 32;
constexpr int kWave = 64;

// Byte offset of lane `lane`'s 16-byte fragment slice inside a 1 KiB chunk.
__device__ __forceinline__ int frag_offset(int lane) {
  const int g = lane >> 4;
  return ((g >> 1) << 9) + ((lane & 15) << 5) + ((g & 1) << 4);
}

// Inverse map: the lane whose fragment slice is the 16-byte piece j of a chunk.
__device__ __forceinline__ int frag_lane_of_piece(int j) {
  const int tile = j >> 5, row = (j & 31) >> 1, half = j & 1;
  return (((tile << 1) | half) << 4) | row;
}

__device__ __forceinline__ bf16x8 as_bf16x8(u32x4 v) { return __builtin_bit_cast(bf16x8, v); }

__device__ __forceinline__ u32x4 load16(const void* p) { return *reinterpret_cast<const u32x4*>(p); }
// Streamed operands are read once per launch: weight chunks (each wave
// instruction reads one whole 1 KiB chunk) and V rows of attention pages.
// STRIDE_TC_WNT / STRIDE_TC_KVNT = 1 issues their loads with the non-temporal
// hint. (K rows are not: a lane reads its 128-byte K row 16 bytes at a time over
// eight instructions, which the hint would turn into eight fetches of the line.)
#ifndef STRIDE_TC_WNT
#define STRIDE_TC_WNT 1
#endif
#ifndef STRIDE_TC_KVNT
#define STRIDE_TC_KVNT 1
#endif
template <int NT = STRIDE_TC_WNT>
__device__ __forceinline__ u32x4 ld_weight(const void* p) {
  if constexpr (NT != 0) return __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
  else return load16(p);
}
__device__ __forceinline__ u32x4 ld_kv(const void* p) {
  if constexpr (STRIDE_TC_KVNT) return __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
  else return load16(p);
}

__device__ __forceinline__ f32x4 mfma(u32x4 a, u32x4 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(a), as_bf16x8(b), c, 0, 0, 0);
}

// v_mfma_f32_32x32x16_bf16: A 32 rows x 16 k (lane l: row l%32, k 8*(l/32) ..
// +7), B 16 k x 32 lanes (lane l: lane l%32, same k), C 32 x 32 (lane l: lane
// l%32, rows 8*(i/4) + 4*(l/32) + i%4). Two of them over k 0-15 then 16-31 give
// the same bits as one v_mfma_f32_16x16x32_bf16 per 16x16 tile over the 32-column
// chunk (checked on the device by the shape-equivalence known-answer test,
// tests/test_gpu_kat.py).
__device__ __forceinline__ f32x16 mfma32(u32x4 a, u32x4 b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(as_bf16x8(a), as_bf16x8(b), c, 0, 0, 0);
}

// 16x16 tile (a, b) (row half a, lane half b) of a 32x32 accumulator, in the
// 16x16x32 C layout (lane l: lane l%16, rows 4*(l/16) + j). Tile element (row
// 4q + j, lane c) with q = l/16 sits in block lane (q%2)*32 + 16b + c, register
// 4*(2a + q/2) + j. Every lane of the wavefront must call it.
__device__ __forceinline__ f32x4 tile_of_block(const f32x16& v, int a, int b, int lane) {
  const int q = lane >> 4;
  const int src = ((q & 1) << 5) + (b << 4) + (lane & 15);
  f32x4 out;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const float v0 = __shfl(v[4 * (2 * a) + j], src);
    const float v1 = __shfl(v[4 * (2 * a + 1) + j], src);
    out[j] = (q >> 1) ? v1 : v0;
  }
  return out;
}

// Inverse: a 32x32 accumulator from its four 16x16 tiles t[a][b]. Block lane l,
// register i holds row 8*(i/4) + 4*(l/32) + i%4, lane l%32: tile (i/8, (l%32)/16),
// tile lane (2*((i/4)%2) + l/32)*16 + l%16, register i%4.
__device__ __forceinline__ f32x16 block_of_tiles(const f32x4 (&t)[2][2], int lane) {
  const int b = (lane >> 4) & 1;
  f32x16 v;
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    const int a = i >> 3;
    const int src = ((2 * ((i >> 2) & 1) + (lane >> 5)) << 4) + (lane & 15);
    const float x0 = __shfl(t[a][0][i & 3], src);
    const float x1 = __shfl(t[a][1][i & 3], src);
    v[i] = b ? x1 : x0;
  }
  return v;
}

__device__ __forceinline__ float f32_of(uint32_t u) { return __uint_as_float(u); }
__device__ __forceinline__ uint32_t u32_of(float f) { return __float_as_uint(f); }

// fp32 -> bf16, round to nearest even on the bit pattern (no NaN special case),
// as the reference's bf16_round_bits (src/kernel_common.h:29-32).
__device__ __forceinline__ uint32_t bf16_rne(float f) {
  const uint32_t u = u32_of(f);
  return (u + 0x7FFFu + ((u >> 16) & 1u)) >> 16;
}

// Deterministic exp (src/numerics.h:16-30): k = floor(x*log2e + 1/2), two-part
// Cody-Waite ln2 reduction, degree-6 Cephes polynomial by FMA, exponent scale.
// Only correctly rounded operations (fma, floor, add) so the bits are fixed.
__device__ __forceinline__ float det_exp(float x) {
  if (x < -87.0f) return 0.0f;
  if (x > 88.0f) return f32_of(0x7F800000u);
  const float kf = floorf(fmaf(x, 1.44269504088896341f, 0.5f));
  float r = fmaf(-kf, 0.693359375f, x);
  r = fmaf(-kf, -2.12194440e-4f, r);
  float p = 1.9875691500e-4f;
  p = fmaf(p, r, 1.3981999507e-3f);
  p = fmaf(p, r, 8.3334519073e-3f);
  p = fmaf(p, r, 4.1665795894e-2f);
  p = fmaf(p, r, 1.6666665459e-1f);
  p = fmaf(p, r, 5.0000001201e-1f);
  const float y = fmaf(fmaf(p, r, 1.0f), r, 1.0f);
  return f32_of(u32_of(y) + (static_cast<uint32_t>(static_cast<int32_t>(kf)) << 23));
}

// x * sigmoid(x) as x / (1 + exp(-x)); the division is IEEE (hipcc's default
// correctly rounded fp32 divide).
__device__ __forceinline__ float det_silu(float x) { return x / (1.0f + det_exp(-x)); }

// Lexicographic order on (value, -index): larger value wins, ties go to the
// smaller index (src/kernel_common.h:58-60).
__device__ __forceinline__ bool better_than(float v, int32_t i, float cv, int32_t ci) {
  return v > cv || (v == cv && i < ci);
}

// Merge (value, index) into a BestEntry with a 64-bit compare-and-swap. The
// result is the lexicographic max whatever order the updates arrive in
// (src/kernel_common.h:64-82).
__device__ __forceinline__ void best_update(StrideBestEntry* slot, float value, int32_t index) {
  unsigned long long* word = reinterpret_cast<unsigned long long*>(slot);
  const unsigned long long want =
      (static_cast<unsigned long long>(static_cast<uint32_t>(index)) << 32) | u32_of(value);
  unsigned long long seen = __hip_atomic_load(word, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  for (;;) {
    const float cv = f32_of(static_cast<uint32_t>(seen));
    const int32_t ci = static_cast<int32_t>(seen >> 32);
    if (!better_than(value, index, cv, ci)) return;
    const unsigned long long prev = atomicCAS(word, seen, want);
    if (prev == seen) return;
    seen = prev;
  }
}

}  // namespace stride_tc
