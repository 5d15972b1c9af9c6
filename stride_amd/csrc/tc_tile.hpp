// Prefill-regime kernel (more than 8 lane tiles): LDS-staged block GEMM.
#pragma once

#include "tc_epilogue.hpp"

namespace stride_tc {

// ---------------------------------------------------------------------------
// Prefill regime: LDS-staged block GEMM, 4 waves in a 2x2 grid.

template <class Epi, int WRT, int WLT>
__global__ __launch_bounds__(256) void k_tile(Geometry g, typename Epi::Out o) {
  constexpr int M = Epi::kMats;
  constexpr int BR = 2 * WRT, BL = 2 * WLT;
  constexpr int NB = M * BR + BL;  // 1 KiB blocks staged per chunk
  static_assert(NB % 4 == 0, "staging assumes whole rounds of 256 x 16 B");
  constexpr int ROUNDS = NB / 4;
  __shared__ u32x4 stage[2][NB * kWave];

  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int wr = wave >> 1, wl = wave & 1;
  const int lblocks = (g.lane_groups + BL - 1) / BL;
  const int b = xcd_remap(blockIdx.x, gridDim.x);
  int rb = b / lblocks;
  const int lt0 = (b % lblocks) * BL;
  const int si = locate_segment(g, rb);
  const Segment sg = seg_at(g, si);
  const int rt0 = rb * BR;
  const int chunks = g.col_tiles >> 1;
  const int per = chunks / sg.splits;
  const int64_t strip = static_cast<int64_t>(g.col_tiles) * kTileElems;

  // Staging assignment: thread tid moves piece P = q*256 + tid of each chunk.
  const char* src[ROUNDS];
  int dst[ROUNDS];
#pragma unroll
  for (int q = 0; q < ROUNDS; ++q) {
    const int P = q * 256 + tid;
    const int blk = P >> 6, j = P & 63;
    const uint16_t* base;
    if (blk < M * BR) {
      const int m = blk / BR;
      const int rt = min(rt0 + blk % BR, sg.row_tiles - 1);
      base = sg.w[m] + rt * strip;
    } else {
      const int lt = min(lt0 + blk - M * BR, g.lane_groups - 1);
      base = g.x + lt * strip;
    }
    src[q] = reinterpret_cast<const char*>(base) + j * 16;
    dst[q] = blk * kWave + frag_lane_of_piece(j);
  }

  u32x4 pre[ROUNDS];
#pragma unroll
  for (int q = 0; q < ROUNDS; ++q) pre[q] = load16(src[q]);
#pragma unroll
  for (int q = 0; q < ROUNDS; ++q) stage[0][dst[q]] = pre[q];
  __syncthreads();

  f32x4 acc[M][WRT][WLT], y[M][WRT][WLT];
  for (int c = 0; c < chunks; ++c) {
    const int buf = c & 1;
    if (c + 1 < chunks) {
#pragma unroll
      for (int q = 0; q < ROUNDS; ++q) pre[q] = load16(src[q] + static_cast<int64_t>(c + 1) * kChunkBytes);
    }
    const int s = c / per;
    if (c == s * per) {
#pragma unroll
      for (int m = 0; m < M; ++m)
#pragma unroll
        for (int r = 0; r < WRT; ++r)
#pragma unroll
          for (int l = 0; l < WLT; ++l) {
            acc[m][r][l] = f32x4{0.f, 0.f, 0.f, 0.f};
            if constexpr (Epi::kInitFromOutput) {
              const int rt = rt0 + wr * WRT + r, lt = lt0 + wl * WLT + l;
              if (s == 0 && rt < sg.row_tiles && lt < g.lane_groups) acc[m][r][l] = Epi::init(o, rt, lt, lane);
            }
          }
    }
    u32x4 af[M][WRT], bf[WLT];
#pragma unroll
    for (int m = 0; m < M; ++m)
#pragma unroll
      for (int r = 0; r < WRT; ++r) af[m][r] = stage[buf][(m * BR + wr * WRT + r) * kWave + lane];
#pragma unroll
    for (int l = 0; l < WLT; ++l) bf[l] = stage[buf][(M * BR + wl * WLT + l) * kWave + lane];
#pragma unroll
    for (int l = 0; l < WLT; ++l)
#pragma unroll
      for (int m = 0; m < M; ++m)
#pragma unroll
        for (int r = 0; r < WRT; ++r) acc[m][r][l] = mfma(af[m][r], bf[l], acc[m][r][l]);
    if (c + 1 == (s + 1) * per) {
#pragma unroll
      for (int m = 0; m < M; ++m)
#pragma unroll
        for (int r = 0; r < WRT; ++r)
#pragma unroll
          for (int l = 0; l < WLT; ++l) y[m][r][l] = s == 0 ? acc[m][r][l] : y[m][r][l] + acc[m][r][l];
    }
    if (c + 1 < chunks) {
#pragma unroll
      for (int q = 0; q < ROUNDS; ++q) stage[buf ^ 1][dst[q]] = pre[q];
    }
    __syncthreads();
  }

#pragma unroll
  for (int r = 0; r < WRT; ++r) {
    const int rt = rt0 + wr * WRT + r;
    if (rt >= sg.row_tiles) continue;
#pragma unroll
    for (int l = 0; l < WLT; ++l) {
      const int lt = lt0 + wl * WLT + l;
      if (lt >= g.lane_groups) continue;
      f32x4 yy[M];
#pragma unroll
      for (int m = 0; m < M; ++m) yy[m] = y[m][r][l];
      Epi::apply(o, g, si, rt, lt, yy, lane);
    }
  }
}

}  // namespace stride_tc
