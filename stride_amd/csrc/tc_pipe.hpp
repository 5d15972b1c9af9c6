// Prefill-regime kernel: a multi-stage LDS pipeline fed by direct global->LDS
// loads (global_load_lds_dwordx4, gfx950).
//
// A workgroup of WM x WN wavefronts owns a block of BR = WM*WRT row tiles by
// BL = WN*WLT lane tiles. K is consumed in stages of KC 32-column chunks. For
// each stage the workgroup copies M*BR weight chunks and BL activation chunks
// (1 KiB each) from HBM straight into an NS-deep LDS ring: one wave instruction
// moves one chunk, each lane fetching the 16 bytes its MFMA fragment position
// needs, so the chunk lands in LDS already in fragment order and every later
// ds_read_b128 is a linear, conflict-free 1 KiB read. No registers hold data in
// flight, so up to NS stages (tens of KiB) are outstanding per workgroup.
//
// Synchronisation per stage: each wave waits until its own copies of the stage
// have landed (s_waitcnt vmcnt with the later stages still outstanding), then one
// s_barrier makes every wave's copies visible and guarantees that the slot about
// to be refilled has been consumed. The raw s_barrier is used instead of
// __syncthreads() because the latter also waits for every outstanding load.
//
// Arithmetic: per output tile, the chunks of each split are chained in ascending
// order by v_mfma_f32_16x16x32_bf16 into an accumulator that starts at zero (at h
// for split 0 of a residual GEMM) and finished splits are folded into a running
// sum, y = ((c0 + c1) + c2) + ..., exactly as the decode kernels compute it.
#pragma once

#include "tc_epilogue.hpp"

namespace stride_tc {

#define STRIDE_TC_GLOBAL(p) ((const __attribute__((address_space(1))) void*)(p))
#define STRIDE_TC_LDS(p) ((__attribute__((address_space(3))) void*)(p))

// s_waitcnt immediate for "at most n vector-memory operations outstanding"
// (gfx9 encoding: vmcnt low bits [3:0], high bits [15:14]; expcnt and lgkmcnt
// left at their no-wait maxima).
constexpr int vmcnt_imm(int n) { return (n & 0xF) | ((n >> 4) << 14) | (0x7 << 4) | (0xF << 8); }
// The same with lgkmcnt = 0 (all LDS reads of this wave returned).
constexpr int vm_lgkm0_imm(int n) { return (n & 0xF) | ((n >> 4) << 14) | (0x7 << 4); }
// lgkmcnt = 0 only (vmcnt and expcnt at their no-wait maxima).
constexpr int lgkm0_imm() { return vmcnt_imm(63) & ~(0xF << 8); }

// FLAT: the segments' row tiles form one range (they share the split count), so
// a block may straddle two segments; each row tile reads its own segment's
// weights and goes to its own segment's epilogue. This lets the block height be
// chosen for the grid size (e.g. 12 row tiles: the fused QKV's 192 row tiles in
// 16 blocks) rather than for the segment sizes.
template <class Epi, int WRT, int WLT, int WM, int WN, int KC, int NS, int OCC, bool HASY, bool FLAT = false>
__global__ __launch_bounds__(kWave * WM * WN, OCC) void k_pipe(Geometry g, typename Epi::Out o) {
  constexpr int M = Epi::kMats;
  constexpr int NW = WM * WN;
  constexpr int BR = WM * WRT, BL = WN * WLT;
  constexpr int NBLK = (M * BR + BL) * KC;          // 1 KiB chunks per stage
  static_assert(NBLK % NW == 0, "stage copies must split evenly over the waves");
  constexpr int PER_WAVE = NBLK / NW;               // copy instructions per wave per stage
  constexpr int STAGE = NBLK * kWave;               // u32x4 slots per stage
  __shared__ u32x4 ring[NS * STAGE];

  const int lane = threadIdx.x & (kWave - 1);
  const int wave = threadIdx.x / kWave;
  const int wr = wave / WN, wn = wave % WN;
  const int lblocks = (g.lane_groups + BL - 1) / BL;

  // Block -> (segment, row block, lane block): groups of G row blocks walk the
  // lane blocks together so that consecutive workgroups (which the hardware puts
  // on one XCD after xcd_remap) share activation tiles in L2.
  int b = xcd_remap(blockIdx.x, gridDim.x);
  const int si = FLAT ? 0 : locate_segment(g, b, lblocks);
  const Segment sg = seg_at(g, si);
  // Row tiles of this block's range (FLAT: all segments; the host sets
  // seg[0].blocks to the row blocks of the whole range).
  const int total = FLAT ? g.seg[0].row_tiles + g.seg[1].row_tiles + g.seg[2].row_tiles : sg.row_tiles;
  constexpr int G = 8;
  const int group = b / (G * lblocks);
  const int gsize = min(G, sg.blocks - group * G);
  const int within = b % (G * lblocks);
  const int rb = group * G + within % gsize;
  const int lb = within / gsize;
  const int rt0 = rb * BR, lt0 = lb * BL;

  const int chunks = g.col_tiles >> 1;
  const int per = chunks / sg.splits;
  const int nst = chunks / KC;
  const int64_t strip = static_cast<int64_t>(g.col_tiles) * kTileElems;
  const int foff = frag_offset(lane);

  // This wave's copy sources: block j = wave + i*NW of each stage.
  const char* src[PER_WAVE];
#pragma unroll
  for (int i = 0; i < PER_WAVE; ++i) {
    const int j = wave + i * NW;
    const int kc = j % KC, blk = j / KC;
    const uint16_t* base;
    if (blk < M * BR) {
      const int m = blk / BR;
      const int rt = min(rt0 + blk % BR, total - 1);
      if constexpr (FLAT) {
        int local = 0;
        const Segment ss = seg_at(g, flat_segment(g, rt, local));
        base = (m == 0 ? ss.w[0] : ss.w[1]) + local * strip;
      } else {
        base = (m == 0 ? sg.w[0] : sg.w[1]) + rt * strip;  // no run-time index into sg
      }
    } else {
      const int lt = min(lt0 + blk - M * BR, g.lane_groups - 1);
      base = g.x + lt * strip;
    }
    src[i] = reinterpret_cast<const char*>(base) + static_cast<int64_t>(kc) * kChunkBytes + foff;
  }
  auto issue = [&](int stage) {
    u32x4* dst = ring + (stage % NS) * STAGE;
#pragma unroll
    for (int i = 0; i < PER_WAVE; ++i) {
      const int j = wave + i * NW;
      __builtin_amdgcn_global_load_lds(STRIDE_TC_GLOBAL(src[i] + static_cast<int64_t>(stage) * KC * kChunkBytes),
                                       STRIDE_TC_LDS(dst + j * kWave), 16, 0, 0);
    }
  };

  // Fragments are double-buffered by chunk parity. With an odd chunk count per
  // stage the parity flips from stage to stage, so stages are processed in pairs
  // (the host only selects such a configuration when every split has an even
  // number of stages).
  constexpr bool kPairStages = KC % 2 != 0;
  f32x4 acc[M][WRT][WLT];
  f32x4 y[HASY ? M : 1][HASY ? WRT : 1][HASY ? WLT : 1];
  u32x4 fa[2][M][WRT], fb[2][WLT];  // fragments of the current and the next chunk

  auto read_frags = [&](int buf, int stage, int kc) {
    const u32x4* stg = ring + (stage % NS) * STAGE;
#pragma unroll
    for (int m = 0; m < M; ++m)
#pragma unroll
      for (int r = 0; r < WRT; ++r) fa[buf][m][r] = stg[((m * BR + wr * WRT + r) * KC + kc) * kWave + lane];
#pragma unroll
    for (int l = 0; l < WLT; ++l) fb[buf][l] = stg[((M * BR + wn * WLT + l) * KC + kc) * kWave + lane];
  };
  // Wait until stage `next` has landed everywhere (later stages may stay in
  // flight) and this wave's LDS reads have returned, then barrier.
  auto sync_for = [&](int next) {
    const int ahead = min(NS - 2, nst - 1 - next);
    if (ahead >= NS - 2) __builtin_amdgcn_s_waitcnt(vm_lgkm0_imm((NS - 2) * PER_WAVE));
    else if (ahead == 2) __builtin_amdgcn_s_waitcnt(vm_lgkm0_imm(2 * PER_WAVE));
    else if (ahead == 1) __builtin_amdgcn_s_waitcnt(vm_lgkm0_imm(PER_WAVE));
    else __builtin_amdgcn_s_waitcnt(vm_lgkm0_imm(0));
    __builtin_amdgcn_s_barrier();
  };

#pragma unroll
  for (int st = 0; st < NS; ++st)
    if (st < nst) issue(st);
  sync_for(0);
  read_frags(0, 0, 0);

  // One stage: KC chunks; the fragments of chunk kc+1 are read while chunk kc's
  // MFMAs run. Before the last chunk, the wave waits for stage i+1, hands stage
  // i's slot back to the copy engine and starts reading stage i+1.
  auto stage = [&](int i, auto parity) {
#pragma unroll
    for (int kc = 0; kc < KC; ++kc) {
      const int cur = (decltype(parity)::value + kc) & 1, nxt = cur ^ 1;
      // This step's fragments were read during the previous step.
      __builtin_amdgcn_s_waitcnt(lgkm0_imm());
      const bool last = kc + 1 == KC;
      if (last && i + 1 < nst) {
        sync_for(i + 1);
        if (i + NS < nst) issue(i + NS);
      }
      // Read the next chunk's fragments (after the final chunk: a harmless
      // re-read of the current stage) in one straight block with this chunk's
      // MFMAs, interleaved so that LDS reads and the matrix pipe overlap.
      read_frags(nxt, last ? min(i + 1, nst - 1) : i, last ? 0 : kc + 1);
#pragma unroll
      for (int l = 0; l < WLT; ++l)
#pragma unroll
        for (int m = 0; m < M; ++m)
#pragma unroll
          for (int r = 0; r < WRT; ++r) acc[m][r][l] = mfma(fa[cur][m][r], fb[cur][l], acc[m][r][l]);
      constexpr int kReads = M * WRT + WLT, kMfma = M * WRT * WLT;
#pragma unroll
      for (int q = 0; q < kReads; ++q) {
        __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);               // one ds_read
        __builtin_amdgcn_sched_group_barrier(0x008, kMfma / kReads, 0);  // MFMAs
      }
      if constexpr (kMfma % kReads != 0) __builtin_amdgcn_sched_group_barrier(0x008, kMfma % kReads, 0);
    }
  };

  const int stages_per_split = per / KC;
  int i = 0;
  for (int s = 0; s < sg.splits; ++s) {
#pragma unroll
    for (int m = 0; m < M; ++m)
#pragma unroll
      for (int r = 0; r < WRT; ++r)
#pragma unroll
        for (int l = 0; l < WLT; ++l) {
          acc[m][r][l] = f32x4{0.f, 0.f, 0.f, 0.f};
          if constexpr (Epi::kInitFromOutput) {
            const int rt = rt0 + wr * WRT + r, lt = lt0 + wn * WLT + l;
            int local = rt;
            if constexpr (FLAT) flat_segment(g, rt, local);
            if (s == 0 && rt < total && lt < g.lane_groups) acc[m][r][l] = Epi::init(o, local, lt, lane);
          }
        }
    if constexpr (kPairStages) {
      for (int j = 0; j < stages_per_split; j += 2, i += 2) {
        stage(i, std::integral_constant<int, 0>{});
        stage(i + 1, std::integral_constant<int, 1>{});
      }
    } else {
      for (int j = 0; j < stages_per_split; ++j, ++i) stage(i, std::integral_constant<int, 0>{});
    }
    if constexpr (HASY) {
#pragma unroll
      for (int m = 0; m < M; ++m)
#pragma unroll
        for (int r = 0; r < WRT; ++r)
#pragma unroll
          for (int l = 0; l < WLT; ++l) y[m][r][l] = s == 0 ? acc[m][r][l] : y[m][r][l] + acc[m][r][l];
    }
  }

  if constexpr (Epi::kReduce) {
    // Merge this workgroup's row tiles per batch lane, then one update per lane.
    __syncthreads();  // the LDS ring is reused for the candidates
    float* cand_v = reinterpret_cast<float*>(ring);
    int32_t* cand_i = reinterpret_cast<int32_t*>(ring) + WM * BL * 16;
#pragma unroll
    for (int l = 0; l < WLT; ++l) {
      float bv = f32_of(0xFF800000u);
      int32_t bi = -1;
#pragma unroll
      for (int r = 0; r < WRT; ++r) {
        const int rt = rt0 + wr * WRT + r;
        if (rt >= total) continue;
        int local = rt;
        if constexpr (FLAT) flat_segment(g, rt, local);
        if constexpr (HASY) Epi::merge_tile(o, local, y[0][r][l], lane, bv, bi);
        else Epi::merge_tile(o, local, acc[0][r][l], lane, bv, bi);
      }
      if (lane < 16) {
        cand_v[(wr * BL + wn * WLT + l) * 16 + lane] = bv;
        cand_i[(wr * BL + wn * WLT + l) * 16 + lane] = bi;
      }
    }
    __syncthreads();
    if (wr == 0) {
#pragma unroll
      for (int l = 0; l < WLT; ++l) {
        const int lt = lt0 + wn * WLT + l;
        if (lt >= g.lane_groups) continue;
        float v = f32_of(0xFF800000u);
        int32_t i = -1;
#pragma unroll
        for (int w = 0; w < WM; ++w)
          arg_merge(v, i, cand_v[(w * BL + wn * WLT + l) * 16 + (lane & 15)], cand_i[(w * BL + wn * WLT + l) * 16 + (lane & 15)]);
        Epi::commit(o, g, lt, lane, v, i, rb);
      }
    }
    return;
  }
  unroll<WRT>([&](auto r) {
    const int rt = rt0 + wr * WRT + r;
    if (rt >= total) return;
    int local = rt, seg = si;
    if constexpr (FLAT) seg = flat_segment(g, rt, local);
    unroll<WLT>([&](auto l) {
      const int lt = lt0 + wn * WLT + l;
      if (lt >= g.lane_groups) return;
      f32x4 t[M];
#pragma unroll
      for (int m = 0; m < M; ++m) {
        if constexpr (HASY) t[m] = y[m][r][l];
        else t[m] = acc[m][r][l];
      }
      Epi::apply(o, g, seg, local, lt, t, lane);
    });
  });
}


// The same pipeline with v_mfma_f32_32x32x16_bf16: each wave owns WRT/2 x WLT/2
// blocks of 32 rows x 32 lanes, and a 32-column chunk is two MFMAs per block
// (columns 0-15, then 16-31), which gives the bits of the 16x16x32 form (see
// mfma32) at half the instruction count - the form that keeps the matrix pipe
// busy at one or two waves per SIMD. The LDS staging is unchanged: a lane reads
// the 16 bytes of its 32x32x16 fragment (row or lane l%32 of the pair of tiles,
// k half h, k group l/32) from the 16x16x32 fragment order of its tile's chunk.
// Accumulators enter (h for the residual) and leave (the epilogues) as 16x16
// tiles, converted with cross-lane shuffles.
template <class Epi, int WRT, int WLT, int WM, int WN, int KC, int NS, int OCC, bool HASY>
__global__ __launch_bounds__(kWave * WM * WN, OCC) void k_pipe32(Geometry g, typename Epi::Out o) {
  static_assert(WRT % 2 == 0 && WLT % 2 == 0, "32x32 blocks need even tile counts per wave");
  constexpr int M = Epi::kMats;
  constexpr int NW = WM * WN;
  constexpr int BR = WM * WRT, BL = WN * WLT;
  constexpr int PR = WRT / 2, PL = WLT / 2;         // 32x32 blocks per wave (rows, lanes)
  constexpr int NBLK = (M * BR + BL) * KC;          // 1 KiB chunks per stage
  static_assert(NBLK % NW == 0, "stage copies must split evenly over the waves");
  constexpr int PER_WAVE = NBLK / NW;
  constexpr int STAGE = NBLK * kWave;
  __shared__ u32x4 ring[NS * STAGE];

  const int lane = threadIdx.x & (kWave - 1);
  const int wave = threadIdx.x / kWave;
  const int wr = wave / WN, wn = wave % WN;
  const int lblocks = (g.lane_groups + BL - 1) / BL;

  int b = xcd_remap(blockIdx.x, gridDim.x);
  const int si = locate_segment(g, b, lblocks);
  const Segment sg = seg_at(g, si);
  constexpr int G = 8;
  const int group = b / (G * lblocks);
  const int gsize = min(G, sg.blocks - group * G);
  const int within = b % (G * lblocks);
  const int rb = group * G + within % gsize;
  const int lb = within / gsize;
  const int rt0 = rb * BR, lt0 = lb * BL;

  const int chunks = g.col_tiles >> 1;
  const int per = chunks / sg.splits;
  const int nst = chunks / KC;
  const int64_t strip = static_cast<int64_t>(g.col_tiles) * kTileElems;
  const int foff = frag_offset(lane);

  const char* src[PER_WAVE];
#pragma unroll
  for (int i = 0; i < PER_WAVE; ++i) {
    const int j = wave + i * NW;
    const int kc = j % KC, blk = j / KC;
    const uint16_t* base;
    if (blk < M * BR) {
      const int m = blk / BR;
      const int rt = min(rt0 + blk % BR, sg.row_tiles - 1);
      base = (m == 0 ? sg.w[0] : sg.w[1]) + rt * strip;
    } else {
      const int lt = min(lt0 + blk - M * BR, g.lane_groups - 1);
      base = g.x + lt * strip;
    }
    src[i] = reinterpret_cast<const char*>(base) + static_cast<int64_t>(kc) * kChunkBytes + foff;
  }
  auto issue = [&](int stage) {
    u32x4* dst = ring + (stage % NS) * STAGE;
#pragma unroll
    for (int i = 0; i < PER_WAVE; ++i) {
      const int j = wave + i * NW;
      __builtin_amdgcn_global_load_lds(STRIDE_TC_GLOBAL(src[i] + static_cast<int64_t>(stage) * KC * kChunkBytes),
                                       STRIDE_TC_LDS(dst + j * kWave), 16, 0, 0);
    }
  };

  constexpr bool kPairStages = KC % 2 != 0;
  f32x16 acc[M][PR][PL];
  f32x16 y[HASY ? M : 1][HASY ? PR : 1][HASY ? PL : 1];
  u32x4 fa[2][2][M][PR], fb[2][2][PL];  // [chunk parity][k half]
  // This lane's piece inside a pair of tiles' chunks: tile (lane/16)%2 of the
  // pair, 16x16x32 fragment slot (2h + lane/32)*16 + lane%16.
  const int poff = ((lane >> 4) & 1) * KC * kWave + (lane >> 5) * 16 + (lane & 15);

  auto read_frags = [&](int buf, int stage, int kc) {
    const u32x4* stg = ring + (stage % NS) * STAGE + poff;
#pragma unroll
    for (int h = 0; h < 2; ++h) {
#pragma unroll
      for (int m = 0; m < M; ++m)
#pragma unroll
        for (int p = 0; p < PR; ++p) fa[buf][h][m][p] = stg[((m * BR + wr * WRT + 2 * p) * KC + kc) * kWave + 32 * h];
#pragma unroll
      for (int q = 0; q < PL; ++q) fb[buf][h][q] = stg[((M * BR + wn * WLT + 2 * q) * KC + kc) * kWave + 32 * h];
    }
  };
  auto sync_for = [&](int next) {
    const int ahead = min(NS - 2, nst - 1 - next);
    if (ahead >= NS - 2) __builtin_amdgcn_s_waitcnt(vm_lgkm0_imm((NS - 2) * PER_WAVE));
    else if (ahead == 2) __builtin_amdgcn_s_waitcnt(vm_lgkm0_imm(2 * PER_WAVE));
    else if (ahead == 1) __builtin_amdgcn_s_waitcnt(vm_lgkm0_imm(PER_WAVE));
    else __builtin_amdgcn_s_waitcnt(vm_lgkm0_imm(0));
    __builtin_amdgcn_s_barrier();
  };

#pragma unroll
  for (int st = 0; st < NS; ++st)
    if (st < nst) issue(st);
  sync_for(0);
  read_frags(0, 0, 0);

  auto stage = [&](int i, auto parity) {
#pragma unroll
    for (int kc = 0; kc < KC; ++kc) {
      const int cur = (decltype(parity)::value + kc) & 1, nxt = cur ^ 1;
      __builtin_amdgcn_s_waitcnt(lgkm0_imm());
      const bool last = kc + 1 == KC;
      if (last && i + 1 < nst) {
        sync_for(i + 1);
        if (i + NS < nst) issue(i + NS);
      }
      read_frags(nxt, last ? min(i + 1, nst - 1) : i, last ? 0 : kc + 1);
#pragma unroll
      for (int h = 0; h < 2; ++h)
#pragma unroll
        for (int q = 0; q < PL; ++q)
#pragma unroll
          for (int m = 0; m < M; ++m)
#pragma unroll
            for (int p = 0; p < PR; ++p) acc[m][p][q] = mfma32(fa[cur][h][m][p], fb[cur][h][q], acc[m][p][q]);
      constexpr int kReads = 2 * (M * PR + PL), kMfma = 2 * M * PR * PL;
      constexpr int kPer = kMfma / kReads > 0 ? kMfma / kReads : 1;
#pragma unroll
      for (int r = 0; r < kReads; ++r) {
        __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);     // one ds_read
        __builtin_amdgcn_sched_group_barrier(0x008, kPer, 0);  // MFMAs
      }
    }
  };

  const int stages_per_split = per / KC;
  int i = 0;
  for (int s = 0; s < sg.splits; ++s) {
#pragma unroll
    for (int m = 0; m < M; ++m)
#pragma unroll
      for (int p = 0; p < PR; ++p)
#pragma unroll
        for (int q = 0; q < PL; ++q) {
          if constexpr (Epi::kInitFromOutput) {
            if (s == 0) {
              f32x4 t[2][2];
#pragma unroll
              for (int a = 0; a < 2; ++a)
#pragma unroll
                for (int bb = 0; bb < 2; ++bb) {
                  const int rt = rt0 + wr * WRT + 2 * p + a, lt = lt0 + wn * WLT + 2 * q + bb;
                  t[a][bb] = rt < sg.row_tiles && lt < g.lane_groups ? Epi::init(o, rt, lt, lane) : f32x4{0.f, 0.f, 0.f, 0.f};
                }
              acc[m][p][q] = block_of_tiles(t, lane);
              continue;
            }
          }
          acc[m][p][q] = f32x16{};
        }
    if constexpr (kPairStages) {
      for (int j = 0; j < stages_per_split; j += 2, i += 2) {
        stage(i, std::integral_constant<int, 0>{});
        stage(i + 1, std::integral_constant<int, 1>{});
      }
    } else {
      for (int j = 0; j < stages_per_split; ++j, ++i) stage(i, std::integral_constant<int, 0>{});
    }
    if constexpr (HASY) {
#pragma unroll
      for (int m = 0; m < M; ++m)
#pragma unroll
        for (int p = 0; p < PR; ++p)
#pragma unroll
          for (int q = 0; q < PL; ++q) y[m][p][q] = s == 0 ? acc[m][p][q] : y[m][p][q] + acc[m][p][q];
    }
  }

  auto block = [&](int m, int p, int q) -> const f32x16& {
    if constexpr (HASY) return y[m][p][q];
    else return acc[m][p][q];
  };
  if constexpr (Epi::kReduce) {
    __syncthreads();  // the LDS ring is reused for the candidates
    float* cand_v = reinterpret_cast<float*>(ring);
    int32_t* cand_i = reinterpret_cast<int32_t*>(ring) + WM * BL * 16;
    unroll<PL>([&](auto q) {
      unroll<2>([&](auto bb) {
        float bv = f32_of(0xFF800000u);
        int32_t bi = -1;
        unroll<PR>([&](auto p) {
          unroll<2>([&](auto a) {
            const f32x4 t = tile_of_block(block(0, p, q), a, bb, lane);
            const int rt = rt0 + wr * WRT + 2 * p + a;
            if (rt < sg.row_tiles) Epi::merge_tile(o, rt, t, lane, bv, bi);
          });
        });
        const int l = 2 * q + bb;
        if (lane < 16) {
          cand_v[(wr * BL + wn * WLT + l) * 16 + lane] = bv;
          cand_i[(wr * BL + wn * WLT + l) * 16 + lane] = bi;
        }
      });
    });
    __syncthreads();
    if (wr == 0) {
#pragma unroll
      for (int l = 0; l < WLT; ++l) {
        const int lt = lt0 + wn * WLT + l;
        if (lt >= g.lane_groups) continue;
        float v = f32_of(0xFF800000u);
        int32_t ii = -1;
#pragma unroll
        for (int w = 0; w < WM; ++w)
          arg_merge(v, ii, cand_v[(w * BL + wn * WLT + l) * 16 + (lane & 15)], cand_i[(w * BL + wn * WLT + l) * 16 + (lane & 15)]);
        Epi::commit(o, g, lt, lane, v, ii, rb);
      }
    }
    return;
  }
  unroll<PR>([&](auto p) {
    unroll<PL>([&](auto q) {
      unroll<2>([&](auto a) {
        unroll<2>([&](auto bb) {
          f32x4 t[M];
#pragma unroll
          for (int m = 0; m < M; ++m) t[m] = tile_of_block(block(m, p, q), a, bb, lane);
          const int rt = rt0 + wr * WRT + 2 * p + a, lt = lt0 + wn * WLT + 2 * q + bb;
          if (rt < sg.row_tiles && lt < g.lane_groups) Epi::apply(o, g, si, rt, lt, t, lane);
        });
      });
    });
  });
}

}  // namespace stride_tc
