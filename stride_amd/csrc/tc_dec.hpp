// Decode-regime kernel for many live lane tiles (M up to 128): weights streamed
// HBM -> registers, activations through a shared LDS ring.
//
// A workgroup of NW waves works on LT lane tiles. Its waves form WS split
// groups of NR = NW/WS row waves: group s chains K split s, and row wave r owns
// the R row tiles rb*NR*R + r*R .. +R-1 (x M matrices for the paired gate/up
// GEMM). With WS > 1 the groups' partial tiles are folded in ascending split
// order through LDS at the end; with XS (WS = 1) each workgroup runs one split
// and the last arriving workgroup of a tile group folds the partials; otherwise
// the matrix has a single split.
//
// K is consumed in stages of KC 32-column chunks. Per stage each wave loads its
// own M*R*KC weight chunks straight into registers (one 1 KiB chunk per wave
// instruction, each lane fetching the 16 bytes of its MFMA fragment), and the
// workgroup copies the stage's LT*KC activation chunks into an NSS-slot LDS ring
// with global_load_lds (so the chunk lands in fragment order and every
// ds_read_b128 is linear). Weights are used once, by the wave that loaded them,
// so they never touch LDS; the activations, which every wave needs, are copied
// once per workgroup. NSS stages of weights and activations are in flight per
// wave (NSS-1 while a stage is being multiplied), which keeps enough HBM
// requests outstanding where LT lane tiles of activations would crowd the
// weights out of an LDS ring.
//
// Synchronisation per stage: before its last chunk, the wave waits until its own
// loads of the next stage have landed (s_waitcnt vmcnt with the later stages
// still outstanding), then one s_barrier makes every wave's activation copies of
// that stage visible and guarantees that every wave has read the current slot,
// which is then refilled.
//
// Arithmetic: per output tile, the chunks of the split are chained in ascending
// order by v_mfma_f32_16x16x32_bf16 into an accumulator that starts at zero (at h
// for split 0 of a residual GEMM): the same expression as every other kernel.
#pragma once

#include "tc_pipe.hpp"
#include "tc_stream.hpp"

namespace stride_tc {

template <class Epi, int R, int LT, int NW, int KC, int NSS, bool XS, int WS, int OCC, int WNT>
__global__ __launch_bounds__(kWave * NW, OCC) void k_dec(Geometry g, typename Epi::Out o) {
  static_assert(!(XS && Epi::kReduce), "the argmax epilogue needs whole tiles");
  static_assert(NSS >= 2, "at least one stage in flight");
  static_assert(NW % WS == 0 && (!XS || WS == 1), "split groups divide the waves; XS runs one split");
  constexpr int NR = NW / WS;                    // row waves per split group
  constexpr int M = Epi::kMats;
  constexpr int XCH = LT * KC;                   // activation chunks per stage
  static_assert(XCH % NR == 0, "activation copies must split evenly over a group's waves");
  constexpr int PX = XCH / NR;                   // copy instructions per wave per stage
  constexpr int PW = KC * M * R;                 // weight loads per wave per stage
  constexpr int PB = PX + PW;                    // vector-memory instructions per wave per stage
  static_assert((NSS - 1) * PB <= 63, "vmcnt range");
  constexpr int GSLOT = XCH * kWave;             // u32x4 per ring slot and split group
  constexpr int SLOT = WS * GSLOT;               // u32x4 per ring slot
  // One LDS object per ring slot: the compiler tells distinct objects apart, so
  // a read of one slot does not wait for the copies in flight into the others.
  __shared__ u32x4 ring0[SLOT], ring1[SLOT], ring2[NSS > 2 ? SLOT : 1], ring3[NSS > 3 ? SLOT : 1];
  __shared__ u32x4 ring4[NSS > 4 ? SLOT : 1], ring5[NSS > 5 ? SLOT : 1], ring6[NSS > 6 ? SLOT : 1],
      ring7[NSS > 7 ? SLOT : 1];
  static_assert(NSS <= 8, "at most 8 ring slots");
  auto slot_ptr = [&](auto slot) -> u32x4* {
    constexpr int s = decltype(slot)::value;
    if constexpr (s == 0) return ring0;
    else if constexpr (s == 1) return ring1;
    else if constexpr (s == 2) return ring2;
    else if constexpr (s == 3) return ring3;
    else if constexpr (s == 4) return ring4;
    else if constexpr (s == 5) return ring5;
    else if constexpr (s == 6) return ring6;
    else return ring7;
  };

  const int lane = threadIdx.x & (kWave - 1);
  const int wave = threadIdx.x / kWave;
  const int lgroups = (g.lane_groups + LT - 1) / LT;
  const int b = xcd_remap(blockIdx.x, gridDim.x);
  int rb = b / lgroups;
  const int lt0 = (b % lgroups) * LT;
  int si = 0, xsplit = 0;
  if constexpr (XS) {
    // Block -> (segment, split, row block, lane group), row blocks fastest, so
    // that neighbouring workgroups (one XCD after xcd_remap) share activation
    // chunks in L2.
#pragma unroll
    for (int k = 0; k < 2; ++k) {
      if (si == k && k + 1 < g.nseg && rb >= g.seg[k].blocks * g.seg[k].splits) {
        rb -= g.seg[k].blocks * g.seg[k].splits;
        si = k + 1;
      }
    }
    const int bps = seg_at(g, si).blocks;
    xsplit = rb / bps;
    rb -= xsplit * bps;
  } else {
    si = locate_segment(g, rb);
  }
  const Segment sg = seg_at(g, si);
  const int ws = wave / NR, wr = wave % NR;
  const int rt_first = rb * (NR * R) + wr * R;
  const int nlt = min(LT, g.lane_groups - lt0);
  const int chunks = g.col_tiles >> 1;
  const int splits = sg.splits;
  const int per = chunks / splits;
  const int off = frag_offset(lane);
  const int64_t strip = static_cast<int64_t>(g.col_tiles) * kTileElems;
  // Wave-uniform bounds (scalar registers): an MFMA ignores EXEC, so control
  // flow around MFMAs must be scalar branches.
  const int my_split = XS ? xsplit : ws;
  const int c0 = __builtin_amdgcn_readfirstlane(my_split * per);
  const int nst = __builtin_amdgcn_readfirstlane(per / KC);  // a multiple of NSS (host)

  const char* wp[M][R];
#pragma unroll
  for (int m = 0; m < M; ++m)
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const int rt = min(rt_first + r, sg.row_tiles - 1);
      wp[m][r] = reinterpret_cast<const char*>((m == 0 ? sg.w[0] : sg.w[1]) + rt * strip) +
                 static_cast<int64_t>(c0) * kChunkBytes + off;
    }
  // Activation copy q = wr + t*NR of a group's stage is chunk (kc = q % KC, lane
  // tile q / KC); lane tiles past the live ones copy a clamped (valid) tile whose
  // results are discarded.
  const char* xsrc[PX];
#pragma unroll
  for (int t = 0; t < PX; ++t) {
    const int q = wr + t * NR;
    const int lt = min(lt0 + q / KC, g.lane_groups - 1);
    xsrc[t] = reinterpret_cast<const char*>(g.x + lt * strip) + static_cast<int64_t>(c0 + q % KC) * kChunkBytes + off;
  }

  u32x4 wb[NSS][KC][M][R];
  auto issue_x = [&](int stage, auto slot) {
    u32x4* dst = slot_ptr(slot) + ws * GSLOT;
#pragma unroll
    for (int t = 0; t < PX; ++t)
      __builtin_amdgcn_global_load_lds(STRIDE_TC_GLOBAL(xsrc[t] + static_cast<int64_t>(stage) * KC * kChunkBytes),
                                       STRIDE_TC_LDS(dst + (wr + t * NR) * kWave), 16, 0, 0);
  };
  auto issue_w = [&](int stage, auto slot) {
    constexpr int s = decltype(slot)::value;
#pragma unroll
    for (int kc = 0; kc < KC; ++kc)
#pragma unroll
      for (int m = 0; m < M; ++m)
#pragma unroll
        for (int r = 0; r < R; ++r)
          wb[s][kc][m][r] = ld_weight<WNT>(wp[m][r] + static_cast<int64_t>(stage * KC + kc) * kChunkBytes);
  };

  f32x4 acc[M][R][LT];
#pragma unroll
  for (int m = 0; m < M; ++m)
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
      for (int l = 0; l < LT; ++l) {
        acc[m][r][l] = f32x4{0.f, 0.f, 0.f, 0.f};
        if constexpr (Epi::kInitFromOutput) {
          if (my_split == 0 && l < nlt && rt_first + r < sg.row_tiles) acc[m][r][l] = Epi::init(o, rt_first + r, lt0 + l, lane);
        }
      }

  // Activation fragments, double-buffered by chunk parity.
  u32x4 xf[2][LT];
  auto read_x = [&](int buf, auto slot, int kc) {
    const u32x4* stg = slot_ptr(slot) + ws * GSLOT;
#pragma unroll
    for (int l = 0; l < LT; ++l) xf[buf][l] = stg[(l * KC + kc) * kWave + lane];
  };
  // Wait until this wave's loads of a stage have landed with `ahead` later
  // stages still in flight, then barrier. The scheduling barriers keep the
  // compiler from moving loads across the wait.
  auto sync = [&](auto ahead) {
    __builtin_amdgcn_sched_barrier(0);
    __builtin_amdgcn_s_waitcnt(vm_lgkm0_imm(decltype(ahead)::value * PB));
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_sched_barrier(0);
  };

  // Stage i (ring slot s, fragment parity P): per chunk, the next chunk's
  // fragments are read while this chunk's MFMAs run. At the last chunk the wave
  // first waits for stage i+1 (NEXT: there is one; AHEAD: stages beyond it
  // still in flight), and refills slot s with stage i+NSS (REFILL): the
  // activation copy right after the barrier (every wave has read slot s by
  // then), the weights after the MFMAs that still read them.
  auto stage = [&](int i, auto slot, auto parity, auto next, auto ahead, auto refill) {
    constexpr int s = decltype(slot)::value;
#pragma unroll
    for (int kc = 0; kc < KC; ++kc) {
      const int cur = (decltype(parity)::value + kc) & 1, nxt = cur ^ 1;
      const bool last = kc + 1 == KC;
      __builtin_amdgcn_s_waitcnt(lgkm0_imm());
      if (last) {
        if constexpr (decltype(next)::value) {
          sync(ahead);
          if constexpr (decltype(refill)::value) issue_x(i + NSS, slot);
          read_x(nxt, std::integral_constant<int, (s + 1) % NSS>{}, 0);
        }
      } else {
        read_x(nxt, slot, kc + 1);
      }
#pragma unroll
      for (int l = 0; l < LT; ++l)
#pragma unroll
        for (int m = 0; m < M; ++m)
#pragma unroll
          for (int r = 0; r < R; ++r) acc[m][r][l] = mfma(wb[s][kc][m][r], xf[cur][l], acc[m][r][l]);
      constexpr int kReads = LT, kMfma = M * R * LT;
#pragma unroll
      for (int q = 0; q < kReads; ++q) {
        __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);               // one ds_read
        __builtin_amdgcn_sched_group_barrier(0x008, kMfma / kReads, 0);  // MFMAs
      }
      if constexpr (kMfma % kReads != 0) __builtin_amdgcn_sched_group_barrier(0x008, kMfma % kReads, 0);
    }
    if constexpr (decltype(refill)::value) issue_w(i + NSS, slot);
  };

  static_assert(KC % 2 == 0 || NSS % 2 == 0, "fragment parity must repeat every ring cycle");
  using Yes = std::true_type;
  using No = std::false_type;
  unroll<NSS>([&](auto s) {
    issue_x(s, s);
    issue_w(s, s);
  });
  sync(std::integral_constant<int, NSS - 1>{});
  read_x(0, std::integral_constant<int, 0>{}, 0);
  const int ngroups = nst / NSS;
  for (int grp = 0; grp + 1 < ngroups; ++grp)
    unroll<NSS>([&](auto s) {
      stage(grp * NSS + s, s, std::integral_constant<int, (s * KC) & 1>{}, Yes{}, std::integral_constant<int, NSS - 2>{},
            Yes{});
    });
  // Last ring cycle: nothing left to issue; stage j waits for stage j+1 with
  // NSS-2-j stages behind it.
  unroll<NSS>([&](auto s) {
    constexpr int j = decltype(s)::value;
    constexpr int a = NSS - 2 - j > 0 ? NSS - 2 - j : 0;
    stage((ngroups - 1) * NSS + j, s, std::integral_constant<int, (j * KC) & 1>{},
          std::integral_constant<bool, (j + 1 < NSS)>{}, std::integral_constant<int, a>{}, No{});
  });

  if constexpr (XS) {
    int* cnt = g.split_cnt + static_cast<int64_t>(xs_unit0(g, si) + rb) * lgroups + (lt0 / LT);
    xs_finish<Epi, R, LT>(g, o, si, sg, rt_first, lt0, nlt, cnt, splits, xsplit, acc, lane);
  } else if constexpr (WS > 1) {
    // Ordered fold through LDS, one matrix at a time: group 0 stores, groups
    // 1 .. WS-2 add, and the last group adds its own partial, which evaluates
    // ((c0 + c1) + c2) + ... exactly as the other kernels do; it then runs the
    // epilogue.
    static_assert(NR * R * LT * kWave <= SLOT, "the fold buffer fits one ring slot");
    f32x4* ybuf = reinterpret_cast<f32x4*>(ring0);
    __syncthreads();  // every wave is done with the ring
#pragma unroll
    for (int m = 0; m < M; ++m) {
#pragma unroll
      for (int s = 0; s + 1 < WS; ++s) {
        if (ws == s) {
#pragma unroll
          for (int r = 0; r < R; ++r)
#pragma unroll
            for (int l = 0; l < LT; ++l) {
              f32x4& y = ybuf[((wr * R + r) * LT + l) * kWave + lane];
              y = s == 0 ? acc[m][r][l] : y + acc[m][r][l];
            }
        }
        __syncthreads();
      }
      if (ws == WS - 1) {
#pragma unroll
        for (int r = 0; r < R; ++r)
#pragma unroll
          for (int l = 0; l < LT; ++l) acc[m][r][l] = ybuf[((wr * R + r) * LT + l) * kWave + lane] + acc[m][r][l];
      }
      __syncthreads();
    }
    if (ws == WS - 1) {
#pragma unroll
      for (int r = 0; r < R; ++r) {
        if (rt_first + r >= sg.row_tiles) continue;
#pragma unroll
        for (int l = 0; l < LT; ++l) {
          if (l >= nlt) continue;
          f32x4 y[M];
#pragma unroll
          for (int m = 0; m < M; ++m) y[m] = acc[m][r][l];
          Epi::apply(o, g, si, rt_first + r, lt0 + l, y, lane);
        }
      }
    }
  } else if constexpr (Epi::kReduce) {
    // Per batch lane: this wave's row tiles, then the workgroup's waves, then
    // one update.
    __syncthreads();  // the first ring slot is reused for the candidates
    static_assert(SLOT * 16 >= NW * LT * 16 * 8, "candidates fit one slot");
    float* cand_v = reinterpret_cast<float*>(ring0);
    int32_t* cand_i = reinterpret_cast<int32_t*>(ring0) + NW * LT * 16;
#pragma unroll
    for (int l = 0; l < LT; ++l) {
      float bv = f32_of(0xFF800000u);
      int32_t bi = -1;
#pragma unroll
      for (int r = 0; r < R; ++r) {
        if (rt_first + r >= sg.row_tiles) continue;
        Epi::merge_tile(o, rt_first + r, acc[0][r][l], lane, bv, bi);
      }
      if (lane < 16) {
        cand_v[(wave * LT + l) * 16 + lane] = bv;
        cand_i[(wave * LT + l) * 16 + lane] = bi;
      }
    }
    __syncthreads();
    if (wave == 0) {
#pragma unroll
      for (int l = 0; l < LT; ++l) {
        if (l >= nlt) continue;
        float v = f32_of(0xFF800000u);
        int32_t i = -1;
        for (int w = 0; w < NW; ++w) arg_merge(v, i, cand_v[(w * LT + l) * 16 + (lane & 15)], cand_i[(w * LT + l) * 16 + (lane & 15)]);
        Epi::commit(o, g, lt0 + l, lane, v, i, rb);
      }
    }
  } else {
#pragma unroll
    for (int r = 0; r < R; ++r) {
      if (rt_first + r >= sg.row_tiles) continue;
#pragma unroll
      for (int l = 0; l < LT; ++l) {
        if (l >= nlt) continue;
        f32x4 y[M];
#pragma unroll
        for (int m = 0; m < M; ++m) y[m] = acc[m][r][l];
        Epi::apply(o, g, si, rt_first + r, lt0 + l, y, lane);
      }
    }
  }
}

}  // namespace stride_tc
