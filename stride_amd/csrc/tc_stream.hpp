// Decode-regime kernel (at most 8 lane tiles, M <= 128): weight streaming.
//
// Workgroup = WS x WR wavefronts. The WS "split waves" each own one K split
// (WS >= the matrix's split count S; waves past S idle), so all splits of a row
// tile run concurrently. The WR "row waves" of one split each own R row tiles,
// so a workgroup covers WR*R row tiles and LT lane tiles. Each wave streams its
// weight chunks straight from HBM into registers (16-byte loads, one 1 KiB chunk
// per wave instruction), double-buffered U chunks at a time. Activation chunks
// come either straight from L2 (XL = false) or, with XL = true, are staged once
// per split group into LDS and shared by its WR row waves, which cuts the L2
// traffic of x by WR*R when many lane tiles are live.
//
// The S split partials are combined in ascending split order through one LDS
// tile buffer: split 0 stores, then split 1 adds, then split 2, ... with a
// barrier between steps, which evaluates ((c0 + c1) + c2) + ... exactly as the
// prefill kernel does in registers.
#pragma once

#include "tc_epilogue.hpp"

namespace stride_tc {

// Largest split count served by cross-workgroup split launches (XS).
constexpr int kMaxXSplits = 8;

// Buffer-instruction cache policy bit sc1 (device-scope coherence on gfx950) and
// word 3 of a raw, untyped buffer resource.
constexpr int kCachePolicySc1 = 16;
constexpr int kRawBufferWord3 = 0x00020000;
// s_waitcnt immediate for vmcnt(0) with expcnt and lgkmcnt left at their
// no-wait maxima.
constexpr int kVmcnt0 = 0x0F70;
typedef int32_t i32x4 __attribute__((ext_vector_type(4)));

// Output-tile and unit bases of segment si for the cross-workgroup split scratch.
__device__ __forceinline__ int xs_tile0(const Geometry& g, int si) {
  int t = 0;
#pragma unroll
  for (int i = 0; i < 2; ++i)
    if (i < si) t += g.seg[i].row_tiles * g.lane_groups;
  return t;
}
__device__ __forceinline__ int xs_unit0(const Geometry& g, int si) {
  int u = 0;
#pragma unroll
  for (int i = 0; i < 2; ++i)
    if (i < si) u += g.seg[i].blocks;
  return u;
}

// Fold of the last arriving workgroup of a cross-workgroup split unit, for a
// split count S known at compile time. Every split's partial tile is loaded back
// (its own too: it was stored before the arrival count, and the copy is
// bit-identical), in batches of up to 16 loads across tiles, so a batch costs
// one memory round trip rather than one per tile; each tile is then folded in
// ascending split order, and the batch's epilogue stores go out together.
template <class Epi, int R, int LT, int S, class Off>
__device__ __forceinline__ void xs_fold(const Geometry& g, const typename Epi::Out& o, int si, const Segment& sg,
                                        int rt_first, int lt0, int nlt, int lane, __amdgpu_buffer_rsrc_t part,
                                        Off offset) {
  constexpr int M = Epi::kMats;
  constexpr int T = R * LT;
  constexpr int TB0 = 16 / (S * M);
  constexpr int TB = TB0 < 1 ? 1 : (TB0 > T ? T : TB0);  // tiles per batch
  unroll<(T + TB - 1) / TB>([&](auto batch) {
    constexpr int t0 = decltype(batch)::value * TB;
    f32x4 pv[TB][S][M];
    unroll<TB>([&](auto i) {
      constexpr int t = t0 + decltype(i)::value;
      if constexpr (t < T) {
        // Tiles past the matrix or the live lanes have no partials (their
        // offsets could lie past the scratch): they load the last live tile's
        // instead, and their sums are discarded. Unconditional loads stay
        // together ahead of the folds.
        const int r = min(rt_first + t / LT, sg.row_tiles - 1) - rt_first;
        const int l = min(t % LT, nlt - 1);
#pragma unroll
        for (int s = 0; s < S; ++s)
#pragma unroll
          for (int m = 0; m < M; ++m)
            pv[decltype(i)::value][s][m] = __builtin_bit_cast(
                f32x4, __builtin_amdgcn_raw_buffer_load_b128(part, offset(r, l, s, m), 0, kCachePolicySc1));
      }
    });
    // All of the batch's loads have landed before the first fold; without this
    // wait the compiler, which cannot tell that the tile conditions are
    // wave-uniform, waits per tile with vmcnt(0) after the previous tile's
    // epilogue store, paying each store's round trip.
    __builtin_amdgcn_s_waitcnt(kVmcnt0);
    f32x4 y[TB][M];
    unroll<TB>([&](auto i) {
#pragma unroll
      for (int m = 0; m < M; ++m) {
        y[decltype(i)::value][m] = pv[decltype(i)::value][0][m];
#pragma unroll
        for (int s = 1; s < S; ++s) y[decltype(i)::value][m] = y[decltype(i)::value][m] + pv[decltype(i)::value][s][m];
      }
    });
    unroll<TB>([&](auto i) {
      constexpr int t = t0 + decltype(i)::value;
      if constexpr (t < T) {
        constexpr int r = t / LT, l = t % LT;
        if (rt_first + r < sg.row_tiles && l < nlt) Epi::apply(o, g, si, rt_first + r, lt0 + l, y[decltype(i)::value], lane);
      }
    });
  });
}

// Finish of a cross-workgroup split launch (one split per workgroup). With a
// single split the tiles are final. Otherwise every workgroup of a (row block,
// lane group) unit publishes its partial tiles with device-coherent stores and
// counts itself in at `cnt`; the last one to arrive folds the splits in
// ascending order, y = ((c0 + c1) + c2) + ..., applies the epilogue and re-arms
// the counter for the next launch. Nothing waits on another workgroup. Rows
// rt_first .. rt_first+R-1 and lane tiles lt0 .. lt0+nlt-1 are this wave's.
template <class Epi, int R, int LT>
__device__ __forceinline__ void xs_finish(const Geometry& g, const typename Epi::Out& o, int si, const Segment& sg,
                                          int rt_first, int lt0, int nlt, int* cnt, int splits, int my_split,
                                          const f32x4 (&acc)[Epi::kMats][R][LT], int lane) {
  constexpr int M = Epi::kMats;
  if (splits == 1) {
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
    return;
  }
  const int tile0 = xs_tile0(g, si);
  // Partial tiles travel as 16-byte buffer stores and loads with the sc1 cache
  // policy, which makes them coherent at device scope across XCDs (the policy
  // the compiler gives agent-scope relaxed atomics on this target), four lanes
  // to a full 64-byte segment. Byte offsets stay below the 16 MiB scratch.
  const __amdgpu_buffer_rsrc_t part = __builtin_amdgcn_make_buffer_rsrc(g.part, 0, 0x7fffffff, kRawBufferWord3);
  auto offset = [&](int r, int l, int s, int m) -> int {
    const int tile = tile0 + (rt_first + r) * g.lane_groups + lt0 + l;
    return (((tile * g.part_splits + s) * M + m) * kWave + lane) * 16;
  };
#pragma unroll
  for (int r = 0; r < R; ++r) {
    if (rt_first + r >= sg.row_tiles) continue;
#pragma unroll
    for (int l = 0; l < LT; ++l) {
      if (l >= nlt) continue;
#pragma unroll
      for (int m = 0; m < M; ++m)
        __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(i32x4, acc[m][r][l]), part, offset(r, l, my_split, m), 0,
                                               kCachePolicySc1);
    }
  }
  // The partial stores are complete (performed at device scope: sc1 stores
  // write through this XCD's L2) before this workgroup is counted, and the last
  // arriver reads them with sc1 loads, which read past its own L1 and L2. That
  // is the ordering an agent-scope release/acquire pair would give; the pair
  // itself is not used because on this target it also writes back and
  // invalidates the whole L2 of the XCD (buffer_wbl2 / buffer_inv sc1), which
  // measured +30 % on the down projection at M = 128 (18.7 -> 24.9 us) while
  // the sc1 traffic already needs neither.
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  __shared__ int last;
  if (threadIdx.x == 0) {
    const int before = __hip_atomic_fetch_add(cnt, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    last = before == splits - 1;
    if (last) __hip_atomic_store(cnt, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  __syncthreads();
  // Compiler ordering only (no cache maintenance at workgroup scope): the
  // partial loads below stay after the barrier that published `last`.
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
  if (!last) return;
  if (splits == 4) {
    xs_fold<Epi, R, LT, 4>(g, o, si, sg, rt_first, lt0, nlt, lane, part, offset);
  } else if (splits == 8) {
    xs_fold<Epi, R, LT, 8>(g, o, si, sg, rt_first, lt0, nlt, lane, part, offset);
  } else {
#pragma unroll
    for (int r = 0; r < R; ++r) {
      if (rt_first + r >= sg.row_tiles) continue;
#pragma unroll
      for (int l = 0; l < LT; ++l) {
        if (l >= nlt) continue;
        f32x4 pv[kMaxXSplits][M];
#pragma unroll
        for (int s = 0; s < kMaxXSplits; ++s) {
          if (s >= splits || s == my_split) continue;
#pragma unroll
          for (int m = 0; m < M; ++m)
            pv[s][m] = __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(part, offset(r, l, s, m), 0, kCachePolicySc1));
        }
        f32x4 y[M];
#pragma unroll
        for (int s = 0; s < kMaxXSplits; ++s) {
          if (s >= splits) continue;
#pragma unroll
          for (int m = 0; m < M; ++m) {
            const f32x4 v = s == my_split ? acc[m][r][l] : pv[s][m];
            y[m] = s == 0 ? v : y[m] + v;
          }
        }
        Epi::apply(o, g, si, rt_first + r, lt0 + l, y, lane);
      }
    }
  }
}

template <class Epi, int R, int LT, int WS, int WR, int UC, bool XLC, bool XS, bool FLAT = false>
__global__ __launch_bounds__(kWave * WS * WR) void k_stream(Geometry g, typename Epi::Out o) {
  static_assert(!XS || (WS == 1 && !Epi::kReduce), "cross-workgroup splits use one split group and a plain epilogue");
  static_assert(!FLAT || (!XS && !Epi::kReduce && !Epi::kInitFromOutput), "flat row blocks serve plain split-group launches");
  constexpr int M = Epi::kMats;
  // UC counts weight chunks in flight per batch; a paired GEMM loads M chunks per step.
  constexpr int U0 = UC / M > 0 ? UC / M : 1;
  // With x staged in LDS, keep the ring (WS groups x 2 buffers x U chunks x LT
  // tiles x 1 KiB) within 128 KiB.
  constexpr int UMAX = XLC ? (128 / (WS * 2 * LT) > 0 ? 128 / (WS * 2 * LT) : 1) : U0;
  constexpr int U = U0 < UMAX ? U0 : UMAX;
  // x staging needs each batch to split evenly over the row waves of a split group.
  constexpr bool XL = XLC && (U * LT) % WR == 0;
  constexpr int kY1 = WR * M * R * LT * kWave;                       // one split's tiles (f32x4 slots)
  // The split partials get a slot each when they fit in 64 KiB: one barrier, then
  // each tile's owner adds them in split order. Otherwise one buffer, the splits
  // adding in turn with a barrier after each.
  constexpr bool kSplitSlots = WS > 1 && !Epi::kReduce && WS * kY1 * 16 <= 64 * 1024;
  constexpr int kY = WS > 1 ? (kSplitSlots ? WS * kY1 : kY1) : 1;      // combine buffer (f32x4 slots)
  constexpr int kX = XL ? WS * 2 * U * LT * kWave : 1;                // x staging (u32x4 slots)
  constexpr int kXPieces = U * LT * kWave;                            // 16-byte pieces per x batch
  constexpr int kXPer = XL ? kXPieces / (WR * kWave) : 1;
  // The x staging ring is dead once the K loop ends, so the combine buffer
  // reuses the same LDS.
  constexpr int kSlots = kY > kX ? kY : kX;
  __shared__ u32x4 smem[kSlots];
  f32x4* ybuf = reinterpret_cast<f32x4*>(smem);
  u32x4* xs = smem;
  // Per-wave argmax candidates (value, index) for the workgroup-level reduction.
  constexpr int kCand = Epi::kReduce ? WS * WR * LT * 16 : 1;
  __shared__ float cand_v[kCand];
  __shared__ int32_t cand_i[kCand];

  const int lane = threadIdx.x & (kWave - 1);
  const int wave = threadIdx.x / kWave;
  const int ws = wave % WS, wr = wave / WS;
  const int lgroups = (g.lane_groups + LT - 1) / LT;
  const int b = xcd_remap(blockIdx.x, gridDim.x);
  int rb = b / lgroups;
  const int lt0 = (b % lgroups) * LT;
  int si = 0, xsplit = 0;
  if constexpr (XS) {
    // Block -> (segment, split, row block, lane group), row blocks fastest, so
    // that neighbouring workgroups (one XCD after xcd_remap) read the same
    // activation chunks.
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
  } else if constexpr (!FLAT) {
    si = locate_segment(g, rb);
  }
  const Segment sg = seg_at(g, si);
  // Row tiles of this block's range (FLAT: the segments laid end to end, which
  // share the split count; the host sets seg[0].blocks to the whole range's row
  // blocks, so a block may straddle two segments).
  const int total = FLAT ? g.seg[0].row_tiles + g.seg[1].row_tiles + g.seg[2].row_tiles : sg.row_tiles;
  const int rt_first = rb * (WR * R) + wr * R;
  const int nlt = min(LT, g.lane_groups - lt0);
  const int chunks = g.col_tiles >> 1;
  const int splits = sg.splits;
  const int per = chunks / splits;
  const int off = frag_offset(lane);
  const int64_t strip = static_cast<int64_t>(g.col_tiles) * kTileElems;
  const bool active = XS || ws < splits;
  const int my_split = XS ? xsplit : ws;

  const char* wp[M][R];
#pragma unroll
  for (int m = 0; m < M; ++m)
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const int rt = min(rt_first + r, total - 1);
      if constexpr (FLAT) {
        int local = 0;
        const Segment ss = seg_at(g, flat_segment(g, rt, local));
        wp[m][r] = reinterpret_cast<const char*>((m == 0 ? ss.w[0] : ss.w[1]) + local * strip) + off;
      } else {
        wp[m][r] = reinterpret_cast<const char*>(sg.w[m] + rt * strip) + off;
      }
    }
  const char* xp[LT];
#pragma unroll
  for (int l = 0; l < LT; ++l) {
    const int lt = min(lt0 + l, g.lane_groups - 1);
    xp[l] = reinterpret_cast<const char*>(g.x + lt * strip) + off;
  }
  // XL staging: thread (wr, lane) of split group ws moves pieces P = i*WR*64 + wr*64 + lane
  // of each batch; piece P is (chunk u, lane tile l, 16-byte slot j).
  const char* xsrc[kXPer];
  int xdst[kXPer];
  if constexpr (XL) {
#pragma unroll
    for (int i = 0; i < kXPer; ++i) {
      const int P = (i * WR + wr) * kWave + lane;
      const int u = P / (LT * kWave), l = (P / kWave) % LT, j = P % kWave;
      const int lt = min(lt0 + l, g.lane_groups - 1);
      xsrc[i] = reinterpret_cast<const char*>(g.x + lt * strip) + static_cast<int64_t>(u) * kChunkBytes + j * 16;
      xdst[i] = (u * LT + l) * kWave + frag_lane_of_piece(j);
    }
  }

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

  // Chunk range of this wave's split (idle waves of a WG with fewer splits run an
  // empty range but still take part in the barriers).
  // The bounds are made wave-uniform (scalar registers): control flow around
  // MFMAs must be scalar branches, because an MFMA ignores the EXEC mask and
  // would still accumulate inside an exec-masked block the compiler chose not
  // to branch around.
  const int c0 = __builtin_amdgcn_readfirstlane(active ? my_split * per : 0);
  const int c1 = __builtin_amdgcn_readfirstlane(active ? c0 + per : 0);
  const int nbatch = (c1 - c0) / U;
  const int cb = c0 + nbatch * U;  // batched range [c0, cb), then single chunks up to c1

  u32x4 a0[U][M][R], a1[U][M][R];
  u32x4 b0[XL ? 1 : U][LT], b1[XL ? 1 : U][LT];
  u32x4 xr[kXPer];
  const int xbase = ws * 2 * U * LT * kWave;

  auto load_w = [&](u32x4 (&a)[U][M][R], int c) {
#pragma unroll
    for (int u = 0; u < U; ++u)
#pragma unroll
      for (int m = 0; m < M; ++m)
#pragma unroll
        for (int r = 0; r < R; ++r) a[u][m][r] = ld_weight(wp[m][r] + static_cast<int64_t>(c + u) * kChunkBytes);
  };
  auto load_x = [&](u32x4 (&bx)[XL ? 1 : U][LT], int c) {
    if constexpr (!XL) {
#pragma unroll
      for (int u = 0; u < U; ++u)
#pragma unroll
        for (int l = 0; l < LT; ++l) bx[u][l] = load16(xp[l] + static_cast<int64_t>(c + u) * kChunkBytes);
    }
  };
  auto fetch_xl = [&](int c) {
    if constexpr (XL) {
#pragma unroll
      for (int i = 0; i < kXPer; ++i) xr[i] = load16(xsrc[i] + static_cast<int64_t>(c) * kChunkBytes);
    }
  };
  auto store_xl = [&](int buf) {
    if constexpr (XL) {
#pragma unroll
      for (int i = 0; i < kXPer; ++i) xs[xbase + buf * U * LT * kWave + xdst[i]] = xr[i];
    }
  };
  auto mma = [&](const u32x4 (&a)[U][M][R], const u32x4 (&bx)[XL ? 1 : U][LT], int buf) {
#pragma unroll
    for (int u = 0; u < U; ++u)
#pragma unroll
      for (int l = 0; l < LT; ++l) {
        // Lane tiles past the live ones read a clamped (valid) tile; their
        // results are discarded. Keeping this loop branch-free lets the compiler
        // wait only for the loads each MFMA needs.
        u32x4 bv;
        if constexpr (XL) bv = xs[xbase + (buf * U * LT + u * LT + l) * kWave + lane];
        else bv = bx[u][l];
#pragma unroll
        for (int m = 0; m < M; ++m)
#pragma unroll
          for (int r = 0; r < R; ++r) acc[m][r][l] = mfma(a[u][m][r], bv, acc[m][r][l]);
      }
  };

  if constexpr (XL) {
    // The host only selects x staging when every split group is active
    // (WS == S for all segments) and U divides the split length.
    const int nb = per / U;
    fetch_xl(c0);
    store_xl(0);
    load_w(a0, c0);
    __syncthreads();
    for (int i = 0; i < nb; ++i) {
      const int buf = i & 1;
      const bool more = i + 1 < nb;
      if (more) fetch_xl(c0 + (i + 1) * U);
      if ((i & 1) == 0) {
        if (more) load_w(a1, c0 + (i + 1) * U);
        mma(a0, b0, buf);
      } else {
        if (more) load_w(a0, c0 + (i + 1) * U);
        mma(a1, b1, buf);
      }
      if (more) store_xl(buf ^ 1);
      __syncthreads();
    }
  } else {
    // Batch b's loads go out while batch b - 1 is multiplied. With few
    // accumulators and small batches (every decode configuration) the loop body
    // runs while two more batches remain, so its loads are unconditional (a load
    // behind a branch makes the compiler's wait before the next MFMAs assume the
    // path without it), and a scheduling barrier keeps each batch's loads ahead
    // of the previous batch's MFMAs. Wider blocks cannot hold both batches and
    // the accumulators in registers that way (they spilled); they keep a loop
    // the compiler may interleave.
    constexpr bool kTwoBatch = R * M * LT * 4 <= 96 && 2 * U * (R * M + LT) * 4 <= 192;
    if (nbatch > 0 && !kTwoBatch) {
      load_w(a0, c0);
      load_x(b0, c0);
      int c = c0;
      for (;;) {
        if (c + U < cb) {
          load_w(a1, c + U);
          load_x(b1, c + U);
        }
        mma(a0, b0, 0);
        c += U;
        if (c >= cb) break;
        if (c + U < cb) {
          load_w(a0, c + U);
          load_x(b0, c + U);
        }
        mma(a1, b1, 0);
        c += U;
        if (c >= cb) break;
      }
    }
    if (nbatch > 0 && kTwoBatch) {
      load_w(a0, c0);
      load_x(b0, c0);
      int c = c0;
      for (; c + 2 * U < cb; c += 2 * U) {
        load_w(a1, c + U);
        load_x(b1, c + U);
        __builtin_amdgcn_sched_barrier(0);
        mma(a0, b0, 0);
        __builtin_amdgcn_sched_barrier(0);
        load_w(a0, c + 2 * U);
        load_x(b0, c + 2 * U);
        __builtin_amdgcn_sched_barrier(0);
        mma(a1, b1, 0);
        __builtin_amdgcn_sched_barrier(0);
      }
      if (c + U < cb) {
        load_w(a1, c + U);
        load_x(b1, c + U);
        __builtin_amdgcn_sched_barrier(0);
        mma(a0, b0, 0);
        mma(a1, b1, 0);
      } else {
        mma(a0, b0, 0);
      }
    }
    for (int c = cb; c < c1; ++c) {  // tail when U does not divide the split
#pragma unroll
      for (int l = 0; l < LT; ++l) {
        const u32x4 bv = load16(xp[l] + static_cast<int64_t>(c) * kChunkBytes);
#pragma unroll
        for (int m = 0; m < M; ++m)
#pragma unroll
          for (int r = 0; r < R; ++r) acc[m][r][l] = mfma(ld_weight(wp[m][r] + static_cast<int64_t>(c) * kChunkBytes), bv, acc[m][r][l]);
      }
    }
  }

  // K = 32 * chunks + 16: the last split ends with a half chunk, the 16 columns
  // of column tile 2 * chunks. Lanes 0..31 hold its k 0..15 (tile 0 of a chunk's
  // fragment layout); lanes 32..63, the MFMA's k 16..31, hold zeros. (The host
  // only selects configurations without x staging for such K.)
  if (__builtin_amdgcn_readfirstlane((g.col_tiles & 1) && active && my_split == splits - 1)) {
    const u32x4 zero = {0u, 0u, 0u, 0u};
    const int64_t tail = static_cast<int64_t>(chunks) * kChunkBytes;
#pragma unroll
    for (int l = 0; l < LT; ++l) {
      const u32x4 bv = lane < 32 ? load16(xp[l] + tail) : zero;
#pragma unroll
      for (int m = 0; m < M; ++m)
#pragma unroll
        for (int r = 0; r < R; ++r) {
          const u32x4 av = lane < 32 ? ld_weight(wp[m][r] + tail) : zero;
          acc[m][r][l] = mfma(av, bv, acc[m][r][l]);
        }
    }
  }

  if constexpr (XS) {
    int* cnt = g.split_cnt + static_cast<int64_t>(xs_unit0(g, si) + rb) * lgroups + (lt0 / LT);
    xs_finish<Epi, R, LT>(g, o, si, sg, rt_first, lt0, nlt, cnt, splits, my_split, acc, lane);
  } else if constexpr (Epi::kReduce) {
    // Candidates of every tile this workgroup owns are merged first; then one
    // wave publishes a single update per batch lane.
    float bv[LT];
    int32_t bi[LT];
#pragma unroll
    for (int l = 0; l < LT; ++l) {
      bv[l] = f32_of(0xFF800000u);
      bi[l] = -1;
    }
    if constexpr (WS == 1) {
#pragma unroll
      for (int r = 0; r < R; ++r) {
        if (rt_first + r >= sg.row_tiles) continue;
#pragma unroll
        for (int l = 0; l < LT; ++l) Epi::merge_tile(o, rt_first + r, acc[0][r][l], lane, bv[l], bi[l]);
      }
    } else {
      for (int s = 0; s < splits; ++s) {
        if (ws == s) {
#pragma unroll
          for (int r = 0; r < R; ++r)
#pragma unroll
            for (int l = 0; l < LT; ++l) {
              f32x4& y = ybuf[((wr * R + r) * LT + l) * kWave + lane];
              y = s == 0 ? acc[0][r][l] : y + acc[0][r][l];
            }
        }
        __syncthreads();
      }
      for (int t = wave; t < WR * R; t += WS * WR) {
        const int twr = t / R, r = t % R;
        const int rt = rb * (WR * R) + twr * R + r;
        if (rt >= sg.row_tiles) continue;
#pragma unroll
        for (int l = 0; l < LT; ++l) Epi::merge_tile(o, rt, ybuf[((twr * R + r) * LT + l) * kWave + lane], lane, bv[l], bi[l]);
      }
    }
    if (lane < 16) {
#pragma unroll
      for (int l = 0; l < LT; ++l) {
        cand_v[(wave * LT + l) * 16 + lane] = bv[l];
        cand_i[(wave * LT + l) * 16 + lane] = bi[l];
      }
    }
    __syncthreads();
    if (wave == 0) {
#pragma unroll
      for (int l = 0; l < LT; ++l) {
        if (l >= nlt) continue;
        float v = f32_of(0xFF800000u);
        int32_t i = -1;
        for (int w = 0; w < WS * WR; ++w) arg_merge(v, i, cand_v[(w * LT + l) * 16 + (lane & 15)], cand_i[(w * LT + l) * 16 + (lane & 15)]);
        Epi::commit(o, g, lt0 + l, lane, v, i, rb);
      }
    }
  } else if constexpr (WS == 1) {
#pragma unroll
    for (int r = 0; r < R; ++r) {
      if (rt_first + r >= total) continue;
      int rt = rt_first + r, ts = si;
      if constexpr (FLAT) ts = flat_segment(g, rt_first + r, rt);
#pragma unroll
      for (int l = 0; l < LT; ++l) {
        if (l >= nlt) continue;
        f32x4 y[M];
#pragma unroll
        for (int m = 0; m < M; ++m) y[m] = acc[m][r][l];
        Epi::apply(o, g, ts, rt, lt0 + l, y, lane);
      }
    }
  } else {
    // Ordered combine: y = c0, then y = y + c1, y = y + c2, ...
    if constexpr (kSplitSlots) {
      if (ws < splits) {
#pragma unroll
        for (int m = 0; m < M; ++m)
#pragma unroll
          for (int r = 0; r < R; ++r)
#pragma unroll
            for (int l = 0; l < LT; ++l) ybuf[ws * kY1 + (((wr * M + m) * R + r) * LT + l) * kWave + lane] = acc[m][r][l];
      }
      __syncthreads();
    } else {
      for (int s = 0; s < splits; ++s) {
        if (ws == s) {
#pragma unroll
          for (int m = 0; m < M; ++m)
#pragma unroll
            for (int r = 0; r < R; ++r)
#pragma unroll
              for (int l = 0; l < LT; ++l) {
                f32x4& y = ybuf[(((wr * M + m) * R + r) * LT + l) * kWave + lane];
                y = s == 0 ? acc[m][r][l] : y + acc[m][r][l];
              }
        }
        __syncthreads();
      }
    }
    for (int t = wave; t < WR * R * LT; t += WS * WR) {
      const int twr = t / (R * LT), r = (t / LT) % R, l = t % LT;
      int rt = rb * (WR * R) + twr * R + r, ts = si;
      if (l >= nlt || rt >= total) continue;
      if constexpr (FLAT) ts = flat_segment(g, rb * (WR * R) + twr * R + r, rt);
      f32x4 y[M];
      const int at = (((twr * M) * R + r) * LT + l) * kWave + lane;
#pragma unroll
      for (int m = 0; m < M; ++m) {
        if constexpr (kSplitSlots) {
          y[m] = ybuf[at + m * R * LT * kWave];
          for (int s = 1; s < splits; ++s) y[m] = y[m] + ybuf[s * kY1 + at + m * R * LT * kWave];
        } else {
          y[m] = ybuf[at + m * R * LT * kWave];
        }
      }
      Epi::apply(o, g, ts, rt, lt0 + l, y, lane);
    }
  }
}

}  // namespace stride_tc
