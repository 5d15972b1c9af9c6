// Host-side launch selection shared by the GEMM entry points: the split rule,
// argument checks, the configuration tables of every kernel family and run<Epi>,
// which picks a configuration and launches it. Each entry point lives in its own
// translation unit (one epilogue each) so that the library builds in parallel;
// the mutable state (forced configurations, last error, device scratch) is
// defined once, in tc_gemm.hip.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdio>
#include <cstddef>
#include <algorithm>
#include <cstring>
#include <string>

#include "tc_dec.hpp"
#include "tc_epilogue.hpp"
#include "tc_pipe.hpp"
#include "tc_stream.hpp"
#include "tc_tile.hpp"

namespace stride_tc {

extern thread_local std::string g_last_error;
int fail(int code, const std::string& msg);

// ---------------------------------------------------------------------------
// Host side: split rule, validation, launch selection.


// The fixed K-split for an N x K weight matrix. Matrices with few row tiles
// (N <= 4096: Q, K, V, output, down) get 4 splits so that a decode launch has
// enough independent weight streams (measured on MI355X against 2 and 8: at
// M = 128, 8 splits cost 8 % more time on QKV, O and down, 2 splits 5-35 % more;
// prefill is equal or faster with 4); larger ones (gate and up at N = 8192, the
// LM head) get 1: they have row tiles enough for the decode launches, and a
// single split lets the prefill kernels keep one accumulator per tile instead
// of a split partial and a running sum. S is then capped by the chunk count and
// halved until it divides it.
// The split count of matrices with N <= 4096 is a constant of the build (4). A
// library built with another STRIDE_TC_SPLIT_FEW computes other bits, so it is a
// different library; nothing at run time can change it.
#ifndef STRIDE_TC_SPLIT_FEW
#define STRIDE_TC_SPLIT_FEW 4
#endif
constexpr int kSplitFew = STRIDE_TC_SPLIT_FEW;
static_assert(kSplitFew == 1 || kSplitFew == 2 || kSplitFew == 4 || kSplitFew == 8 || kSplitFew == 16,
              "split count of the few-row matrices: 1, 2, 4, 8 or 16");

inline int split_count(int n, int k) {
  const int chunks = k / kChunkCols;
  int s = n <= 4096 ? kSplitFew : 1;
  if (s > chunks) s = chunks;
  while (s > 1 && chunks % s != 0) s >>= 1;
  return s < 1 ? 1 : s;
}

inline bool lanes_ok(const StrideLanes& l, std::string& why) {
  if (l.rows < 0 || l.lane_groups != (l.rows + 15) / 16) {
    why = "lane_groups must equal ceil(rows / 16) (rows=" + std::to_string(l.rows) +
          ", lane_groups=" + std::to_string(l.lane_groups) + ")";
    return false;
  }
  return true;
}

inline bool mat_ok(const StrideGemmMat& m, const char* name, std::string& why) {
  if (!m.w || m.groups <= 0 || m.cols <= 0 || m.cols % 16 != 0) {
    why = std::string(name) + ": need a weight pointer, groups > 0 and cols a positive multiple of 16 (groups=" +
          std::to_string(m.groups) + ", cols=" + std::to_string(m.cols) + ")";
    return false;
  }
  return true;
}

// Decode-regime configurations of k_stream: (R row tiles per wave, LT lane tiles,
// WS split waves, WR row waves, U chunks per batch, XL x staged in LDS, XS one
// split per workgroup, the last arriving workgroup of a tile group combining, F
// flat row blocks over all segments, which may straddle the fused QKV's Q/K/V
// boundaries: each row tile reads its own segment's weights and goes to its own
// segment's epilogue). Which
// one runs never changes results: all evaluate the same chunk order and the same
// split combine. The table is indexed by stride_tc_set_stream_config() for tuning
// sweeps and by pick_decode() otherwise.
#define STRIDE_TC_DECODE_CONFIGS(S) \
  S(0, 1, 1, 8, 1, 8, false, false, false) \
  S(1, 1, 1, 8, 1, 4, false, false, false) \
  S(2, 1, 1, 2, 4, 8, false, false, false) \
  S(3, 1, 1, 1, 8, 8, false, false, false) \
  S(4, 1, 1, 1, 4, 8, false, false, false) \
  S(5, 1, 2, 8, 1, 8, false, false, false) \
  S(6, 1, 2, 2, 4, 8, false, false, false) \
  S(7, 1, 2, 1, 8, 8, false, false, false) \
  S(8, 1, 4, 8, 1, 4, false, false, false) \
  S(9, 2, 4, 8, 1, 2, false, false, false) \
  S(10, 1, 4, 2, 4, 4, false, false, false) \
  S(11, 1, 4, 2, 4, 2, true, false, false) \
  S(12, 1, 4, 1, 8, 4, false, false, false) \
  S(13, 2, 4, 1, 8, 2, true, false, false) \
  S(14, 1, 8, 8, 1, 2, false, false, false) \
  S(15, 2, 8, 8, 1, 2, false, false, false) \
  S(16, 1, 8, 1, 8, 2, true, false, false) \
  S(17, 1, 8, 1, 8, 2, false, false, false) \
  S(18, 1, 1, 16, 1, 4, false, false, false) \
  S(19, 1, 1, 16, 1, 8, false, false, false) \
  S(20, 1, 2, 16, 1, 4, false, false, false) \
  S(21, 1, 4, 16, 1, 2, false, false, false) \
  S(22, 1, 2, 4, 2, 4, false, false, false) \
  S(23, 1, 1, 4, 2, 8, false, false, false) \
  S(24, 1, 4, 4, 2, 4, false, false, false) \
  S(25, 1, 2, 16, 1, 2, false, false, false) \
  S(26, 1, 1, 16, 1, 2, false, false, false) \
  S(27, 2, 4, 8, 1, 4, false, false, false) \
  S(28, 2, 8, 8, 1, 1, false, false, false) \
  S(29, 4, 4, 8, 1, 1, false, false, false) \
  S(30, 4, 8, 8, 1, 1, false, false, false) \
  S(31, 2, 8, 8, 2, 1, true, false, false) \
  S(32, 1, 8, 8, 2, 1, true, false, false) \
  S(33, 2, 2, 8, 1, 4, false, false, false) \
  S(34, 1, 1, 8, 2, 8, false, false, false) \
  S(35, 2, 1, 8, 1, 8, false, false, false) \
  S(36, 1, 4, 2, 4, 8, true, false, false) \
  S(37, 1, 8, 2, 4, 8, true, false, false) \
  S(38, 2, 4, 2, 4, 8, true, false, false) \
  S(39, 1, 8, 1, 8, 4, true, false, false) \
  S(40, 2, 8, 1, 8, 4, true, false, false) \
  S(41, 1, 4, 2, 8, 8, true, false, false) \
  S(42, 2, 8, 2, 4, 4, true, false, false) \
  S(43, 1, 8, 1, 4, 8, true, true, false) \
  S(44, 2, 8, 1, 4, 4, true, true, false) \
  S(45, 1, 8, 1, 8, 8, true, true, false) \
  S(46, 1, 8, 1, 2, 4, true, true, false) \
  S(47, 1, 4, 1, 4, 8, true, true, false) \
  S(48, 2, 4, 1, 4, 4, true, true, false) \
  S(49, 1, 8, 1, 4, 4, true, true, false) \
  S(50, 2, 8, 1, 2, 4, true, true, false) \
  S(51, 4, 8, 1, 2, 2, true, true, false) \
  S(52, 2, 8, 1, 4, 2, true, true, false) \
  S(53, 1, 1, 1, 4, 8, false, true, false) \
  S(54, 1, 1, 1, 8, 8, false, true, false) \
  S(55, 1, 1, 1, 2, 8, false, true, false) \
  S(56, 2, 1, 1, 4, 4, false, true, false) \
  S(57, 1, 2, 1, 4, 8, false, true, false) \
  S(58, 1, 8, 1, 4, 8, false, true, false) \
  S(59, 2, 2, 4, 1, 4, false, false, false) \
  S(60, 3, 2, 8, 1, 4, false, false, true) \
  S(61, 3, 2, 4, 1, 8, false, false, true)

struct DecodeCfg {
  int r, lt, ws, wr, u;
  bool xl, xs, flat;
};

#define STRIDE_TC_ROW(i, R, LT, WS, WR, U, XL, XS, F) {R, LT, WS, WR, U, XL, XS, F},
constexpr DecodeCfg kDecodeCfgs[] = {STRIDE_TC_DECODE_CONFIGS(STRIDE_TC_ROW)};
#undef STRIDE_TC_ROW
constexpr int kNumDecodeCfgs = sizeof(kDecodeCfgs) / sizeof(kDecodeCfgs[0]);

extern int g_forced_cfg;

// Device scratch for two uses: the greedy LM head's argmax candidates (one
// 8-byte (value, index) slot per (row block, batch lane)) and the fp32 split
// partials of cross-workgroup split launches. Fixed file-scope device arrays, so
// the entry points allocate nothing; one set per stream (scratch_for), so
// launches on up to kScratchSets streams of a device may run concurrently.
constexpr int64_t kScratchBytes = int64_t{16} << 20;
constexpr int64_t kCandSlots = kScratchBytes / 8;
constexpr int kSplitUnits = 1 << 16;  // arrival counters of cross-workgroup split launches

// Scratch sets: a launch on stream st uses the set scratch_for(st) returns.
constexpr int kScratchSets = 4;
struct ScratchSet {
  unsigned long long* scratch;
  int32_t* counters;
};
ScratchSet scratch_for(hipStream_t st);
extern int g_last_cfg;  // configuration of the last decode-regime launch (-2: prefill kernel)

template <class Epi, int R, int LT, int WS, int WR, int U, bool XL, bool XS, bool F>
void launch_stream(Geometry g, const typename Epi::Out& o, hipStream_t st) {
  if constexpr ((XS && Epi::kReduce) || (F && (XS || Epi::kReduce || Epi::kInitFromOutput))) {
    return;  // never selected (decode_cfg_fits)
  } else {
    int blocks = 0;
    if constexpr (F) {  // one range of row tiles over all segments
      int total = 0;
      for (int i = 0; i < g.nseg; ++i) total += g.seg[i].row_tiles;
      for (int i = g.nseg; i < 3; ++i) g.seg[i].row_tiles = 0;
      for (int i = 1; i < 3; ++i) g.seg[i].blocks = 0;
      g.seg[0].blocks = blocks = (total + WR * R - 1) / (WR * R);
    } else {
      for (int i = 0; i < g.nseg; ++i) {
        g.seg[i].blocks = (g.seg[i].row_tiles + WR * R - 1) / (WR * R);
        blocks += XS ? g.seg[i].blocks * g.seg[i].splits : g.seg[i].blocks;
      }
    }
    blocks *= (g.lane_groups + LT - 1) / LT;
    hipLaunchKernelGGL((k_stream<Epi, R, LT, WS, WR, U, XL, XS, F>), dim3(blocks), dim3(kWave * WS * WR), 0, st, g, o);
  }
}

template <class Epi>
void launch_decode_cfg(int idx, const Geometry& g, const typename Epi::Out& o, hipStream_t st) {
  switch (idx) {
#define STRIDE_TC_CASE(i, R, LT, WS, WR, U, XL, XS, F)          \
  case i:                                                       \
    launch_stream<Epi, R, LT, WS, WR, U, XL, XS, F>(g, o, st); \
    break;
    STRIDE_TC_DECODE_CONFIGS(STRIDE_TC_CASE)
#undef STRIDE_TC_CASE
    default:
      break;
  }
}

// Output tiles of a launch (all segments).
inline int64_t total_tiles(const Geometry& g) {
  int64_t t = 0;
  for (int i = 0; i < g.nseg; ++i) t += static_cast<int64_t>(g.seg[i].row_tiles) * g.lane_groups;
  return t;
}

// Can configuration c serve this launch?
inline bool decode_cfg_fits(const DecodeCfg& c, Geometry g, int smax, int mats, bool reduce) {
  if (c.xl && (g.col_tiles & 1)) return false;  // a trailing half chunk is read from L2 only
  int u = c.u / mats > 0 ? c.u / mats : 1;
  if (c.xl) {
    const int umax = 128 / (c.ws * 2 * c.lt) > 0 ? 128 / (c.ws * 2 * c.lt) : 1;
    u = u < umax ? u : umax;  // as k_stream clamps it
  }
  const int chunks = g.col_tiles >> 1;
  if (c.flat) {
    if (c.xs || reduce || g.nseg < 2) return false;
    for (int i = 1; i < g.nseg; ++i)
      if (g.seg[i].splits != g.seg[0].splits) return false;
  }
  if (c.xs) {
    if (reduce || c.ws != 1 || smax < 2 || smax > kMaxXSplits) return false;
    if (total_tiles(g) * smax * mats * 1024 > kScratchBytes) return false;
    int64_t units = 0;
    for (int i = 0; i < g.nseg; ++i) units += (g.seg[i].row_tiles + c.wr * c.r - 1) / (c.wr * c.r);
    if (units * ((g.lane_groups + c.lt - 1) / c.lt) > kSplitUnits) return false;
    if (c.xl && (u * c.lt) % c.wr == 0)
      for (int i = 0; i < g.nseg; ++i)
        if ((chunks / g.seg[i].splits) % u != 0) return false;
    return true;
  }
  if (c.ws < smax) return false;
  if (c.xl && (u * c.lt) % c.wr == 0) {
    for (int i = 0; i < g.nseg; ++i)
      if (g.seg[i].splits != c.ws || (chunks / g.seg[i].splits) % u != 0) return false;
  }
  return true;
}

// Configurations of k_dec (weights to registers, activations through an LDS
// ring): (R row tiles per wave, LT lane tiles, NW waves, KC chunks per stage,
// NSS ring slots, XS one split per workgroup, WS split groups per workgroup, OCC
// workgroups per CU the register allocation is bounded for, WNT weight loads with
// the non-temporal hint). Configurations 23-30 repeat 1, 2, 12, 14, 16, 19, 22
// and 7 with plain weight loads, for launches whose lane groups re-read each
// weight chunk from L2 (where the hint costs HBM re-reads). Index 1000 + i in the tuning hook
// selects configuration i.
#define STRIDE_TC_DEC_CONFIGS(D)       \
  D(0, 1, 8, 4, 2, 4, true, 1, 1, 1)     \
  D(1, 1, 8, 4, 1, 8, true, 1, 1, 1)     \
  D(2, 1, 8, 8, 2, 4, true, 1, 1, 1)     \
  D(3, 1, 8, 4, 2, 4, false, 2, 1, 1)    \
  D(4, 1, 8, 4, 2, 4, false, 1, 1, 1)    \
  D(5, 2, 8, 4, 2, 4, false, 1, 1, 1)    \
  D(6, 1, 4, 4, 2, 4, true, 1, 1, 1)     \
  D(7, 1, 4, 4, 1, 8, true, 1, 1, 1)     \
  D(8, 2, 4, 4, 2, 4, false, 1, 1, 1)    \
  D(9, 1, 8, 4, 1, 8, false, 2, 1, 1)    \
  D(10, 1, 4, 4, 2, 4, false, 1, 1, 1)   \
  D(11, 1, 4, 4, 2, 4, false, 2, 1, 1)   \
  D(12, 2, 8, 4, 1, 4, false, 1, 2, 1)   \
  D(13, 1, 4, 4, 1, 8, false, 2, 1, 1)   \
  D(14, 2, 8, 4, 1, 8, false, 1, 1, 1)   \
  D(15, 1, 2, 2, 2, 4, true, 1, 1, 1)    \
  D(16, 1, 8, 4, 1, 4, false, 1, 2, 1)   \
  D(17, 2, 8, 4, 1, 6, false, 1, 2, 1)   \
  D(18, 2, 4, 4, 2, 4, false, 1, 2, 1)   \
  D(19, 4, 4, 4, 1, 4, false, 1, 2, 1)   \
  D(20, 1, 8, 4, 1, 4, false, 2, 2, 1)   \
  D(21, 2, 8, 8, 1, 4, false, 1, 1, 1)   \
  D(22, 1, 10, 4, 2, 4, false, 1, 1, 1) \
  D(23, 1, 8, 4, 1, 8, true, 1, 1, 0)   \
  D(24, 1, 8, 8, 2, 4, true, 1, 1, 0)   \
  D(25, 2, 8, 4, 1, 4, false, 1, 2, 0)  \
  D(26, 2, 8, 4, 1, 8, false, 1, 1, 0)  \
  D(27, 1, 8, 4, 1, 4, false, 1, 2, 0)  \
  D(28, 4, 4, 4, 1, 4, false, 1, 2, 0)  \
  D(29, 1, 10, 4, 2, 4, false, 1, 1, 0) \
  D(30, 1, 4, 4, 1, 8, true, 1, 1, 0)   \
  D(31, 1, 4, 4, 1, 8, false, 1, 1, 1)

struct DecCfg {
  int r, lt, nw, kc, nss;
  bool xs;
  int ws, occ, wnt;
};
#define STRIDE_TC_DEC_ROW(i, R, LT, NW, KC, NSS, XS, WS, OCC, WNT) {R, LT, NW, KC, NSS, XS, WS, OCC, WNT},
constexpr DecCfg kDecCfgs[] = {STRIDE_TC_DEC_CONFIGS(STRIDE_TC_DEC_ROW)};
#undef STRIDE_TC_DEC_ROW
constexpr int kNumDecCfgs = sizeof(kDecCfgs) / sizeof(kDecCfgs[0]);
constexpr int kDecIndexBase = 1000;
extern int g_forced_dec;

inline bool dec_cfg_fits(const DecCfg& c, const Geometry& g, int smax, int mats, bool reduce) {
  if (g.col_tiles & 1) return false;  // whole 32-column chunks only
  const int chunks = g.col_tiles >> 1;
  if (c.xs) {
    if (reduce || smax < 2 || smax > kMaxXSplits) return false;
    if (total_tiles(g) * smax * mats * 1024 > kScratchBytes) return false;
    int64_t units = 0;
    for (int i = 0; i < g.nseg; ++i) units += (g.seg[i].row_tiles + c.nw * c.r - 1) / (c.nw * c.r);
    if (units * ((g.lane_groups + c.lt - 1) / c.lt) > kSplitUnits) return false;
  } else {
    if (reduce && c.ws != 1) return false;
    for (int i = 0; i < g.nseg; ++i)
      if (g.seg[i].splits != c.ws) return false;
  }
  for (int i = 0; i < g.nseg; ++i) {
    const int per = chunks / g.seg[i].splits;
    if (per % c.kc != 0 || (per / c.kc) % c.nss != 0) return false;
  }
  return true;
}

template <class Epi, int R, int LT, int NW, int KC, int NSS, bool XS, int WS, int OCC, int WNT>
void launch_dec(Geometry g, const typename Epi::Out& o, hipStream_t st) {
  if constexpr ((XS || WS > 1) && Epi::kReduce) {
    return;  // never selected (dec_cfg_fits)
  } else {
    constexpr int NR = NW / WS;
    int blocks = 0;
    for (int i = 0; i < g.nseg; ++i) {
      g.seg[i].blocks = (g.seg[i].row_tiles + NR * R - 1) / (NR * R);
      blocks += XS ? g.seg[i].blocks * g.seg[i].splits : g.seg[i].blocks;
    }
    blocks *= (g.lane_groups + LT - 1) / LT;
    hipLaunchKernelGGL((k_dec<Epi, R, LT, NW, KC, NSS, XS, WS, OCC, WNT>), dim3(blocks), dim3(kWave * NW), 0, st, g, o);
  }
}

template <class Epi>
void launch_dec_cfg(int idx, const Geometry& g, const typename Epi::Out& o, hipStream_t st) {
  switch (idx) {
#define STRIDE_TC_DEC_CASE(i, R, LT, NW, KC, NSS, XS, WS, OCC, WNT) \
  case i:                                                            \
    launch_dec<Epi, R, LT, NW, KC, NSS, XS, WS, OCC, WNT>(g, o, st); \
    break;
    STRIDE_TC_DEC_CONFIGS(STRIDE_TC_DEC_CASE)
#undef STRIDE_TC_DEC_CASE
    default:
      break;
  }
}

// Default choice by lane-tile count, split count, segment count and split
// length, from measured sweeps on MI355X (HIP-graph timing, weights rotated past
// the MALL).
inline int pick_decode(int T, int smax, int mats, int nseg, int per) {
  (void)mats;
  if (smax > 8) return T <= 1 ? 18 : (T <= 2 ? 20 : 21);
  if (T <= 1) {
    if (smax == 1) return 4;
    if (smax == 2) return 34;
    return nseg == 1 && per >= 32 ? 53 : 0;  // long splits: one split per workgroup
  }
  if (T <= 2) return smax == 1 ? 7 : (smax == 2 ? 22 : (nseg == 3 ? 5 : 0));
  if (T <= 4) return smax == 1 ? 13 : (smax == 2 ? 27 : (nseg == 3 ? 33 : 5));
  return smax == 1 ? 16 : (smax == 2 ? 36 : (nseg == 3 ? 27 : 33));
}

// Streaming configuration (no x staging) for K = 16 (mod 32), any lane-tile count.
inline int pick_half(int T, int smax) {
  if (smax == 1) return T <= 1 ? 3 : 17;
  if (smax == 2) return T <= 1 ? 2 : 6;
  return T <= 1 ? 0 : 33;
}

template <class Epi, int WRT, int WLT>
int launch_tile(Geometry g, const typename Epi::Out& o, hipStream_t st) {
  int blocks = 0;
  for (int i = 0; i < g.nseg; ++i) {
    g.seg[i].blocks = (g.seg[i].row_tiles + 2 * WRT - 1) / (2 * WRT);
    blocks += g.seg[i].blocks;
  }
  blocks *= (g.lane_groups + 2 * WLT - 1) / (2 * WLT);
  hipLaunchKernelGGL((k_tile<Epi, WRT, WLT>), dim3(blocks), dim3(256), 0, st, g, o);
  return 0;
}

template <class Epi, int WRT, int WLT, int WM, int WN, int KC, int NS, int OCC, int MF32 = 0>
void launch_pipe(Geometry g, const typename Epi::Out& o, int smax, hipStream_t st) {
  constexpr int BR = WM * WRT, BL = WN * WLT;
  int blocks = 0;
  if constexpr (MF32 == 2) {  // FLAT: one range of row tiles over all segments
    int total = 0;
    for (int i = 0; i < g.nseg; ++i) total += g.seg[i].row_tiles;
    for (int i = g.nseg; i < 3; ++i) g.seg[i].row_tiles = 0;
    for (int i = 1; i < 3; ++i) g.seg[i].blocks = 0;
    g.seg[0].blocks = blocks = (total + BR - 1) / BR;
  } else {
    for (int i = 0; i < g.nseg; ++i) {
      g.seg[i].blocks = (g.seg[i].row_tiles + BR - 1) / BR;
      blocks += g.seg[i].blocks;
    }
  }
  blocks *= (g.lane_groups + BL - 1) / BL;
  if constexpr (MF32 == 2) {
    if (smax > 1)
      hipLaunchKernelGGL((k_pipe<Epi, WRT, WLT, WM, WN, KC, NS, OCC, true, true>), dim3(blocks), dim3(kWave * WM * WN), 0, st, g, o);
    else
      hipLaunchKernelGGL((k_pipe<Epi, WRT, WLT, WM, WN, KC, NS, OCC, false, true>), dim3(blocks), dim3(kWave * WM * WN), 0, st, g, o);
  } else if constexpr (MF32) {
    if (smax > 1)
      hipLaunchKernelGGL((k_pipe32<Epi, WRT, WLT, WM, WN, KC, NS, OCC, true>), dim3(blocks), dim3(kWave * WM * WN), 0, st, g, o);
    else
      hipLaunchKernelGGL((k_pipe32<Epi, WRT, WLT, WM, WN, KC, NS, OCC, false>), dim3(blocks), dim3(kWave * WM * WN), 0, st, g, o);
  } else {
    if (smax > 1)
      hipLaunchKernelGGL((k_pipe<Epi, WRT, WLT, WM, WN, KC, NS, OCC, true>), dim3(blocks), dim3(kWave * WM * WN), 0, st, g, o);
    else
      hipLaunchKernelGGL((k_pipe<Epi, WRT, WLT, WM, WN, KC, NS, OCC, false>), dim3(blocks), dim3(kWave * WM * WN), 0, st, g, o);
  }
}

// Prefill configurations of k_pipe: (WRT, WLT, WM, WN, KC, NS, OCC, MF32). For
// the paired gate/up GEMM WRT counts pairs and is halved (two matrices per row
// tile). MF32 = 1 runs k_pipe32 (32x32x16 MFMAs; same bits); MF32 = 2 runs
// k_pipe with FLAT row blocks (blocks may straddle QKV segments; same bits).
// Index -3 - i in the tuning hook selects configuration i.
#define STRIDE_TC_PIPE_CONFIGS(X) \
  X(0, 4, 4, 2, 2, 2, 3, 1, 0) \
  X(1, 4, 4, 4, 2, 2, 2, 1, 0) \
  X(2, 4, 4, 2, 4, 2, 2, 1, 0) \
  X(3, 8, 4, 2, 4, 2, 2, 1, 0) \
  X(4, 4, 8, 4, 2, 2, 2, 1, 0) \
  X(5, 4, 8, 2, 2, 2, 3, 1, 0) \
  X(6, 4, 4, 4, 4, 2, 2, 1, 0) \
  X(7, 8, 4, 2, 2, 2, 3, 1, 0) \
  X(8, 4, 4, 4, 2, 2, 3, 1, 0) \
  X(9, 4, 8, 2, 2, 2, 2, 1, 0) \
  X(10, 4, 2, 1, 4, 2, 4, 1, 0) \
  X(11, 4, 4, 1, 2, 2, 4, 1, 0) \
  X(12, 2, 2, 2, 4, 2, 4, 1, 0) \
  X(13, 2, 4, 1, 2, 2, 4, 1, 0) \
  X(14, 4, 1, 1, 4, 2, 4, 1, 0) \
  X(15, 2, 2, 1, 4, 2, 4, 2, 0) \
  X(16, 4, 2, 2, 2, 2, 4, 1, 0) \
  X(17, 4, 1, 1, 4, 2, 6, 1, 0) \
  X(18, 4, 8, 4, 2, 1, 4, 1, 0) \
  X(19, 4, 8, 4, 2, 1, 5, 1, 0) \
  X(20, 8, 4, 2, 4, 1, 4, 1, 0) \
  X(21, 4, 4, 4, 2, 1, 5, 1, 0) \
  X(22, 4, 4, 4, 2, 1, 6, 1, 0) \
  X(23, 4, 4, 2, 4, 1, 5, 1, 0) \
  X(24, 8, 8, 2, 2, 1, 4, 1, 0) \
  X(25, 4, 8, 2, 2, 1, 6, 1, 0) \
  X(26, 4, 4, 4, 2, 2, 3, 1, 1) \
  X(27, 4, 4, 2, 4, 1, 5, 1, 1) \
  X(28, 4, 4, 2, 4, 2, 3, 1, 0) \
  X(29, 4, 4, 2, 4, 1, 4, 1, 0) \
  X(30, 4, 4, 2, 4, 1, 6, 1, 0) \
  X(31, 4, 8, 2, 2, 1, 4, 1, 0) \
  X(32, 3, 4, 4, 2, 2, 3, 1, 2) \
  X(33, 6, 2, 2, 4, 2, 3, 1, 2) \
  X(34, 4, 2, 2, 4, 2, 3, 1, 0) \
  X(35, 2, 4, 4, 2, 2, 3, 1, 0) \
  X(36, 4, 2, 2, 4, 1, 6, 1, 0) \
  X(37, 2, 4, 4, 2, 1, 6, 1, 0) \
  X(38, 4, 2, 2, 4, 1, 4, 2, 0) \
  X(39, 2, 2, 4, 4, 2, 3, 1, 0)

#define STRIDE_TC_PIPE_ONE(i, WRT, WLT, WM, WN, KC, NS, OCC, MF) +1
constexpr int kNumPipeCfgs = 0 STRIDE_TC_PIPE_CONFIGS(STRIDE_TC_PIPE_ONE);
#undef STRIDE_TC_PIPE_ONE
extern int g_forced_pipe;

template <class Epi>
void launch_pipe_cfg(int idx, const Geometry& g, const typename Epi::Out& o, int smax, hipStream_t st) {
  switch (idx) {
#define STRIDE_TC_PIPE_CASE(i, WRT, WLT, WM, WN, KC, NS, OCC, MF)                                                 \
  case i:                                                                                                         \
    launch_pipe<Epi, (Epi::kMats == 2 ? (WRT > 2 ? WRT / 2 : WRT) : WRT), WLT, WM, WN, KC, NS, OCC, MF>(g, o, smax, st); \
    break;
    STRIDE_TC_PIPE_CONFIGS(STRIDE_TC_PIPE_CASE)
#undef STRIDE_TC_PIPE_CASE
    default:
      break;
  }
}

// Default prefill configuration (from measured sweeps): 256-row x 256-lane tiles
// (8 waves of 4x8) when there are no K splits to carry and enough row tiles;
// 256 x 128 (8 waves of 4x4, splits folded in registers) when the grid still
// fills the CUs; 128 x 128 (4 waves) for small matrices.
inline int pick_pipe(const Geometry& g, int smax) {
  int rows = 0;
  for (int i = 0; i < g.nseg; ++i) rows += g.seg[i].row_tiles;
  if (smax == 1 && rows >= 512) return 4;
  const int blocks_256x128 = ((rows + 15) / 16) * ((g.lane_groups + 7) / 8);
  return blocks_256x128 >= 256 ? 8 : 0;
}

inline bool pipe_cfg_fits(int idx, const Geometry& g) {
  static const int kc[] = {
#define STRIDE_TC_PIPE_KC(i, WRT, WLT, WM, WN, KC, NS, OCC, MF) KC,
      STRIDE_TC_PIPE_CONFIGS(STRIDE_TC_PIPE_KC)
#undef STRIDE_TC_PIPE_KC
  };
  static const int mf[] = {
#define STRIDE_TC_PIPE_MF(i, WRT, WLT, WM, WN, KC, NS, OCC, MF) MF,
      STRIDE_TC_PIPE_CONFIGS(STRIDE_TC_PIPE_MF)
#undef STRIDE_TC_PIPE_MF
  };
  if (g.col_tiles & 1) return false;  // whole 32-column chunks only
  if (mf[idx] == 2)  // FLAT blocks: one split count for every segment
    for (int i = 1; i < g.nseg; ++i)
      if (g.seg[i].splits != g.seg[0].splits) return false;
  const int chunks = g.col_tiles >> 1;
  // An odd chunk count per stage is processed two stages at a time.
  const int step = kc[idx] % 2 ? 2 * kc[idx] : kc[idx];
  for (int i = 0; i < g.nseg; ++i)
    if ((chunks / g.seg[i].splits) % step != 0) return false;
  return true;
}

// Largest lane-tile count served by the streaming kernel.
constexpr int kStreamMaxLaneTiles = 8;

// Row tiles per workgroup of prefill configuration idx.
inline int pipe_rows_per_block(int idx, int mats) {
  static const int wrt[] = {
#define STRIDE_TC_PIPE_WRT(i, WRT, WLT, WM, WN, KC, NS, OCC, MF) WRT,
      STRIDE_TC_PIPE_CONFIGS(STRIDE_TC_PIPE_WRT)
#undef STRIDE_TC_PIPE_WRT
  };
  static const int wm[] = {
#define STRIDE_TC_PIPE_WM(i, WRT, WLT, WM, WN, KC, NS, OCC, MF) WM,
      STRIDE_TC_PIPE_CONFIGS(STRIDE_TC_PIPE_WM)
#undef STRIDE_TC_PIPE_WM
  };
  const int r = mats == 2 && wrt[idx] > 2 ? wrt[idx] / 2 : wrt[idx];  // as launch_pipe_cfg halves it
  return wm[idx] * r;
}

// Automatic choice of kernel family and configuration, from measured sweeps on
// MI355X (HIP-graph timing, weights rotated past the MALL; every choice computes
// the same bits). kind 0: k_stream configuration, kind 1: k_pipe configuration,
// kind 3: k_dec configuration.
struct Pick {
  int kind, idx;
};

// At most 8 lane tiles (sweeps with every weight set rotated past the MALL, at
// least 512 MiB per pass). The register-streamed kernel with an activation ring
// wins for the LM head at up to four and at eight lane tiles, for the paired
// gate/up GEMM at two to four (two split groups per workgroup) and for down at
// two to four (one split per workgroup); otherwise the LDS-pipelined kernel with
// small blocks wins for the LM head and for gate/up from five lane tiles.
inline Pick pick_small(int T, int smax, int mats, int nseg, int per) {
  if (smax == 1 && mats == 2) {  // gate/up (single split): 14.2 / 15.1 / 15.4 / 20.6 us at M = 1 / 32 / 64 / 128
    if (T <= 1) return {0, 34};
    if (T <= 4) return {1, 14};
    // one chunk per stage, eight stages in flight: 0.5-0.7 % faster decode step at
    // M = 128 than two chunks per stage and four stages (configuration 10)
    return {3, 31};
  }
  if (smax == 4) {  // the split rule's few-row matrices; per = chunks per split (down: 64, O and QKV: 16)
    // QKV: 5.7 / 6.5 / 7.9 / 9.3 us at M = 1 / 32 / 64 / 128. From five lane tiles the
    // flat row blocks of three row tiles (straddling the Q/K/V boundaries) fill all
    // 256 CUs with 64 x 4 workgroups (9.3 against 9.7 us for 2-tile blocks at M = 128).
    if (nseg == 3) return {0, T <= 1 ? 0 : (T <= 2 ? 5 : (T <= 4 ? 33 : 60))};
    if (per >= 32) {  // down: 10.3 / 11.6 / 13.8 / 15.7 us at M = 1 / 32 / 64 / 128
      if (T <= 1) return {0, 55};
      // Two lane tiles, two waves, one split per workgroup: 1.5-3 % faster decode
      // steps at M = 32-64 than the streaming kernel (configurations 0 and 5).
      if (T <= 4) return {3, 15};
      // Non-temporal weight loads: in the measured decode step at M = 128 the step is
      // 0.9 % faster than with plain loads (configuration 30, which the same op
      // timed alone prefers: 14.9 against 15.7 us).
      return {3, 7};
    }
    return {0, T <= 2 ? 0 : (T <= 4 ? 5 : 33)};  // O: 5.1 / 5.0 / 5.7 / 7.1 us at M = 1 / 32 / 64 / 128
  }
  if (smax == 1 && T <= 2) return {3, 10};
  if (smax == 1 && T >= 3 && T <= 4) return {3, 8};
  if (smax == 1 && T == 8) return {3, 12};
  if (smax == 1 && T >= 5) return {3, 12};  // LM head at M = 65-128: 101.6 us at M = 96 (pipeline: 117.9)
  if (smax == 1 && T >= 2) return {1, 14};
  if (smax == 2 && mats == 2 && T >= 2 && T <= 4) return {3, 13};
  if (smax == 2 && mats == 2 && T >= 3) return {1, 15};
  if (smax == 8 && nseg == 1 && per >= 32 && T >= 2 && T <= 4) return {3, 7};  // long splits (down), one split per workgroup
  return {0, pick_decode(T, smax, mats, nseg, per)};
}

// More than 8 lane tiles. Matrices with several splits (QKV, O, down) have few row
// tiles and long split chains: up to a few hundred rows the streaming kernel,
// whose waves run the splits side by side, beats the pipeline, which walks them
// one after another; beyond, the pipeline with a block shape per size.
inline Pick pick_large(const Geometry& g, int T, int smax, int mats, int per) {
  if (smax == 1 && mats == 2) {  // gate/up (single split)
    if (T <= 16) return {3, 16};  // 24.6 / 24.1 / 26.1 us at M = 160 / 192 / 256
    if (T <= 20) return {3, 22};  // ten lane tiles per workgroup: 30.1 us at M = 290 (pipeline: 35.5)
    if (T <= 32) return {3, 14};  // 37.9 / 40.5 us at M = 384 / 512
    if (T <= 40) return {3, 16};  // 55.3 us at M = 640 (pipeline: 69.4)
    return {1, 4};                // 256 x 256 blocks: 63.0 / 122.5 / 233.4 us at M = 1024 / 2048 / 4096
  }
  if (smax == 1) {  // LM head: weights to registers at 9-12 and 17-24 lane tiles (M = 160 / 290 / 384:
                    // 150 / 205 / 226 us against 186 / 269 / 263 with the pipeline), 256 x 256 blocks otherwise
    // several lane groups re-read each weight chunk: plain weight loads
    if (T <= 12 || (T > 16 && T <= 20)) return {3, 28};  // 148 / 152 / 216 us at M = 160 / 192 / 290
    if (T > 20 && T <= 24) return {3, 25};               // 239 us at M = 384
    if (T > 32 && T <= 40) return {3, 14};               // 366 us at M = 640 (pipeline: 388)
    return {1, 6};
  }
  if (smax == 2) {
    if (T <= 12) return {1, 12};
    if (T <= 24) return {1, 8};
    if (T <= 48) return {1, 2};
    if (T <= 64) return {1, pick_pipe(g, smax)};
    return {1, 28};
  }
  if (smax == 4) {  // the split rule's few-row matrices (sweeps at M = 160 ... 4096)
    if (g.nseg == 3) {  // fused QKV
      if (T <= 10) return {0, 59};   // four split waves for the four splits: 10.6 us at M = 160 (12.5 with eight)
      if (T <= 19) return {0, 29};   // 12.9 / 13.1 / 13.0 us at M = 192 / 256 / 290
      if (T <= 24) return {1, 15};   // 17.8 us at M = 384
      if (T <= 40) return {1, 12};   // 19.1 / 20.6 us at M = 512 / 640
      if (T <= 80) return {1, 39};   // 16 waves on 128 x 128: 25.2 / 25.9 / 28.3 us at M = 768 / 1024 / 1280
      if (T <= 128) return {1, 33};  // straddling 12-row-tile blocks: 35.9 / 40.3 us at M = 1536 / 2048
      return {1, 38};                // 46.4 / 67.2 / 74.2 us at M = 2560 / 3072 / 4096
    }
    if (per >= 32) {  // down
      if (T <= 16) return {3, 23};   // 22.1 / 22.1 / 23.6 us at M = 160 / 192 / 256
      if (T <= 20) return {3, 24};   // 26.8 us at M = 290
      if (T <= 32) return {3, 2};    // 29.1 / 30.6 us at M = 384 / 512
      if (T <= 56) return {1, 14};   // 49.2 / 49.5 / 51.0 us at M = 640 / 768 / 896
      if (T <= 64) return {0, 30};   // 50.9 us at M = 1024 (pipeline: 54.2)
      if (T <= 128) return {1, 39};  // 75.6 / 75.8 / 78.8 us at M = 1280 / 1536 / 2048
      if (T <= 160) return {1, 33};  // 100.2 us at M = 2560
      return {1, 23};                // 117.3 / 121.5 us at M = 3072 / 4096
    }
    // O
    if (T <= 16) return {0, 27};     // 8.7 / 9.0 / 9.1 us at M = 160 / 192 / 256
    if (T <= 20) return {0, 59};     // 11.9 us at M = 290
    if (T <= 32) return {0, 29};     // 12.6 / 12.6 us at M = 384 / 512
    if (T <= 48) return {1, 14};     // 17.0 / 17.4 us at M = 640 / 768
    if (T <= 64) return {1, 12};     // 18.3 / 18.6 us at M = 896 / 1024 (streaming: 31-32)
    if (T <= 128) return {1, 39};    // 23.9 / 24.1 / 27.1 us at M = 1280 / 1536 / 2048
    if (T <= 160) return {1, 33};    // 34.6 us at M = 2560
    return {1, 28};                  // 39.2 / 44.1 us at M = 3072 / 4096
  }
  if (g.nseg == 3) {  // fused QKV
    if (T <= 12) return {0, 33};
    if (T <= 24) return {0, 29};
    if (T <= 40) return {1, 14};
    // 16 waves on 128 x 128 blocks: 25.6 / 26.1 / 28.2 us at M = 768 / 1024 / 1280
    // (against 33-37); again at M = 2560 (52.4 against 68.1), where it quantizes onto
    // the CUs better than the straddling blocks below.
    if (T <= 80 || (T > 144 && T <= 176)) return {1, 39};
    // 12-row-tile blocks straddling the q/k/v segments: the 192 row tiles make
    // 16 row blocks, 256 workgroups at M = 2048 (the segment-aligned blocks give
    // 192 or 384): 39.0 against 46.5 us at M = 2048, 76.9 against 89.5 at 4096.
    return {1, 33};
  }
  if (per >= 32) {  // long splits (down)
    if (T <= 12 && dec_cfg_fits(kDecCfgs[7], g, smax, 1, false)) return {3, 7};  // one split per workgroup
    if (T <= 12) return {0, 27};
    if (T <= 32) return {0, 29};
    if (T <= 64) return {0, 30};
    if (T <= 128) return {1, 39};  // 16 waves on 128 x 128: 77.6-78.4 against 86-87 us at M = 1280-2048
    if (T <= 160) return {1, 33};  // 12-row-tile blocks: 101 against 164 us at M = 2560
    return {1, 8};                 // 256 x 128 blocks: 123-125 us at M = 3072-4096 (164-167 before)
  }
  if (T <= 12) return {0, 27};
  if (T <= 32) return {0, 29};
  if (T <= 64) return {1, 14};
  if (T <= 128) return {1, 39};  // 16 waves on 128 x 128: 26.0-28.3 against 32.7-35.6 us at M = 1280-2048 (O)
  if (T <= 160) return {1, 33};  // 12-row-tile blocks: 37.4 against 42.3 us at M = 2560
  return {1, 2};
}

// The configuration tables are instantiated once per epilogue and kernel family
// in tc_gemm_inst.hip (compiled once per pair, so the library builds in
// parallel); the entry points' translation units only declare them.
#define STRIDE_TC_EXTERN_TABLES(E)                                                                   \
  extern template void launch_decode_cfg<E>(int, const Geometry&, const E::Out&, hipStream_t);      \
  extern template void launch_dec_cfg<E>(int, const Geometry&, const E::Out&, hipStream_t);         \
  extern template void launch_pipe_cfg<E>(int, const Geometry&, const E::Out&, int, hipStream_t);
STRIDE_TC_EXTERN_TABLES(EpiResidual)
STRIDE_TC_EXTERN_TABLES(EpiLogits)
STRIDE_TC_EXTERN_TABLES(EpiGateUp)
STRIDE_TC_EXTERN_TABLES(EpiArgmax)
STRIDE_TC_EXTERN_TABLES(EpiQkv)
#undef STRIDE_TC_EXTERN_TABLES

template <class Epi>
int run(Geometry g, const typename Epi::Out& o_in, hipStream_t st) {
  if (g.rows == 0) return 0;
  typename Epi::Out o = o_in;
  int smax = 1;
  for (int i = 0; i < g.nseg; ++i) {
    if (g.seg[i].splits > 16) return fail(STRIDE_TC_EINVAL, "split count above 16");
    smax = g.seg[i].splits > smax ? g.seg[i].splits : smax;
  }
  const int T = g.lane_groups;
  int kind = 0, idx = 0, rows_per_block = 0;  // kind 0: streaming, 1: pipe, 2: legacy tile, 3: dec
  const int per = (g.col_tiles >> 1) / smax;
  const bool forced_stream =
      g_forced_cfg >= 0 && decode_cfg_fits(kDecodeCfgs[g_forced_cfg], g, smax, Epi::kMats, Epi::kReduce);
  const bool forced_pipe = g_forced_pipe >= 0 && pipe_cfg_fits(g_forced_pipe, g);
  const bool forced_dec =
      g_forced_dec >= 0 && dec_cfg_fits(kDecCfgs[g_forced_dec], g, smax, Epi::kMats, Epi::kReduce);
  if (forced_dec) {
    kind = 3;
    idx = g_forced_dec;
  } else if (forced_stream) {
    idx = g_forced_cfg;
  } else if (forced_pipe) {
    kind = 1;
    idx = g_forced_pipe;
  } else {
    const Pick p = T <= kStreamMaxLaneTiles ? pick_small(T, smax, Epi::kMats, g.nseg, per) : pick_large(g, T, smax, Epi::kMats, per);
    kind = p.kind;
    idx = p.idx;
    if (g.col_tiles & 1) {
      // K = 16 (mod 32): only the register-streaming kernel reads the trailing
      // half chunk, so every M runs it (same expression for every row).
      kind = 0;
      idx = pick_half(T, smax);
    }
    if (kind == 1 && !pipe_cfg_fits(idx, g)) {
      idx = pick_pipe(g, smax);
      if (!pipe_cfg_fits(idx, g)) idx = 0;
      if (!pipe_cfg_fits(idx, g)) kind = 2;
    }
    if (kind == 3 && !dec_cfg_fits(kDecCfgs[idx], g, smax, Epi::kMats, Epi::kReduce)) {
      kind = 0;
      idx = pick_decode(T, smax, Epi::kMats, g.nseg, per);
    }
    if (kind == 0 && !decode_cfg_fits(kDecodeCfgs[idx], g, smax, Epi::kMats, Epi::kReduce)) {
      // a register-only in-workgroup configuration with a wave per split always fits
      idx = smax == 1 ? 3 : (smax == 2 ? 2 : (smax <= 8 ? 0 : 18));
    }
  }
  if (kind == 0) rows_per_block = kDecodeCfgs[idx].wr * kDecodeCfgs[idx].r;
  if (kind == 1) rows_per_block = pipe_rows_per_block(idx, Epi::kMats);
  if (kind == 3) rows_per_block = kDecCfgs[idx].nw / kDecCfgs[idx].ws * kDecCfgs[idx].r;
  // Greedy LM head: two passes through the candidate scratch when it fits.
  int nrb = 0;
  if constexpr (Epi::kReduce) {
    o.cand = nullptr;
    if (kind != 2 && g.nseg == 1) {
      nrb = (g.seg[0].row_tiles + rows_per_block - 1) / rows_per_block;
      if (static_cast<int64_t>(nrb) * g.rows <= kCandSlots) {
        o.cand = scratch_for(st).scratch;
        if (!o.cand) return fail(STRIDE_TC_EINVAL, "argmax scratch unavailable");
      }
      if (!o.cand) nrb = 0;
      o.nrb = nrb;
    }
  }
  if (kind == 0) {
    g_last_cfg = idx;
    const bool xs = kDecodeCfgs[idx].xs;
    if (xs) {
      const ScratchSet ss = scratch_for(st);
      g.part = reinterpret_cast<float*>(ss.scratch);
      g.split_cnt = ss.counters;
      g.part_splits = smax;
      if (!g.part || !g.split_cnt) return fail(STRIDE_TC_EINVAL, "split scratch unavailable");
    }
    launch_decode_cfg<Epi>(idx, g, o, st);
  } else if (kind == 3) {
    g_last_cfg = kDecIndexBase + idx;
    if (kDecCfgs[idx].xs) {
      const ScratchSet ss = scratch_for(st);
      g.part = reinterpret_cast<float*>(ss.scratch);
      g.split_cnt = ss.counters;
      g.part_splits = smax;
      if (!g.part || !g.split_cnt) return fail(STRIDE_TC_EINVAL, "split scratch unavailable");
    }
    launch_dec_cfg<Epi>(idx, g, o, st);
  } else if (kind == 1) {
    g_last_cfg = -3 - idx;
    launch_pipe_cfg<Epi>(idx, g, o, smax, st);
  } else {
    g_last_cfg = -2;
    if constexpr (Epi::kMats == 2) launch_tile<Epi, 2, 4>(g, o, st);
    else launch_tile<Epi, 4, 4>(g, o, st);
  }
  if constexpr (Epi::kReduce) {
    if (nrb > 0) hipLaunchKernelGGL(k_argmax_finish, dim3(g.rows), dim3(256), 0, st, o.cand, nrb, g.rows, o.best);
  }
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(static_cast<int>(e), std::string("kernel launch failed: ") + hipGetErrorString(e));
  return 0;
}


inline Geometry single(const StrideLanes& l, const uint16_t* x, const StrideGemmMat& m, const uint16_t* w2) {
  Geometry g{};
  g.x = x;
  g.col_tiles = m.cols / 16;
  g.rows = l.rows;
  g.lane_groups = l.lane_groups;
  g.nseg = 1;
  g.seg[0].w[0] = m.w;
  g.seg[0].w[1] = w2;
  g.seg[0].row_tiles = m.groups;
  g.seg[0].splits = split_count(m.groups * 16, m.cols);
  return g;
}

}  // namespace stride_tc
