// Batch-invariant BF16 linear-layer GEMMs for MI355X (gfx950), behind the C ABI
// of include/stride_tc.h. These replace the GEMM kernels of stride's tensor-core
// path (reference src/kernels_tc.cu:347-655): fused QKV + RoPE + KV append,
// GEMM + residual (output / down), paired gate/up + SiLU, LM head + argmax and
// LM head full logits.
//
// Arithmetic contract (identical for every kernel variant below, hence batch
// invariant): for a weight matrix with K columns, K is read in 32-column chunks
// (one v_mfma_f32_16x16x32_bf16 each). The chunks are divided into S contiguous
// splits, S = split_count(N, K) depending on the weight shape only. Each split s
// chains its chunks in ascending order into an fp32 accumulator that starts at
// zero, except split 0 of a residual GEMM, which starts from h. The result is
// y = ((c0 + c1) + c2) + ... + c(S-1), then the epilogue. The reference fixes the
// same kind of tree with kFewRowsWarps (src/kernels_tc.cu:29-32, 462-496).
//
// Two kernel families evaluate that expression:
//   k_stream  decode regime (at most 8 lane tiles, M <= 128): weight-streaming.
//             A workgroup owns WR*R row tiles and up to LT lane tiles; its waves
//             split the K range (WS waves along K), stream weight chunks straight
//             from HBM into registers with 16-byte loads, and combine the S split
//             partials through LDS in ascending split order.
//   k_tile    prefill regime (more than 8 lane tiles): an LDS-staged block GEMM.
//             A 2x2-wave workgroup owns a (2*WRT) x (2*WLT) block of tiles; each
//             32-column chunk of weights and activations is staged through a
//             double-buffered LDS ring, and each wave walks the splits in order,
//             folding a finished split into its running sum in registers.
// Both call the same chunk order, the same MFMA instruction and the same
// epilogue functions, so every output row has the same bits for any M.
#include <hip/hip_runtime.h>

#include <cstdio>
#include <cstddef>
#include <cstring>
#include <string>

#include "tc_common.hpp"

namespace stride_tc {

// ---------------------------------------------------------------------------
// Problem geometry shared by all kernels: up to three row segments (Q, K, V for
// the fused QKV; one otherwise), all consuming the same activation tiles.

struct Segment {
  const uint16_t* w[2];  // second matrix used by the paired gate/up GEMM
  int32_t row_tiles;
  int32_t splits;
  int32_t blocks;        // row blocks of this segment in the current launch
};

struct Geometry {
  const uint16_t* x;
  int32_t col_tiles;
  int32_t rows;
  int32_t lane_groups;
  int32_t nseg;
  Segment seg[3];
};

// Spread consecutive logical blocks over one XCD: hardware hands workgroup i to
// XCD i % 8, so logical neighbours (which share weight or activation tiles) are
// made to land on the same L2. Bijective on [0, n).
__device__ __forceinline__ int xcd_remap(int i, int n) {
  const int full = n & ~7;
  if (i >= full) return i;
  return (i & 7) * (full >> 3) + (i >> 3);
}

__device__ __forceinline__ int locate_segment(const Geometry& g, int& rb) {
  int s = 0;
  while (s + 1 < g.nseg && rb >= g.seg[s].blocks) {
    rb -= g.seg[s].blocks;
    ++s;
  }
  return s;
}

// ---------------------------------------------------------------------------
// Epilogues. Each receives one finished 16x16 tile y (fragment layout: lane l
// holds lane l%16, rows 4*(l/16)+i) per matrix and writes it out. They are
// called by whole wavefronts (QKV and the argmax exchange values across lanes).

struct EpiResidual {  // h <- h + W x   (reference src/kernels_tc.cu:438-501)
  static constexpr int kMats = 1;
  static constexpr bool kInitFromOutput = true;
  struct Out {
    float* h;
    int32_t h_tiles;
  };
  __device__ static float* at(const Out& o, int rt, int lt, int lane) {
    return o.h + (static_cast<int64_t>(lt) * o.h_tiles + rt) * kTileElems + (lane & 15) * 16 + (lane >> 4) * 4;
  }
  __device__ static f32x4 init(const Out& o, int rt, int lt, int lane) {
    return *reinterpret_cast<const f32x4*>(at(o, rt, lt, lane));
  }
  __device__ static void apply(const Out& o, const Geometry&, int, int rt, int lt, const f32x4* y, int lane) {
    *reinterpret_cast<f32x4*>(at(o, rt, lt, lane)) = y[0];
  }
};

struct EpiLogits {  // logits tiles [rt][lt][16 rows][16 lanes]  (src/kernels_tc.cu:632-655)
  static constexpr int kMats = 1;
  static constexpr bool kInitFromOutput = false;
  struct Out {
    float* logits;
  };
  __device__ static f32x4 init(const Out&, int, int, int) { return f32x4{0.f, 0.f, 0.f, 0.f}; }
  __device__ static void apply(const Out& o, const Geometry& g, int, int rt, int lt, const f32x4* y, int lane) {
    float* base = o.logits + (static_cast<int64_t>(rt) * g.lane_groups + lt) * kTileElems + (lane >> 4) * 64 + (lane & 15);
    base[0] = y[0][0];
    base[16] = y[0][1];
    base[32] = y[0][2];
    base[48] = y[0][3];
  }
};

struct EpiGateUp {  // z = bf16(det_silu(W1 x) * (W3 x))  (src/kernels_tc.cu:505-564)
  static constexpr int kMats = 2;
  static constexpr bool kInitFromOutput = false;
  struct Out {
    uint16_t* z;
    int32_t z_tiles;
  };
  __device__ static f32x4 init(const Out&, int, int, int) { return f32x4{0.f, 0.f, 0.f, 0.f}; }
  __device__ static void apply(const Out& o, const Geometry&, int, int rt, int lt, const f32x4* y, int lane) {
    uint32_t b[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float gate = det_silu(y[0][i]);
      b[i] = bf16_rne(gate * y[1][i]);
    }
    u32x2 packed = {b[0] | (b[1] << 16), b[2] | (b[3] << 16)};
    uint16_t* z = o.z + (static_cast<int64_t>(lt) * o.z_tiles + rt) * kTileElems + (lane & 15) * 16 + (lane >> 4) * 4;
    *reinterpret_cast<u32x2*>(z) = packed;
  }
};

struct EpiArgmax {  // per-lane greedy argmax  (src/kernels_tc.cu:590-630)
  static constexpr int kMats = 1;
  static constexpr bool kInitFromOutput = false;
  struct Out {
    StrideBestEntry* best;
    int32_t vocab;
  };
  __device__ static f32x4 init(const Out&, int, int, int) { return f32x4{0.f, 0.f, 0.f, 0.f}; }
  __device__ static void apply(const Out& o, const Geometry& g, int, int rt, int lt, const f32x4* y, int lane) {
    float bv = f32_of(0xFF800000u);
    int32_t bi = -1;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int index = rt * 16 + (lane >> 4) * 4 + i;
      if (index < o.vocab && y[0][i] > bv) {
        bv = y[0][i];
        bi = index;
      }
    }
    // Merge the four row groups of this lane column; the merge is the
    // lexicographic max, so the exchange order does not matter.
#pragma unroll
    for (int sh = 16; sh <= 32; sh <<= 1) {
      const float ov = __shfl_xor(bv, sh);
      const int32_t oi = __shfl_xor(bi, sh);
      if (oi >= 0 && (bi < 0 || better_than(ov, oi, bv, bi))) {
        bv = ov;
        bi = oi;
      }
    }
    const int j = lt * 16 + (lane & 15);
    if (lane < 16 && j < g.rows && bi >= 0) best_update(&o.best[j], bv, bi);
  }
};

struct EpiQkv {  // RoPE + q store + bf16 KV append  (src/kernels_tc.cu:347-432)
  static constexpr int kMats = 1;
  static constexpr bool kInitFromOutput = false;
  struct Out {
    float* q_out;
    int32_t q_stride;
    int32_t layer;
    int32_t head_dim;
    int32_t page_shift;  // log2(tokens per KV page) = log2(group_elems / head_dim)
    StrideKvRef kv;
    const float* rope;
    const int32_t* row_slot;
    const int32_t* row_pos;
  };
  __device__ static f32x4 init(const Out&, int, int, int) { return f32x4{0.f, 0.f, 0.f, 0.f}; }
  __device__ static uint16_t* kv_row(const Out& o, int which, int head, int slot, int pos) {
    const StrideKvRef& kv = o.kv;
    const int64_t block = kv.table[static_cast<int64_t>(slot) * kv.max_blocks + (pos >> o.page_shift)];
    const int token = pos & ((1 << o.page_shift) - 1);
    return static_cast<uint16_t*>(kv.arena) + block * kv.block_elems + o.layer * kv.layer_elems + which * kv.which_elems +
           head * kv.group_elems + static_cast<int64_t>(token) * kv.head_dim;
  }
  __device__ static void apply(const Out& o, const Geometry& g, int kind, int rt, int lt, const f32x4* y, int lane) {
    // Row m (< 8) of the tile pairs with row m + 8: lanes l and l ^ 32.
    float partner[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) partner[i] = __shfl_xor(y[0][i], 32);
    if (lane >= 32) return;
    const int D = o.head_dim;
    const int tiles_per_head = D / 16;
    const int head = rt / tiles_per_head;
    const int d0 = (rt % tiles_per_head) * 8;
    const int half = D / 2;
    const int j = lt * 16 + (lane & 15);
    if (j >= g.rows) return;
    const int pos = o.row_pos[j];
    const int slot = o.row_slot[j];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int d = d0 + (lane >> 4) * 4 + i;
      const float a = y[0][i];
      const float b = partner[i];
      if (kind == 2) {
        uint16_t* dst = kv_row(o, 1, head, slot, pos);
        dst[d] = static_cast<uint16_t>(bf16_rne(a));
        dst[d + half] = static_cast<uint16_t>(bf16_rne(b));
      } else {
        const float* cs = o.rope + (static_cast<int64_t>(pos) * half + d) * 2;
        const float co = cs[0], si = cs[1];
        const float ra = a * co - b * si;
        const float rb = b * co + a * si;
        if (kind == 0) {
          float* q = o.q_out + static_cast<int64_t>(j) * o.q_stride + static_cast<int64_t>(head) * D;
          q[d] = ra;
          q[d + half] = rb;
        } else {
          uint16_t* dst = kv_row(o, 0, head, slot, pos);
          dst[d] = static_cast<uint16_t>(bf16_rne(ra));
          dst[d + half] = static_cast<uint16_t>(bf16_rne(rb));
        }
      }
    }
  }
};

// ---------------------------------------------------------------------------
// Decode regime: weight streaming with an in-workgroup K split.

template <class Epi, int R, int LT, int WS, int WR, int SMAX>
__global__ __launch_bounds__(kWave * WS * WR) void k_stream(Geometry g, typename Epi::Out o) {
  constexpr int M = Epi::kMats;
  constexpr int U = (LT >= 8 || M * R >= 4) ? 2 : 4;  // chunks in flight per wave
  constexpr int kPart = SMAX > 1 ? SMAX * WR * M * R * LT * kWave : 1;
  __shared__ f32x4 part[kPart];

  const int lane = threadIdx.x & (kWave - 1);
  const int wave = threadIdx.x / kWave;
  const int ws = wave % WS, wr = wave / WS;
  const int lgroups = (g.lane_groups + LT - 1) / LT;
  const int b = xcd_remap(blockIdx.x, gridDim.x);
  int rb = b / lgroups;
  const int lt0 = (b % lgroups) * LT;
  const int si = locate_segment(g, rb);
  const Segment& sg = g.seg[si];
  const int rt_first = rb * (WR * R) + wr * R;
  const int nlt = min(LT, g.lane_groups - lt0);
  const int chunks = g.col_tiles >> 1;
  const int splits = sg.splits;
  const int per = chunks / splits;
  const int off = frag_offset(lane);
  const int64_t strip = static_cast<int64_t>(g.col_tiles) * kTileElems;  // elements per row-tile strip

  const char* wp[M][R];
#pragma unroll
  for (int m = 0; m < M; ++m)
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const int rt = min(rt_first + r, sg.row_tiles - 1);
      wp[m][r] = reinterpret_cast<const char*>(sg.w[m] + rt * strip) + off;
    }
  const char* xp[LT];
#pragma unroll
  for (int l = 0; l < LT; ++l) {
    const int lt = min(lt0 + l, g.lane_groups - 1);
    xp[l] = reinterpret_cast<const char*>(g.x + lt * strip) + off;
  }

  for (int s = ws; s < splits; s += WS) {
    f32x4 acc[M][R][LT];
#pragma unroll
    for (int m = 0; m < M; ++m)
#pragma unroll
      for (int r = 0; r < R; ++r)
#pragma unroll
        for (int l = 0; l < LT; ++l) {
          acc[m][r][l] = f32x4{0.f, 0.f, 0.f, 0.f};
          if constexpr (Epi::kInitFromOutput) {
            if (s == 0 && l < nlt && rt_first + r < sg.row_tiles) acc[m][r][l] = Epi::init(o, rt_first + r, lt0 + l, lane);
          }
        }
    const int c1 = (s + 1) * per;
    int c = s * per;
    for (; c + U <= c1; c += U) {
      u32x4 a[U][M][R], bx[U][LT];
#pragma unroll
      for (int u = 0; u < U; ++u) {
#pragma unroll
        for (int m = 0; m < M; ++m)
#pragma unroll
          for (int r = 0; r < R; ++r) a[u][m][r] = load16(wp[m][r] + static_cast<int64_t>(c + u) * kChunkBytes);
#pragma unroll
        for (int l = 0; l < LT; ++l)
          if (l < nlt) bx[u][l] = load16(xp[l] + static_cast<int64_t>(c + u) * kChunkBytes);
      }
#pragma unroll
      for (int u = 0; u < U; ++u)
#pragma unroll
        for (int l = 0; l < LT; ++l)
          if (l < nlt) {
#pragma unroll
            for (int m = 0; m < M; ++m)
#pragma unroll
              for (int r = 0; r < R; ++r) acc[m][r][l] = mfma(a[u][m][r], bx[u][l], acc[m][r][l]);
          }
    }
    for (; c < c1; ++c) {
      u32x4 a[M][R], bx[LT];
#pragma unroll
      for (int m = 0; m < M; ++m)
#pragma unroll
        for (int r = 0; r < R; ++r) a[m][r] = load16(wp[m][r] + static_cast<int64_t>(c) * kChunkBytes);
#pragma unroll
      for (int l = 0; l < LT; ++l)
        if (l < nlt) bx[l] = load16(xp[l] + static_cast<int64_t>(c) * kChunkBytes);
#pragma unroll
      for (int l = 0; l < LT; ++l)
        if (l < nlt) {
#pragma unroll
          for (int m = 0; m < M; ++m)
#pragma unroll
            for (int r = 0; r < R; ++r) acc[m][r][l] = mfma(a[m][r], bx[l], acc[m][r][l]);
        }
    }

    if constexpr (SMAX == 1) {
      // One split: the chain is the result.
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
    } else {
#pragma unroll
      for (int m = 0; m < M; ++m)
#pragma unroll
        for (int r = 0; r < R; ++r)
#pragma unroll
          for (int l = 0; l < LT; ++l)
            part[((((s * WR + wr) * M + m) * R + r) * LT + l) * kWave + lane] = acc[m][r][l];
    }
  }

  if constexpr (SMAX > 1) {
    __syncthreads();
    // Combine the split partials of each tile in ascending split order.
    for (int t = wave; t < WR * R * LT; t += WS * WR) {
      const int twr = t / (R * LT), r = (t / LT) % R, l = t % LT;
      const int rt = rb * (WR * R) + twr * R + r;
      if (l >= nlt || rt >= sg.row_tiles) continue;
      f32x4 y[M];
#pragma unroll
      for (int m = 0; m < M; ++m) {
        y[m] = part[((((0 * WR + twr) * M + m) * R + r) * LT + l) * kWave + lane];
        for (int s = 1; s < splits; ++s) y[m] = y[m] + part[((((s * WR + twr) * M + m) * R + r) * LT + l) * kWave + lane];
      }
      Epi::apply(o, g, si, rt, lt0 + l, y, lane);
    }
  }
}

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
  const Segment& sg = g.seg[si];
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

// ---------------------------------------------------------------------------
// Host side: split rule, validation, launch selection.

thread_local std::string g_last_error;

int fail(int code, const std::string& msg) {
  g_last_error = msg;
  return code;
}

// The fixed K-split for an N x K weight matrix. Matrices with few row tiles
// (N <= 4096: Q, K, V, output, down) get 8 splits so that a decode launch has
// enough independent weight streams; gate/up (N <= 16384) get 2; the LM head
// gets 1. S is then capped by the chunk count and halved until it divides it.
int split_count(int n, int k) {
  const int chunks = k / kChunkCols;
  int s = n <= 4096 ? 8 : (n <= 16384 ? 2 : 1);
  if (s > chunks) s = chunks;
  while (s > 1 && chunks % s != 0) s >>= 1;
  return s < 1 ? 1 : s;
}

bool lanes_ok(const StrideLanes& l, std::string& why) {
  if (l.rows < 0 || l.lane_groups != (l.rows + 15) / 16) {
    why = "lane_groups must equal ceil(rows / 16) (rows=" + std::to_string(l.rows) +
          ", lane_groups=" + std::to_string(l.lane_groups) + ")";
    return false;
  }
  return true;
}

bool mat_ok(const StrideGemmMat& m, const char* name, std::string& why) {
  if (!m.w || m.groups <= 0 || m.cols <= 0 || m.cols % kChunkCols != 0) {
    why = std::string(name) + ": need a weight pointer, groups > 0 and cols a positive multiple of 32 (groups=" +
          std::to_string(m.groups) + ", cols=" + std::to_string(m.cols) + ")";
    return false;
  }
  return true;
}

template <class Epi, int R, int LT, int WS, int WR, int SMAX>
int launch_stream(Geometry g, const typename Epi::Out& o, hipStream_t st) {
  int blocks = 0;
  for (int i = 0; i < g.nseg; ++i) {
    g.seg[i].blocks = (g.seg[i].row_tiles + WR * R - 1) / (WR * R);
    blocks += g.seg[i].blocks;
  }
  blocks *= (g.lane_groups + LT - 1) / LT;
  hipLaunchKernelGGL((k_stream<Epi, R, LT, WS, WR, SMAX>), dim3(blocks), dim3(kWave * WS * WR), 0, st, g, o);
  return 0;
}

template <class Epi, int LT>
int dispatch_stream_lt(const Geometry& g, const typename Epi::Out& o, int smax, hipStream_t st) {
  if (smax == 1) return launch_stream<Epi, 1, LT, 1, 4, 1>(g, o, st);
  if (smax == 2) return launch_stream<Epi, 1, LT, 2, 2, 2>(g, o, st);
  return launch_stream<Epi, 1, LT, 4, 1, 8>(g, o, st);
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

// Largest lane-tile count served by the streaming kernel.
constexpr int kStreamMaxLaneTiles = 8;

template <class Epi>
int run(Geometry g, const typename Epi::Out& o, hipStream_t st) {
  if (g.rows == 0) return 0;
  int smax = 1;
  for (int i = 0; i < g.nseg; ++i) {
    if (g.seg[i].splits > 8) return fail(STRIDE_TC_EINVAL, "split count above 8");
    smax = g.seg[i].splits > smax ? g.seg[i].splits : smax;
  }
  const int T = g.lane_groups;
  if (T <= kStreamMaxLaneTiles) {
    if (T <= 1) dispatch_stream_lt<Epi, 1>(g, o, smax, st);
    else if (T <= 2) dispatch_stream_lt<Epi, 2>(g, o, smax, st);
    else if (T <= 4) dispatch_stream_lt<Epi, 4>(g, o, smax, st);
    else dispatch_stream_lt<Epi, 8>(g, o, smax, st);
  } else {
    if constexpr (Epi::kMats == 2) launch_tile<Epi, 2, 4>(g, o, st);
    else launch_tile<Epi, 4, 4>(g, o, st);
  }
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(static_cast<int>(e), std::string("kernel launch failed: ") + hipGetErrorString(e));
  return 0;
}

Geometry single(const StrideLanes& l, const uint16_t* x, const StrideGemmMat& m, const uint16_t* w2) {
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

using namespace stride_tc;

// Layout guards: these structs cross the ABI by address and must match the
// reference's PODs (src/kernels.h, src/kernels_tc.h) byte for byte.
static_assert(sizeof(StrideGemmMat) == 16, "GemmMat layout");
static_assert(sizeof(StrideKvRef) == 56, "KvRef layout");
static_assert(sizeof(StrideLanes) == 16, "Lanes layout");
static_assert(sizeof(StrideBestEntry) == 8 && alignof(StrideBestEntry) == 8, "BestEntry layout");
static_assert(offsetof(StrideTcQkvParams, kv) == 88 && sizeof(StrideTcQkvParams) == 176, "TcQkvParams layout");
static_assert(sizeof(StrideTcGemmResidualParams) == 48, "TcGemmResidualParams layout");
static_assert(sizeof(StrideTcMlp13Params) == 64, "TcMlp13Params layout");
static_assert(sizeof(StrideTcLmGreedyParams) == 56, "TcLmGreedyParams layout");
static_assert(sizeof(StrideTcLmFullParams) == 48, "TcLmFullParams layout");

extern "C" {

int stride_tc_split_count(int32_t n, int32_t k) {
  if (n <= 0 || k <= 0 || k % kChunkCols != 0) return fail(-1, "split_count: need n > 0 and k a positive multiple of 32"), -1;
  return split_count(n, k);
}

const char* stride_tc_last_error(void) { return g_last_error.c_str(); }

const char* stride_tc_version(void) { return "stride_tc 0.1 gfx950 mfma_f32_16x16x32_bf16"; }

int stride_tc_gemm_residual(const StrideTcGemmResidualParams* p, int, int, void* stream) {
  std::string why;
  if (!p) return fail(STRIDE_TC_EINVAL, "gemm_residual: null params");
  if (!lanes_ok(p->l, why) || !mat_ok(p->m, "gemm_residual.m", why)) return fail(STRIDE_TC_EINVAL, "gemm_residual: " + why);
  if (!p->x || !p->h) return fail(STRIDE_TC_EINVAL, "gemm_residual: null x or h");
  Geometry g = single(p->l, p->x, p->m, nullptr);
  EpiResidual::Out o{p->h, p->m.groups};
  return run<EpiResidual>(g, o, static_cast<hipStream_t>(stream));
}

int stride_tc_mlp13(const StrideTcMlp13Params* p, int, int, void* stream) {
  std::string why;
  if (!p) return fail(STRIDE_TC_EINVAL, "mlp13: null params");
  if (!lanes_ok(p->l, why) || !mat_ok(p->w1, "mlp13.w1", why) || !mat_ok(p->w3, "mlp13.w3", why))
    return fail(STRIDE_TC_EINVAL, "mlp13: " + why);
  if (p->w1.groups != p->w3.groups || p->w1.cols != p->w3.cols) return fail(STRIDE_TC_EINVAL, "mlp13: w1 and w3 shapes differ");
  if (!p->x || !p->z) return fail(STRIDE_TC_EINVAL, "mlp13: null x or z");
  Geometry g = single(p->l, p->x, p->w1, p->w3.w);
  EpiGateUp::Out o{p->z, p->w1.groups};
  return run<EpiGateUp>(g, o, static_cast<hipStream_t>(stream));
}

int stride_tc_lm_full(const StrideTcLmFullParams* p, int, void* stream) {
  std::string why;
  if (!p) return fail(STRIDE_TC_EINVAL, "lm_full: null params");
  if (!lanes_ok(p->l, why) || !mat_ok(p->m, "lm_full.m", why)) return fail(STRIDE_TC_EINVAL, "lm_full: " + why);
  if (!p->x || !p->logits) return fail(STRIDE_TC_EINVAL, "lm_full: null x or logits");
  Geometry g = single(p->l, p->x, p->m, nullptr);
  EpiLogits::Out o{p->logits};
  return run<EpiLogits>(g, o, static_cast<hipStream_t>(stream));
}

int stride_tc_lm_greedy(const StrideTcLmGreedyParams* p, int, int, void* stream) {
  std::string why;
  if (!p) return fail(STRIDE_TC_EINVAL, "lm_greedy: null params");
  if (!lanes_ok(p->l, why) || !mat_ok(p->m, "lm_greedy.m", why)) return fail(STRIDE_TC_EINVAL, "lm_greedy: " + why);
  if (!p->x || !p->best) return fail(STRIDE_TC_EINVAL, "lm_greedy: null x or best");
  if (p->vocab <= 0 || p->vocab > p->m.groups * 16) return fail(STRIDE_TC_EINVAL, "lm_greedy: vocab must be in (0, groups*16]");
  Geometry g = single(p->l, p->x, p->m, nullptr);
  EpiArgmax::Out o{p->best, p->vocab};
  return run<EpiArgmax>(g, o, static_cast<hipStream_t>(stream));
}

int stride_tc_qkv(const StrideTcQkvParams* p, void* stream) {
  std::string why;
  if (!p) return fail(STRIDE_TC_EINVAL, "qkv: null params");
  if (!lanes_ok(p->l, why) || !mat_ok(p->q, "qkv.q", why) || !mat_ok(p->k, "qkv.k", why) || !mat_ok(p->v, "qkv.v", why))
    return fail(STRIDE_TC_EINVAL, "qkv: " + why);
  if (p->q.cols != p->k.cols || p->q.cols != p->v.cols || p->k.groups != p->v.groups)
    return fail(STRIDE_TC_EINVAL, "qkv: q, k, v must share cols and k, v must have equal groups");
  const int D = p->head_dim;
  if (D <= 0 || D % 16 != 0 || (p->q.groups * 16) % D != 0 || (p->k.groups * 16) % D != 0)
    return fail(STRIDE_TC_EINVAL, "qkv: head_dim must be a multiple of 16 dividing the q and k rows");
  if (!p->x || !p->q_out || !p->rope || !p->row_slot || !p->row_pos || !p->kv.arena || !p->kv.table)
    return fail(STRIDE_TC_EINVAL, "qkv: null pointer argument");
  if (p->kv.head_dim != D || p->kv.group_elems <= 0 || p->kv.group_elems % D != 0)
    return fail(STRIDE_TC_EINVAL, "qkv: kv.head_dim must equal head_dim and kv.group_elems must be tokens*head_dim");
  const int64_t page = p->kv.group_elems / D;
  int shift = 0;
  while ((int64_t{1} << shift) < page) ++shift;
  if ((int64_t{1} << shift) != page) return fail(STRIDE_TC_EINVAL, "qkv: KV page size (group_elems/head_dim) must be a power of two");
  Geometry g{};
  g.x = p->x;
  g.col_tiles = p->q.cols / 16;
  g.rows = p->l.rows;
  g.lane_groups = p->l.lane_groups;
  g.nseg = 3;
  const StrideGemmMat* mats[3] = {&p->q, &p->k, &p->v};
  for (int i = 0; i < 3; ++i) {
    g.seg[i].w[0] = mats[i]->w;
    g.seg[i].w[1] = nullptr;
    g.seg[i].row_tiles = mats[i]->groups;
    g.seg[i].splits = split_count(mats[i]->groups * 16, mats[i]->cols);
  }
  EpiQkv::Out o{};
  o.q_out = p->q_out;
  o.q_stride = p->q_stride;
  o.layer = p->layer;
  o.head_dim = D;
  o.page_shift = shift;
  o.kv = p->kv;
  o.rope = p->rope;
  o.row_slot = p->row_slot;
  o.row_pos = p->row_pos;
  return run<EpiQkv>(g, o, static_cast<hipStream_t>(stream));
}

}  // extern "C"
