// The exact path on gfx950: the reference's fused FP32 kernels (src/kernels.cu)
// evaluated on the GPU with the same IEEE operations, in the same order, per
// output element as the reference's CPU exact path, so the two agree bit for bit.
//
// Mapping. The reference runs one 32-thread block per (four-row weight group,
// lane group). Here a 64-lane wavefront runs two such blocks side by side (lanes
// 0-31 and 32-63); within a half, lane t is the reference's thread t and owns
// the same 64-byte weight lines (l == t mod 32), chaining fmaf over their columns
// in ascending order. The 32 partial sums go through LDS and are added left to
// right by one lane per output, ((P0 + P1) + P2) + ... + P31. Built with
// -ffp-contract=off, so only the explicit fmaf calls fuse; division and square
// root are the correctly rounded ones. Nothing here depends on the batch: a
// block's result depends on its own weight group and lane group only.
#include <hip/hip_runtime.h>

#include <string>

#include "../../include/stride_exact.h"
#include "tc_common.hpp"

namespace stride_tc {

int fail(int code, const std::string& msg);  // tc_gemm.hip

namespace {

constexpr int kChains = 32;  // partial chains per dot product (src/kernels.h kBlockThreads)

__device__ __forceinline__ float lo_half(uint32_t v) { return f32_of(v << 16); }
__device__ __forceinline__ float hi_half(uint32_t v) { return f32_of(v & 0xFFFF0000u); }

// Chain t of the dot products of one four-row weight group (wg: [col][4] bf16)
// with LG lane groups of J lanes of x (dim-major, lane j of column c at
// x[c * stride + j], lane group i at x + 4 * xi[i]): acc[(i * 4 + r) * J + j] for
// lane group i, row r, lane j. Lines of 8 columns: t, t + 32, ...; each line is
// four 16-byte words, word q holding columns k + 2q (rows 0-3 in its first two
// 32-bit halves' bf16 pairs) and k + 2q + 1 (last two) (src/kernels.cu:22-94).
// A weight line is loaded once for the LG lane groups; every output's FMAs run
// in the same order whatever LG is.
template <int J, int LG>
__device__ __forceinline__ void chain(const uint16_t* wg, const float* x, int stride, int cols, int t,
                                      const int (&xi)[LG], float (&acc)[4 * J * LG]) {
  static_assert(J == 4 || LG == 1, "one lane: one lane group");
#pragma unroll
  for (int e = 0; e < 4 * J * LG; ++e) acc[e] = 0.0f;
  // Line k's weights (four 16-byte words) and x columns k .. k+7 of each lane group.
  struct Line {
    u32x4 v[4];
    f32x4 xc[LG][J == 1 ? 2 : 8];
  };
  auto load = [&](int line, Line& L) {
    const int k = line * 8;
    const u32x4* wl = reinterpret_cast<const u32x4*>(wg + static_cast<int64_t>(k) * 4);
#pragma unroll
    for (int q = 0; q < 4; ++q) L.v[q] = wl[q];
    if constexpr (J == 1) {
      L.xc[0][0] = *reinterpret_cast<const f32x4*>(x + k);
      L.xc[0][1] = *reinterpret_cast<const f32x4*>(x + k + 4);
    } else {
#pragma unroll
      for (int i = 0; i < LG; ++i)
#pragma unroll
        for (int c = 0; c < 8; ++c)
          L.xc[i][c] = *reinterpret_cast<const f32x4*>(x + static_cast<int64_t>(k + c) * stride + 4 * xi[i]);
    }
  };
  auto step = [&](const Line& L) {
#pragma unroll
    for (int q = 0; q < 4; ++q) {
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const int c = 2 * q + h;  // column k + c
        const float w[4] = {lo_half(L.v[q][2 * h]), hi_half(L.v[q][2 * h]), lo_half(L.v[q][2 * h + 1]),
                            hi_half(L.v[q][2 * h + 1])};
        if constexpr (J == 1) {
          const float xc = L.xc[0][c >> 2][c & 3];
#pragma unroll
          for (int r = 0; r < 4; ++r) acc[r] = __builtin_fmaf(w[r], xc, acc[r]);
        } else {
#pragma unroll
          for (int i = 0; i < LG; ++i)
#pragma unroll
            for (int r = 0; r < 4; ++r)
#pragma unroll
              for (int j = 0; j < 4; ++j)
                acc[(i * 4 + r) * 4 + j] = __builtin_fmaf(w[r], L.xc[i][c][j], acc[(i * 4 + r) * 4 + j]);
        }
      }
    }
  };
  // Lines t, t + 32, ... in ascending order, their loads issued NB lines at a
  // time so that a lane waits one memory round trip per batch, not per line.
  constexpr int NB = J == 1 ? 8 : (LG <= 2 ? 2 : 1);
  const int lines = cols / 8;
  int line = t;
  for (; line + (NB - 1) * kChains < lines; line += NB * kChains) {
    Line L[NB];
#pragma unroll
    for (int b = 0; b < NB; ++b) load(line + b * kChains, L[b]);
    __builtin_amdgcn_sched_barrier(0);  // every load of the batch before the first use
#pragma unroll
    for (int b = 0; b < NB; ++b) step(L[b]);
  }
  for (; line < lines; line += kChains) {
    Line L;
    load(line, L);
    step(L);
  }
}

// Columns per slice of the sliced GEMM below: 32 lines of 8, so a slice holds
// exactly one line of each chain.
constexpr int kSlice = 256;

// ---------------------------------------------------------------------------
// GEMM-shaped operators: Op supplies the weight group(s) of a block and the
// epilogue on the folded sums y[m][r * J + j].

struct ResidualOp {  // src/kernels.cu:294-325
  using Params = StrideGemmResidualParams;
  static constexpr int kMats = 1;
  static int groups(const Params& p) { return p.m.groups; }
  static bool cols_sliced(const Params& p) { return p.m.cols % kSlice == 0; }
  __device__ static const uint16_t* w(const Params& p, int, int group, int& cols) {
    cols = p.m.cols;
    return p.m.w + static_cast<int64_t>(group) * p.m.cols * 4;
  }
  template <int J>
  __device__ static void finish(const Params& p, int group, int lg, int t, const float (*y)[16]) {
    if (t >= 4 * J) return;
    const int r = t / J, jj = t % J;
    float* h = p.h + static_cast<int64_t>(group * 4 + r) * p.l.stride + lg * 4 + jj;
    h[0] = h[0] + y[0][t];
  }
};

struct Mlp13Op {  // src/kernels.cu:329-363
  using Params = StrideMlp13Params;
  static constexpr int kMats = 2;
  static int groups(const Params& p) { return p.w1.groups; }
  static bool cols_sliced(const Params& p) { return p.w1.cols % kSlice == 0 && p.w3.cols == p.w1.cols; }
  __device__ static const uint16_t* w(const Params& p, int m, int group, int& cols) {
    const StrideGemmMat& mm = m == 0 ? p.w1 : p.w3;
    cols = mm.cols;
    return mm.w + static_cast<int64_t>(group) * mm.cols * 4;
  }
  template <int J>
  __device__ static void finish(const Params& p, int group, int lg, int t, const float (*y)[16]) {
    if (t >= 4 * J) return;
    const int r = t / J, jj = t % J;
    p.z[static_cast<int64_t>(group * 4 + r) * p.l.stride + lg * 4 + jj] = det_silu(y[0][t]) * y[1][t];
  }
};

struct LmFullOp {  // src/kernels.cu:427-452
  using Params = StrideLmFullParams;
  static constexpr int kMats = 1;
  static int groups(const Params& p) { return p.m.groups; }
  static bool cols_sliced(const Params& p) { return p.m.cols % kSlice == 0; }
  __device__ static const uint16_t* w(const Params& p, int, int group, int& cols) {
    cols = p.m.cols;
    return p.m.w + static_cast<int64_t>(group) * p.m.cols * 4;
  }
  template <int J>
  __device__ static void finish(const Params& p, int group, int lg, int t, const float (*y)[16]) {
    if (t >= 4 * J) return;
    const int r = t / J, jj = t % J;
    p.logits[static_cast<int64_t>(group * 4 + r) * p.l.stride + lg * 4 + jj] = y[0][t];
  }
};

struct LmGreedyOp {  // src/kernels.cu:383-425
  using Params = StrideLmGreedyParams;
  static constexpr int kMats = 1;
  static int groups(const Params& p) { return p.m.groups; }
  static bool cols_sliced(const Params& p) { return p.m.cols % kSlice == 0; }
  __device__ static const uint16_t* w(const Params& p, int, int group, int& cols) {
    cols = p.m.cols;
    return p.m.w + static_cast<int64_t>(group) * p.m.cols * 4;
  }
  template <int J>
  __device__ static void finish(const Params& p, int group, int lg, int t, const float (*y)[16]) {
    if (t >= J) return;
    const int lane = lg * 4 + t;
    if (lane >= p.l.rows) return;
    float best = f32_of(0xFF800000u);
    int32_t best_i = -1;
    for (int r = 0; r < 4; ++r) {
      const int index = group * 4 + r;
      if (index >= p.vocab) continue;
      const float v = y[0][r * J + t];
      if (v > best) {
        best = v;
        best_i = index;
      }
    }
    if (best_i >= 0) best_update(&p.best[lane], best, best_i);
  }
};

struct QkvOp {  // src/kernels.cu:204-284
  using Params = StrideQkvParams;
  static constexpr int kMats = 1;
  static int groups(const Params& p) { return p.q.groups + 2 * p.k.groups; }
  static bool cols_sliced(const Params& p) { return p.q.cols % kSlice == 0; }  // k and v: the same cols
  __device__ static const uint16_t* w(const Params& p, int, int gi, int& cols) {
    const StrideGemmMat& m = gi < p.q.groups ? p.q : (gi < p.q.groups + p.k.groups ? p.k : p.v);
    const int group = gi < p.q.groups ? gi : (gi < p.q.groups + p.k.groups ? gi - p.q.groups : gi - p.q.groups - p.k.groups);
    cols = m.cols;
    return m.w + static_cast<int64_t>(group) * m.cols * 4;
  }
  template <int J>
  __device__ static void finish(const Params& p, int gi, int lg, int t, const float (*y)[16]) {
    if (t >= J) return;
    const int j = lg * 4 + t;
    if (j >= p.l.rows) return;
    const int kind = gi < p.q.groups ? 0 : (gi < p.q.groups + p.k.groups ? 1 : 2);
    const int group = kind == 0 ? gi : (kind == 1 ? gi - p.q.groups : gi - p.q.groups - p.k.groups);
    const int D = p.head_dim, half = D / 2;
    const int head = group / (D / 4);
    const int d0 = 2 * (group % (D / 4));
    const int pos = p.row_pos[j], slot = p.row_slot[j];
    float a0 = y[0][0 * J + t], a1 = y[0][1 * J + t], b0 = y[0][2 * J + t], b1 = y[0][3 * J + t];
    if (kind != 2) {
      const float* cs = p.rope + (static_cast<int64_t>(pos) * half + d0) * 2;
      const float c0 = cs[0], s0 = cs[1], c1 = cs[2], s1 = cs[3];
      const float ra0 = a0 * c0 - b0 * s0, rb0 = b0 * c0 + a0 * s0;
      const float ra1 = a1 * c1 - b1 * s1, rb1 = b1 * c1 + a1 * s1;
      a0 = ra0;
      b0 = rb0;
      a1 = ra1;
      b1 = rb1;
    }
    float* dst;
    if (kind == 0) {
      dst = p.q_out + static_cast<int64_t>(j) * p.q_stride + static_cast<int64_t>(head) * D;
    } else {
      const StrideKvRef& kv = p.kv;
      const int64_t tokens = kv.group_elems / kv.head_dim;  // a power of two (checked on the host)
      const int64_t block = kv.table[static_cast<int64_t>(slot) * kv.max_blocks + pos / tokens];
      dst = static_cast<float*>(kv.arena) + block * kv.block_elems + p.layer * kv.layer_elems +
            (kind - 1) * kv.which_elems + head * kv.group_elems + (pos % tokens) * kv.head_dim;
    }
    dst[d0] = a0;
    dst[d0 + 1] = a1;
    dst[d0 + half] = b0;
    dst[d0 + half + 1] = b1;
  }
};

// Two blocks per 64-lane workgroup: block = 2 * (logical workgroup) + half. A
// block is one reference block (one weight group, one lane group) for LG = 1, or
// the reference blocks of one weight group and LG consecutive lane groups, which
// then share each weight line load: (weight group, lane-group set) = (block /
// sets, block % sets). The hardware hands workgroup i to XCD i % 8; logical
// workgroups are numbered so that consecutive ones (the lane groups of one
// weight group) share an XCD and so read that group's weights through one L2.
__device__ __forceinline__ int exact_wg_order(int i, int n) {
  const int full = n & ~7;
  if (i >= full) return i;
  return (i & 7) * (full >> 3) + (i >> 3);
}

template <class Op, int J, int LG>
__global__ __launch_bounds__(64) void k_exact_gemm(typename Op::Params p, int nblocks) {
  constexpr int M = Op::kMats;
  constexpr int NO = 4 * J;  // outputs per reference block
  __shared__ float part[2][kChains][M][NO * LG];
  __shared__ float ys[2][LG][M][16];
  const int half = threadIdx.x >> 5, t = threadIdx.x & 31;
  const int block = exact_wg_order(blockIdx.x, gridDim.x) * 2 + half;
  const bool live = block < nblocks;
  const int sets = (p.l.lane_groups + LG - 1) / LG;
  const int set = live ? block % sets : 0;
  const int group = live ? block / sets : 0;
  const int lg0 = set * LG, nlg = min(LG, p.l.lane_groups - lg0);
  if (live) {
    const float* x = J == 1 ? p.x : p.x + lg0 * 4;
    int xi[LG];  // lane groups past the last live one read the last live one's x
#pragma unroll
    for (int i = 0; i < LG; ++i) xi[i] = min(i, nlg - 1);
#pragma unroll
    for (int m = 0; m < M; ++m) {
      int cols = 0;
      const uint16_t* wg = Op::w(p, m, group, cols);
      float acc[NO * LG];
      chain<J, LG>(wg, x, p.l.stride, cols, t, xi, acc);
#pragma unroll
      for (int e = 0; e < NO * LG; ++e) part[half][t][m][e] = acc[e];
    }
  }
  __syncthreads();
  if (live) {
    for (int e = t; e < NO * LG; e += kChains) {
#pragma unroll
      for (int m = 0; m < M; ++m) {
        float y = part[half][0][m][e];
        for (int i = 1; i < kChains; ++i) y = y + part[half][i][m][e];
        ys[half][e / NO][m][e % NO] = y;
      }
    }
  }
  __syncthreads();
  if (live)
    for (int i = 0; i < nlg; ++i) Op::template finish<J>(p, group, lg0 + i, t, ys[half][i]);
}

// Sliced form (four batch lanes per reference block, columns a multiple of
// kSlice): a workgroup of NWV waves runs NB = 2 * NWV reference blocks, i.e. NB
// consecutive weight groups with one set of LG lane groups, so the blocks share
// x. K is taken kSlice columns at a time: slice s holds line 32 * s + t of chain
// t, so each lane still chains its lines in ascending order and every output's
// operations are those of chain() (and of the reference). The slice's x is
// staged once per workgroup in LDS (double buffered, the next slice's loads in
// flight while the current one is summed), laid out so that lane t's reads of a
// column are consecutive 16-byte words; each lane loads its own weight line one
// slice ahead. The matrices of a paired GEMM are swept one after the other, and
// each one's partials are folded and finished as in k_exact_gemm.
template <class Op, int LG, int NWV>
__global__ __launch_bounds__(64 * NWV) void k_exact_gemm_s(typename Op::Params p, int nsets, int ngroups) {
  constexpr int M = Op::kMats;
  constexpr int NB = 2 * NWV;
  constexpr int NO = 16;                     // outputs per reference block (4 rows x 4 lanes)
  constexpr int XS = kSlice * LG;            // staged f32x4 per slice: one per column and lane group
  constexpr int NT = 64 * NWV;
  constexpr int XPER = (XS + NT - 1) / NT;   // staging loads per thread
  __shared__ f32x4 xs[2 * XS];
  __shared__ float part[NB][kChains][NO * LG];
  __shared__ float ys[NB][LG][M][16];
  const int tid = threadIdx.x, wave = tid >> 6, half = (tid >> 5) & 1, t = tid & 31;
  const int b = wave * 2 + half;
  const int w = exact_wg_order(blockIdx.x, gridDim.x);
  const int set = w % nsets;
  const int group = (w / nsets) * NB + b;
  const bool live = group < ngroups;
  const int lg0 = set * LG, nlg = min(LG, p.l.lane_groups - lg0);

  // Staging: item q of a slice is column c = q / LG, lane group q % LG (clamped
  // to the last live one); column 8 * l + e (line l, column e of the line) sits
  // at (e * 32 + l) * LG + i.
  f32x4 xr[XPER];
  auto load_x = [&](int sl) {
#pragma unroll
    for (int r = 0; r < XPER; ++r) {
      const int q = tid + r * NT;
      if (q < XS) {
        const int c = q / LG, i = min(q % LG, nlg - 1);
        xr[r] = *reinterpret_cast<const f32x4*>(p.x + static_cast<int64_t>(sl * kSlice + c) * p.l.stride + 4 * (lg0 + i));
      }
    }
  };
  auto store_x = [&](int buf) {
#pragma unroll
    for (int r = 0; r < XPER; ++r) {
      const int q = tid + r * NT;
      if (q < XS) {
        const int c = q / LG, i = q % LG, l = c >> 3, e = c & 7;
        xs[buf * XS + (e * 32 + l) * LG + i] = xr[r];
      }
    }
  };

  unroll<M>([&](auto mm) {
    constexpr int m = decltype(mm)::value;
    int cols = 0;
    const uint16_t* wg = Op::w(p, m, min(group, ngroups - 1), cols);
    const int nsl = cols / kSlice;
    u32x4 wl[2][4];  // this lane's weight line of the current and the next slice
    auto load_w = [&](int sl, auto buf) {
      const u32x4* src = reinterpret_cast<const u32x4*>(wg + static_cast<int64_t>(sl * kChains + t) * 32);
#pragma unroll
      for (int q = 0; q < 4; ++q) wl[decltype(buf)::value][q] = src[q];
    };
    float acc[NO * LG];
#pragma unroll
    for (int e = 0; e < NO * LG; ++e) acc[e] = 0.0f;
    auto step = [&](auto buf) {
      constexpr int c2 = decltype(buf)::value;
#pragma unroll
      for (int q = 0; q < 4; ++q) {
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          const int c = 2 * q + h;  // column c of the line
          const float wv[4] = {lo_half(wl[c2][q][2 * h]), hi_half(wl[c2][q][2 * h]), lo_half(wl[c2][q][2 * h + 1]),
                               hi_half(wl[c2][q][2 * h + 1])};
#pragma unroll
          for (int i = 0; i < LG; ++i) {
            const f32x4 xc = xs[c2 * XS + (c * 32 + t) * LG + i];
#pragma unroll
            for (int r = 0; r < 4; ++r)
#pragma unroll
              for (int j = 0; j < 4; ++j) acc[(i * 4 + r) * 4 + j] = __builtin_fmaf(wv[r], xc[j], acc[(i * 4 + r) * 4 + j]);
          }
        }
      }
    };
    load_x(0);
    load_w(0, std::integral_constant<int, 0>{});
    store_x(0);
    __syncthreads();
    // Slices in pairs so that the register and LDS buffers are compile-time.
    // The next slice's loads are issued unconditionally (the last slice's again
    // after it, into buffers nobody reads), so every pass waits on the same loads.
    int sl = 0;
    auto one = [&](auto cur) {
      constexpr int c = decltype(cur)::value;
      const int nx = min(sl + 1, nsl - 1);
      load_x(nx);
      load_w(nx, std::integral_constant<int, c ^ 1>{});
      step(cur);
      store_x(c ^ 1);
      __syncthreads();
      ++sl;
    };
    while (sl < nsl) {
      one(std::integral_constant<int, 0>{});
      if (sl < nsl) one(std::integral_constant<int, 1>{});
    }
    // Partials of this matrix, folded left to right per output.
#pragma unroll
    for (int e = 0; e < NO * LG; ++e) part[b][t][e] = acc[e];
    __syncthreads();
    for (int e = t; e < NO * LG; e += kChains) {
      float y = part[b][0][e];
      for (int i = 1; i < kChains; ++i) y = y + part[b][i][e];
      ys[b][e / NO][m][e % NO] = y;
    }
    __syncthreads();
  });
  if (live)
    for (int i = 0; i < nlg; ++i) Op::template finish<4>(p, group, lg0 + i, t, ys[b][i]);
}

// ---------------------------------------------------------------------------
// Embedding, RMSNorm, compaction.

// h[k * stride + row] = widen(embed[token][k]); embed in [token/4][dim][4]
// groups (src/kernels.cu:98-117). A thread's kEmbedBatch elements are loaded
// before any is stored, so the row costs one memory round trip per batch, not
// one per element.
constexpr int kEmbedBatch = 8;
__global__ __launch_bounds__(256) void k_exact_embed(StrideEmbedParams p) {
  const int row = blockIdx.x;
  const int token = p.tokens[row];
  const uint16_t* src = p.embed + static_cast<int64_t>(token / 4) * p.dim * 4 + token % 4;
  for (int k0 = threadIdx.x; k0 < p.dim; k0 += 256 * kEmbedBatch) {
    uint16_t v[kEmbedBatch];
#pragma unroll
    for (int i = 0; i < kEmbedBatch; ++i) {
      const int k = min(k0 + 256 * i, p.dim - 1);
      v[i] = src[static_cast<int64_t>(k) * 4];
    }
#pragma unroll
    for (int i = 0; i < kEmbedBatch; ++i) {
      const int k = k0 + 256 * i;
      if (k < p.dim) p.h[static_cast<int64_t>(k) * p.l.stride + row] = f32_of(static_cast<uint32_t>(v[i]) << 16);
    }
  }
}

// RMSNorm over four-dim units (src/kernels.cu:119-200): chain t sums the squares
// of units u == t (mod 32) by fmaf, the 32 partials are added left to right,
// r = 1 / sqrtf(sum / dim + eps), out = w * (v * r). One reference block (lane
// group) per wavefront half.
template <int J>
__global__ __launch_bounds__(64) void k_exact_norm(StrideNormParams p) {
  __shared__ float part[2][kChains][J];
  __shared__ float rs[2][J];
  const int half = threadIdx.x >> 5, t = threadIdx.x & 31;
  const int block = blockIdx.x * 2 + half;
  const bool live = block < p.l.lane_groups;
  const int units = p.dim / 4, stride = p.l.stride;
  const float* in = J == 1 ? p.in : p.in + (live ? block : 0) * 4;
  float* out = J == 1 ? p.out : p.out + (live ? block : 0) * 4;
  // A lane's units u = t, t + 32, ... are loaded NB at a time before their
  // FMAs, so the chain waits one memory round trip per batch, not per unit.
  constexpr int NB = J == 1 ? 8 : 4;
  auto load_unit = [&](int u, f32x4 (&v)[4]) {
    const int k = u * 4;
    if constexpr (J == 1) {
      v[0] = *reinterpret_cast<const f32x4*>(in + k);
    } else {
#pragma unroll
      for (int c = 0; c < 4; ++c) v[c] = *reinterpret_cast<const f32x4*>(in + static_cast<int64_t>(k + c) * stride);
    }
  };
  if (live) {
    float acc[J];
#pragma unroll
    for (int j = 0; j < J; ++j) acc[j] = 0.0f;
    auto sum_unit = [&](const f32x4 (&v)[4]) {
      if constexpr (J == 1) {
#pragma unroll
        for (int e = 0; e < 4; ++e) acc[0] = __builtin_fmaf(v[0][e], v[0][e], acc[0]);
      } else {
#pragma unroll
        for (int c = 0; c < 4; ++c)
#pragma unroll
          for (int j = 0; j < 4; ++j) acc[j] = __builtin_fmaf(v[c][j], v[c][j], acc[j]);
      }
    };
    int u = t;
    for (; u + (NB - 1) * kChains < units; u += NB * kChains) {
      f32x4 v[NB][4];
#pragma unroll
      for (int b = 0; b < NB; ++b) load_unit(u + b * kChains, v[b]);
      __builtin_amdgcn_sched_barrier(0);  // every load of the batch before the first FMA
#pragma unroll
      for (int b = 0; b < NB; ++b) sum_unit(v[b]);
    }
    for (; u < units; u += kChains) {
      f32x4 v[4];
      load_unit(u, v);
      sum_unit(v);
    }
#pragma unroll
    for (int j = 0; j < J; ++j) part[half][t][j] = acc[j];
  }
  __syncthreads();
  if (live && t < J) {
    float sum = part[half][0][t];
    for (int i = 1; i < kChains; ++i) sum = sum + part[half][i][t];
    rs[half][t] = 1.0f / sqrtf(sum / static_cast<float>(p.dim) + p.eps);
  }
  __syncthreads();
  if (!live) return;
  auto scale_unit = [&](int u, const f32x4& w4, const f32x4 (&v)[4]) {
    const int k = u * 4;
    if constexpr (J == 1) {
      const float r = rs[half][0];
      f32x4 o;
#pragma unroll
      for (int e = 0; e < 4; ++e) o[e] = w4[e] * (v[0][e] * r);
      *reinterpret_cast<f32x4*>(out + k) = o;
    } else {
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        f32x4 o;
#pragma unroll
        for (int j = 0; j < 4; ++j) o[j] = w4[c] * (v[c][j] * rs[half][j]);
        *reinterpret_cast<f32x4*>(out + static_cast<int64_t>(k + c) * stride) = o;
      }
    }
  };
  int u = t;
  for (; u + (NB - 1) * kChains < units; u += NB * kChains) {
    f32x4 v[NB][4], w4[NB];
#pragma unroll
    for (int b = 0; b < NB; ++b) {
      w4[b] = *reinterpret_cast<const f32x4*>(p.weight + (u + b * kChains) * 4);
      load_unit(u + b * kChains, v[b]);
    }
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int b = 0; b < NB; ++b) scale_unit(u + b * kChains, w4[b], v[b]);
  }
  for (; u < units; u += kChains) {
    f32x4 v[4];
    load_unit(u, v);
    scale_unit(u, *reinterpret_cast<const f32x4*>(p.weight + u * 4), v);
  }
}

// The same RMSNorm with one 256-thread workgroup per lane group: every thread
// loads its share of the lane group's inputs (and the gains it will scale them
// with) in one memory round trip, the inputs into LDS; the 32 chains then run
// over LDS in the order above, and all 256 threads scale and store. Serves rows
// of up to kNormLdsItems 16-byte items (dim four-lane columns for J = 4, dim / 4
// units for J = 1): 64 KiB of LDS.
constexpr int kNormPer = 16;
constexpr int kNormLdsItems = 256 * kNormPer;
template <int J>
__global__ __launch_bounds__(256) void k_exact_norm_lds(StrideNormParams p) {
  extern __shared__ f32x4 vsm[];  // item i: unit i (J = 1) or column i's four lanes (J = 4)
  __shared__ float part[kChains][J];
  __shared__ float rs[J];
  const int tid = threadIdx.x, block = blockIdx.x;
  const int units = p.dim / 4, stride = p.l.stride;
  const int items = J == 1 ? units : p.dim;
  const float* in = J == 1 ? p.in : p.in + block * 4;
  float* out = J == 1 ? p.out : p.out + block * 4;
  f32x4 v[kNormPer], w4[J == 1 ? kNormPer : 1];
  float wk[J == 1 ? 1 : kNormPer];
#pragma unroll
  for (int r = 0; r < kNormPer; ++r) {
    const int i = tid + 256 * r;
    if (i < items) {
      if constexpr (J == 1) {
        v[r] = *reinterpret_cast<const f32x4*>(in + 4 * i);
        w4[r] = *reinterpret_cast<const f32x4*>(p.weight + 4 * i);
      } else {
        v[r] = *reinterpret_cast<const f32x4*>(in + static_cast<int64_t>(i) * stride);
        wk[r] = p.weight[i];
      }
    }
  }
#pragma unroll
  for (int r = 0; r < kNormPer; ++r)
    if (tid + 256 * r < items) vsm[tid + 256 * r] = v[r];
  __syncthreads();
  if (tid < kChains) {
    float acc[J];
#pragma unroll
    for (int j = 0; j < J; ++j) acc[j] = 0.0f;
    for (int u = tid; u < units; u += kChains) {
      if constexpr (J == 1) {
        const f32x4 x = vsm[u];
#pragma unroll
        for (int e = 0; e < 4; ++e) acc[0] = __builtin_fmaf(x[e], x[e], acc[0]);
      } else {
#pragma unroll
        for (int c = 0; c < 4; ++c) {
          const f32x4 x = vsm[u * 4 + c];
#pragma unroll
          for (int j = 0; j < 4; ++j) acc[j] = __builtin_fmaf(x[j], x[j], acc[j]);
        }
      }
    }
#pragma unroll
    for (int j = 0; j < J; ++j) part[tid][j] = acc[j];
  }
  __syncthreads();
  if (tid < J) {
    float sum = part[0][tid];
    for (int i = 1; i < kChains; ++i) sum = sum + part[i][tid];
    rs[tid] = 1.0f / sqrtf(sum / static_cast<float>(p.dim) + p.eps);
  }
  __syncthreads();
#pragma unroll
  for (int r = 0; r < kNormPer; ++r) {
    const int i = tid + 256 * r;
    if (i >= items) continue;
    f32x4 o;
    if constexpr (J == 1) {
      const float q = rs[0];
#pragma unroll
      for (int e = 0; e < 4; ++e) o[e] = w4[r][e] * (v[r][e] * q);
      *reinterpret_cast<f32x4*>(out + 4 * i) = o;
    } else {
#pragma unroll
      for (int j = 0; j < 4; ++j) o[j] = wk[r] * (v[r][j] * rs[j]);
      *reinterpret_cast<f32x4*>(out + static_cast<int64_t>(i) * stride) = o;
    }
  }
}

// out[k * lm_stride + l] = in[k * stride + lm_rows[l]] (src/kernels.cu:365-380).
__global__ __launch_bounds__(64) void k_exact_compact(StrideCompactParams p) {
  const int k = blockIdx.x * 64 + threadIdx.x;
  if (k >= p.dim) return;
  for (int l = 0; l < p.lm_count; ++l)
    p.out[static_cast<int64_t>(k) * p.lm_stride + l] = p.in[static_cast<int64_t>(k) * p.l.stride + p.lm_rows[l]];
}

// ---------------------------------------------------------------------------
// Host side.

std::string lanes_why(const StrideLanes& l, int J) {
  if (J != 1 && J != 4) return "J must be 1 or 4";
  if (l.rows < 0) return "rows must be >= 0";
  if (J == 1 && (l.rows > 1 || l.lane_groups != 1 || l.stride != 1)) return "J = 1 serves one row with lane_groups 1 and stride 1";
  if (J == 4 && (l.lane_groups != (l.rows + 3) / 4 || l.stride < 4 * l.lane_groups || l.stride % 4 != 0))
    return "J = 4 needs lane_groups = ceil(rows / 4) and a stride that is a multiple of 4 covering them";
  return "";
}

std::string mat_why(const StrideGemmMat& m, const char* name) {
  if (!m.w || m.groups <= 0 || m.cols <= 0 || m.cols % 8 != 0)
    return std::string(name) + ": need a weight pointer, groups > 0 and cols a positive multiple of 8";
  return "";
}

int launched(const char* what) {
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(static_cast<int>(e), std::string(what) + " launch failed: " + hipGetErrorString(e));
  return 0;
}

#ifndef STRIDE_EXACT_LG
#define STRIDE_EXACT_LG 2
#endif
template <class Op>
int run_gemm(const typename Op::Params& p, int J, void* stream, const char* what) {
  constexpr int LG = STRIDE_EXACT_LG;  // lane groups sharing a weight line load
  const int lg = J == 1 ? 1 : LG;
  const int nblocks = Op::groups(p) * ((p.l.lane_groups + lg - 1) / lg);
  if (p.l.rows == 0 || nblocks == 0) return 0;
  hipStream_t st = static_cast<hipStream_t>(stream);
  // Four batch lanes per reference block: the sliced form shares x over eight
  // weight groups. (One lane: the loads are weight-bound, and the streaming
  // form keeps more of them in flight.)
  if (J == 4 && Op::cols_sliced(p)) {
    constexpr int NWV = 4;
    const int sets = (p.l.lane_groups + lg - 1) / lg;
    const dim3 sgrid(((Op::groups(p) + 2 * NWV - 1) / (2 * NWV)) * sets);
    hipLaunchKernelGGL((k_exact_gemm_s<Op, LG, NWV>), sgrid, dim3(64 * NWV), 0, st, p, sets, Op::groups(p));
    return launched(what);
  }
  const dim3 grid((nblocks + 1) / 2);
  if (J == 1) hipLaunchKernelGGL((k_exact_gemm<Op, 1, 1>), grid, dim3(64), 0, st, p, nblocks);
  else hipLaunchKernelGGL((k_exact_gemm<Op, 4, LG>), grid, dim3(64), 0, st, p, nblocks);
  return launched(what);
}

}  // namespace
}  // namespace stride_tc

using namespace stride_tc;

static_assert(sizeof(StrideEmbedParams) == 48, "EmbedParams layout");
static_assert(sizeof(StrideNormParams) == 48, "NormParams layout");
static_assert(offsetof(StrideQkvParams, kv) == 88 && offsetof(StrideQkvParams, rope) == 144 &&
                  sizeof(StrideQkvParams) == 176, "QkvParams layout");
static_assert(sizeof(StrideGemmResidualParams) == 48, "GemmResidualParams layout");
static_assert(sizeof(StrideMlp13Params) == 64, "Mlp13Params layout");
static_assert(sizeof(StrideCompactParams) == 56, "CompactParams layout");
static_assert(offsetof(StrideLmGreedyParams, best) == 48 && sizeof(StrideLmGreedyParams) == 56, "LmGreedyParams layout");
static_assert(sizeof(StrideLmFullParams) == 48, "LmFullParams layout");

extern "C" {

int stride_k_embed(const StrideEmbedParams* p, void* stream) {
  if (!p) return fail(STRIDE_TC_EINVAL, "k_embed: null parameters");
  if (p->l.rows < 0 || p->dim <= 0 || (p->l.rows > 0 && (!p->embed || !p->tokens || !p->h)) ||
      p->l.stride < p->l.rows)
    return fail(STRIDE_TC_EINVAL, "k_embed: need rows >= 0, dim > 0, stride >= rows and pointers");
  if (p->l.rows == 0) return 0;
  hipLaunchKernelGGL(k_exact_embed, dim3(p->l.rows), dim3(256), 0, static_cast<hipStream_t>(stream), *p);
  return launched("k_embed");
}

int stride_k_norm(const StrideNormParams* p, int32_t J, void* stream) {
  if (!p) return fail(STRIDE_TC_EINVAL, "k_norm: null parameters");
  std::string why = lanes_why(p->l, J);
  if (why.empty() && (p->dim <= 0 || p->dim % 4 != 0)) why = "dim must be a positive multiple of 4";
  if (why.empty() && p->l.rows > 0 && (!p->in || !p->out || !p->weight)) why = "missing pointer";
  if (!why.empty()) return fail(STRIDE_TC_EINVAL, "k_norm: " + why);
  if (p->l.rows == 0) return 0;
  hipStream_t st = static_cast<hipStream_t>(stream);
  const int items = J == 1 ? p->dim / 4 : p->dim;
  if (items <= kNormLdsItems) {
    const size_t lds = static_cast<size_t>(items) * 16;
    if (J == 1) hipLaunchKernelGGL(k_exact_norm_lds<1>, dim3(p->l.lane_groups), dim3(256), lds, st, *p);
    else hipLaunchKernelGGL(k_exact_norm_lds<4>, dim3(p->l.lane_groups), dim3(256), lds, st, *p);
    return launched("k_norm");
  }
  const dim3 grid((p->l.lane_groups + 1) / 2);
  if (J == 1) hipLaunchKernelGGL(k_exact_norm<1>, grid, dim3(64), 0, st, *p);
  else hipLaunchKernelGGL(k_exact_norm<4>, grid, dim3(64), 0, st, *p);
  return launched("k_norm");
}

int stride_k_qkv(const StrideQkvParams* p, int32_t J, void* stream) {
  if (!p) return fail(STRIDE_TC_EINVAL, "k_qkv: null parameters");
  std::string why = lanes_why(p->l, J);
  const int D = p->head_dim;
  if (why.empty()) why = mat_why(p->q, "q");
  if (why.empty()) why = mat_why(p->k, "k");
  if (why.empty()) why = mat_why(p->v, "v");
  if (why.empty() && (D <= 0 || D % 4 != 0 || p->kv.head_dim != D)) why = "head_dim must be a positive multiple of 4 matching kv.head_dim";
  if (why.empty() && (p->k.groups != p->v.groups || p->q.cols != p->k.cols || p->k.cols != p->v.cols))
    why = "k and v must have the same groups and all three the same cols";
  if (why.empty()) {
    const int64_t tokens = D > 0 ? p->kv.group_elems / D : 0;
    if (tokens <= 0 || (tokens & (tokens - 1)) != 0) why = "the KV block (group_elems / head_dim) must be a power of two";
  }
  if (why.empty() && p->l.rows > 0 && (!p->x || !p->q_out || !p->rope || !p->row_slot || !p->row_pos || !p->kv.arena || !p->kv.table))
    why = "missing pointer";
  if (!why.empty()) return fail(STRIDE_TC_EINVAL, "k_qkv: " + why);
  return run_gemm<QkvOp>(*p, J, stream, "k_qkv");
}

int stride_k_gemm_residual(const StrideGemmResidualParams* p, int32_t J, void* stream) {
  if (!p) return fail(STRIDE_TC_EINVAL, "k_gemm_residual: null parameters");
  std::string why = lanes_why(p->l, J);
  if (why.empty()) why = mat_why(p->m, "m");
  if (why.empty() && p->l.rows > 0 && (!p->x || !p->h)) why = "missing pointer";
  if (!why.empty()) return fail(STRIDE_TC_EINVAL, "k_gemm_residual: " + why);
  return run_gemm<ResidualOp>(*p, J, stream, "k_gemm_residual");
}

int stride_k_mlp13(const StrideMlp13Params* p, int32_t J, void* stream) {
  if (!p) return fail(STRIDE_TC_EINVAL, "k_mlp13: null parameters");
  std::string why = lanes_why(p->l, J);
  if (why.empty()) why = mat_why(p->w1, "w1");
  if (why.empty()) why = mat_why(p->w3, "w3");
  if (why.empty() && (p->w1.groups != p->w3.groups || p->w1.cols != p->w3.cols)) why = "w1 and w3 must have the same shape";
  if (why.empty() && p->l.rows > 0 && (!p->x || !p->z)) why = "missing pointer";
  if (!why.empty()) return fail(STRIDE_TC_EINVAL, "k_mlp13: " + why);
  return run_gemm<Mlp13Op>(*p, J, stream, "k_mlp13");
}

int stride_k_compact(const StrideCompactParams* p, void* stream) {
  if (!p || p->lm_count < 0 || p->dim <= 0 || (p->lm_count > 0 && (!p->in || !p->out || !p->lm_rows)) ||
      p->lm_stride < p->lm_count)
    return fail(STRIDE_TC_EINVAL, "k_compact: need lm_count >= 0, dim > 0, lm_stride >= lm_count and pointers");
  if (p->lm_count == 0) return 0;
  hipLaunchKernelGGL(k_exact_compact, dim3((p->dim + 63) / 64), dim3(64), 0, static_cast<hipStream_t>(stream), *p);
  return launched("k_compact");
}

int stride_k_lm_greedy(const StrideLmGreedyParams* p, int32_t J, void* stream) {
  if (!p) return fail(STRIDE_TC_EINVAL, "k_lm_greedy: null parameters");
  std::string why = lanes_why(p->l, J);
  if (why.empty()) why = mat_why(p->m, "m");
  if (why.empty() && (p->vocab <= 0 || p->vocab > p->m.groups * 4)) why = "vocab must be in (0, 4 * groups]";
  if (why.empty() && p->l.rows > 0 && (!p->x || !p->best)) why = "missing pointer";
  if (!why.empty()) return fail(STRIDE_TC_EINVAL, "k_lm_greedy: " + why);
  return run_gemm<LmGreedyOp>(*p, J, stream, "k_lm_greedy");
}

int stride_k_lm_full(const StrideLmFullParams* p, int32_t J, void* stream) {
  if (!p) return fail(STRIDE_TC_EINVAL, "k_lm_full: null parameters");
  std::string why = lanes_why(p->l, J);
  if (why.empty()) why = mat_why(p->m, "m");
  if (why.empty() && p->l.rows > 0 && (!p->x || !p->logits)) why = "missing pointer";
  if (!why.empty()) return fail(STRIDE_TC_EINVAL, "k_lm_full: " + why);
  return run_gemm<LmFullOp>(*p, J, stream, "k_lm_full");
}

}  // extern "C"
