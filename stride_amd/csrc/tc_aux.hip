// The non-GEMM entry points of stride's tensor-core path for MI355X (gfx950):
// token embedding into fp32 h tiles, RMSNorm from h to bf16 x tiles, paged
// attention over bf16 KV, and lane compaction. They complete the operator
// surface of the reference's src/kernels_tc.h:79-87, so an engine linking this
// library needs no other device code for a decode step.
//
// Each follows the reference's fixed summation trees exactly (the order of every
// fmaf and add, src/kernels_tc.cu:179-340, src/kernel_common.h:84-309), so the
// results do not depend on the batch, the lane position or the launch shape.
// Work is spread over 64-wide wavefronts wherever the tree leaves freedom
// (independent positions, dimensions and lanes); sequential sums stay sequential.
#include <hip/hip_runtime.h>

#include <cstddef>
#include <string>

#include "../../include/stride_exact.h"
#include "tc_common.hpp"

namespace stride_tc {

int fail(int code, const std::string& msg);  // tc_gemm.hip

namespace {

// Attention summation page: 64 positions (src/kernels.h:20-21). A numeric
// constant of the tree, independent of the KV storage page size.
constexpr int kAttnPageShift = 6;
constexpr int kAttnPage = 1 << kAttnPageShift;
constexpr int kHeadsPerGroup = 4;  // the reference's float4 query packing

// Maximum over the 64 lanes of a wave, in registers: DPP within each row of 16
// lanes (neighbours in a quad, then rotations by 4 and 8), then the row swaps
// of gfx950 (v_permlane16_swap, v_permlane32_swap; each lane receives its own
// value or its partner row's in the two results, so both are folded in). Each
// step keeps the larger of two values (a strict > pick); scores are sums from a
// +0 start, never -0, so the maximum is the same value whatever the pairing.
template <int CTRL>
__device__ __forceinline__ float dpp_f32(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xF, 0xF, false));
}
__device__ __forceinline__ float pick_gt(float o, float m) { return o > m ? o : m; }
__device__ __forceinline__ float wave_max(float m) {
  m = pick_gt(dpp_f32<0xB1>(m), m);   // quad_perm [1,0,3,2]
  m = pick_gt(dpp_f32<0x4E>(m), m);   // quad_perm [2,3,0,1]
  m = pick_gt(dpp_f32<0x124>(m), m);  // row_ror:4
  m = pick_gt(dpp_f32<0x128>(m), m);  // row_ror:8
  const auto r16 = __builtin_amdgcn_permlane16_swap(__float_as_uint(m), __float_as_uint(m), false, false);
  m = pick_gt(__uint_as_float(r16[0]), m);
  m = pick_gt(__uint_as_float(r16[1]), m);
  const auto r32 = __builtin_amdgcn_permlane32_swap(__float_as_uint(m), __float_as_uint(m), false, false);
  m = pick_gt(__uint_as_float(r32[0]), m);
  m = pick_gt(__uint_as_float(r32[1]), m);
  return m;
}

// ---------------------------------------------------------------------------
// Embedding: lane j of the h tiles <- fp32(embed row tokens[j]). The embedding
// is the LM head's weight tiles, so row `token` is slot token % 16 of row tile
// token / 16 (src/kernels_tc.cu:179-203). Thread i moves 8 columns.
__global__ __launch_bounds__(256) void k_embed(StrideTcEmbedParams p) {
  const int b = blockIdx.x;
  const int token = p.tokens[b];
  const int rt = token >> 4, slot = token & 15, lt = b >> 4, jj = b & 15;
  const int col_tiles = p.dim >> 4;
  for (int i = threadIdx.x; i < col_tiles * 2; i += blockDim.x) {
    const int ct = i >> 1, half = i & 1;
    const uint16_t* src = p.embed + (static_cast<int64_t>(rt) * col_tiles + ct) * kTileElems + slot * 16 + half * 8;
    float* dst = p.h + ((static_cast<int64_t>(lt) * col_tiles + ct) * 16 + jj) * 16 + half * 8;
    const u32x4 w = load16(src);
    f32x4 lo, hi;
#pragma unroll
    for (int k = 0; k < 2; ++k) {
      lo[2 * k] = f32_of(w[k] << 16);
      lo[2 * k + 1] = f32_of(w[k] & 0xFFFF0000u);
      hi[2 * k] = f32_of(w[k + 2] << 16);
      hi[2 * k + 1] = f32_of(w[k + 2] & 0xFFFF0000u);
    }
    reinterpret_cast<f32x4*>(dst)[0] = lo;
    reinterpret_cast<f32x4*>(dst)[1] = hi;
  }
}

// ---------------------------------------------------------------------------
// RMSNorm, one wave per lane. Lanes 0..31 of the wave compute the reference's
// 32 partials (partial t: fmaf over columns 0..15 of column tiles ct == t mod
// 32, ascending); lane 0 adds them left to right; then x = bf16(g * (v * r))
// (src/kernels_tc.cu:205-271, 276-340). With TPL > 0 (dim == 32 * 16 * TPL)
// each of lanes 0..31 keeps its TPL tiles and their gains in registers, so h
// is read once; TPL == 0 is the general form.
template <int TPL>
__global__ __launch_bounds__(64) void k_norm(StrideTcNormParams p, int per_lane) {
  const int b = blockIdx.x;  // lane index in [0, lane_groups * 16)
  const int lane = threadIdx.x;
  const int lt = b >> 4, j = b & 15;
  const int col_tiles = p.dim >> 4;
  const int64_t row0 = static_cast<int64_t>(lt) * col_tiles * kTileElems + j * 16;
  auto tile = [&](int ct) { return row0 + static_cast<int64_t>(ct) * kTileElems; };
  auto store = [&](int ct, const f32x4* v, const f32x4* g, float r) {
    uint32_t o[8];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const uint32_t b0 = bf16_rne(g[q][0] * (v[q][0] * r)), b1 = bf16_rne(g[q][1] * (v[q][1] * r));
      const uint32_t b2 = bf16_rne(g[q][2] * (v[q][2] * r)), b3 = bf16_rne(g[q][3] * (v[q][3] * r));
      o[2 * q] = b0 | (b1 << 16);
      o[2 * q + 1] = b2 | (b3 << 16);
    }
    u32x4* out = reinterpret_cast<u32x4*>(p.x + tile(ct));
    out[0] = u32x4{o[0], o[1], o[2], o[3]};
    out[1] = u32x4{o[4], o[5], o[6], o[7]};
  };
  if (b >= p.l.rows) {
    if (per_lane) return;
    for (int ct = lane; ct < col_tiles; ct += 64) {
      u32x4* out = reinterpret_cast<u32x4*>(p.x + tile(ct));
      out[0] = u32x4{0u, 0u, 0u, 0u};
      out[1] = u32x4{0u, 0u, 0u, 0u};
    }
    return;
  }
  // The 32 lane partials added left to right, ((p0 + p1) + p2) + ..., from
  // registers (every lane forms the same sum), then r = 1 / sqrt(sum / dim + eps).
  auto inv_rms = [&](float acc) {
    float sum = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(acc), 0));
#pragma unroll
    for (int i = 1; i < 32; ++i) sum = sum + __int_as_float(__builtin_amdgcn_readlane(__float_as_int(acc), i));
    return 1.0f / sqrtf(sum / static_cast<float>(p.dim) + p.eps);
  };
  if constexpr (TPL > 0) {
    f32x4 v[TPL][4], g[TPL][4];
    float acc = 0.0f;
    if (lane < 32) {
#pragma unroll
      for (int k = 0; k < TPL; ++k) {
        const f32x4* src = reinterpret_cast<const f32x4*>(p.h + tile(lane + 32 * k));
        const f32x4* gs = reinterpret_cast<const f32x4*>(p.weight + (lane + 32 * k) * 16);
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          v[k][q] = src[q];
          g[k][q] = gs[q];
        }
      }
#pragma unroll
      for (int k = 0; k < TPL; ++k)
#pragma unroll
        for (int q = 0; q < 4; ++q)
#pragma unroll
          for (int c = 0; c < 4; ++c) acc = __builtin_fmaf(v[k][q][c], v[k][q][c], acc);
    }
    const float r = inv_rms(acc);
    if (lane < 32) {
#pragma unroll
      for (int k = 0; k < TPL; ++k) store(lane + 32 * k, v[k], g[k], r);
    }
  } else {
    float acc = 0.0f;
    if (lane < 32) {
      for (int ct = lane; ct < col_tiles; ct += 32) {
        const f32x4* v = reinterpret_cast<const f32x4*>(p.h + tile(ct));
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const f32x4 w = v[q];
#pragma unroll
          for (int c = 0; c < 4; ++c) acc = __builtin_fmaf(w[c], w[c], acc);
        }
      }
    }
    const float r = inv_rms(acc);
    for (int ct = lane; ct < col_tiles; ct += 64) {
      const f32x4* v = reinterpret_cast<const f32x4*>(p.h + tile(ct));
      const f32x4* gv = reinterpret_cast<const f32x4*>(p.weight + ct * 16);
      const f32x4 vv[4] = {v[0], v[1], v[2], v[3]}, gg[4] = {gv[0], gv[1], gv[2], gv[3]};
      store(ct, vv, gg, r);
    }
  }
}

// ---------------------------------------------------------------------------
// Lane compaction: out lane l <- in lane lm_rows[l] (src/kernels_tc.cu:566-587).
__global__ __launch_bounds__(64) void k_compact(StrideTcCompactParams p) {
  const int b = blockIdx.x;
  const int src = p.lm_rows[b];
  const int64_t in0 = static_cast<int64_t>(src >> 4) * p.col_tiles * kTileElems + (src & 15) * 16;
  const int64_t out0 = static_cast<int64_t>(b >> 4) * p.col_tiles * kTileElems + (b & 15) * 16;
  for (int ct = threadIdx.x; ct < p.col_tiles; ct += 64) {
    const u32x4* in = reinterpret_cast<const u32x4*>(p.in + in0 + static_cast<int64_t>(ct) * kTileElems);
    u32x4* out = reinterpret_cast<u32x4*>(p.out + out0 + static_cast<int64_t>(ct) * kTileElems);
    out[0] = in[0];
    out[1] = in[1];
  }
}

// ---------------------------------------------------------------------------
// Attention.

// K or V row of position pos for KV group `group` (src/kernel_common.h:20-25),
// with the storage page given by the arena geometry.
template <class KvT>
__device__ __forceinline__ const KvT* kv_row(const StrideKvRef& kv, int page_shift, int layer, int which, int group,
                                             int slot, int pos) {
  const int64_t block = kv.table[static_cast<int64_t>(slot) * kv.max_blocks + (pos >> page_shift)];
  const int token = pos & ((1 << page_shift) - 1);
  return static_cast<const KvT*>(kv.arena) + block * kv.block_elems + layer * kv.layer_elems +
         which * kv.which_elems + group * kv.group_elems + static_cast<int64_t>(token) * kv.head_dim;
}

// One (row, page) item for one KV group (src/kernel_common.h:84-250). The page's
// V rows are fetched with 16-byte loads and parked in LDS, and each lane's K row
// is fetched whole, so both latencies overlap. Lane i scores position p0 + i for
// the four query heads (an fmaf chain over the head dims in order, then times
// scale); the page maximum is order-free; the exponentials follow. Each lane
// then mixes the values of its dims over the positions in order; in the same
// pass lane h < 4 adds head h's weights left to right (one LDS word per
// position), which yields the denominators without a serial phase and without
// every lane repeating the four adds.
// KvT is uint16_t (bf16 KV, the tensor-core path) or float (the exact path);
// the arithmetic is the same, on the widened values.
template <int D, class KvT>
__global__ __launch_bounds__(64) void k_attn_page(StrideAttentionParams p, int page_shift) {
  constexpr int kEl = 16 / static_cast<int>(sizeof(KvT));  // elements per 16-byte piece
  constexpr int kPieces = kAttnPage * D / kEl;  // 16-byte pieces of one page of V
  constexpr int kPer = kPieces / 64;            // per lane
  constexpr int kKey = D / kEl;                 // 16-byte pieces of one K row
  const int item = blockIdx.x / p.n_kv;
  const int g = blockIdx.x % p.n_kv;
  const int lane = threadIdx.x;
  const int j = p.items[2 * item];
  const int page = p.items[2 * item + 1];
  // An item outside the record array (page >= max_pages) would write into the next
  // row's records: it is skipped (the caller sizes max_pages for its longest row).
  if (page < 0 || page >= p.max_pages) return;
  const int slot = p.row_slot[j];
  const int visible = p.row_pos[j] + 1;
  const int p0 = page << kAttnPageShift;
  const int n = min(visible - p0, kAttnPage);
  __shared__ f32x4 q4[D];        // the four heads' query values, per dim
  __shared__ f32x4 w4[kAttnPage];  // the four heads' weights, per position
  __shared__ KvT vs[kAttnPage][D];

  // Positions past the row's last one are clamped to it (their values are never
  // used), so every load is unconditional and stays inside the row's own pages.
  const int last = visible - 1;
  u32x4 vr[kPer], kr[kKey];
#pragma unroll
  for (int k = 0; k < kPer; ++k) {
    const int P = k * 64 + lane, i = P / (D / kEl), c = P % (D / kEl);
    vr[k] = ld_kv(kv_row<KvT>(p.kv, page_shift, p.layer, 1, g, slot, min(p0 + i, last)) + c * kEl);
  }
  {
    const KvT* key = kv_row<KvT>(p.kv, page_shift, p.layer, 0, g, slot, min(p0 + lane, last));
#pragma unroll
    for (int c = 0; c < kKey; ++c) kr[c] = load16(key + kEl * c);
  }
  const float* qrow = p.q + static_cast<int64_t>(j) * p.q_stride + static_cast<int64_t>(g * kHeadsPerGroup) * D;
  for (int d = lane; d < D; d += 64)
    q4[d] = f32x4{qrow[d], qrow[D + d], qrow[2 * D + d], qrow[3 * D + d]};
#pragma unroll
  for (int k = 0; k < kPer; ++k) {
    const int P = k * 64 + lane;
    *reinterpret_cast<u32x4*>(&vs[P / (D / kEl)][(P % (D / kEl)) * kEl]) = vr[k];
  }
  __syncthreads();

  float a0 = 0.0f, a1 = 0.0f, a2 = 0.0f, a3 = 0.0f;
#pragma unroll
  for (int c = 0; c < kKey; ++c) {
#pragma unroll
    for (int e = 0; e < kEl; ++e) {
      float k;
      if constexpr (kEl == 8) k = f32_of(e & 1 ? kr[c][e >> 1] & 0xFFFF0000u : kr[c][e >> 1] << 16);
      else k = f32_of(kr[c][e]);
      const f32x4 qd = q4[kEl * c + e];
      a0 = __builtin_fmaf(qd[0], k, a0);
      a1 = __builtin_fmaf(qd[1], k, a1);
      a2 = __builtin_fmaf(qd[2], k, a2);
      a3 = __builtin_fmaf(qd[3], k, a3);
    }
    __builtin_amdgcn_sched_barrier(0);  // keep each chunk's query reads next to their use
  }
  const float neg_inf = f32_of(0xFF800000u);
  float sc[kHeadsPerGroup] = {a0 * p.scale, a1 * p.scale, a2 * p.scale, a3 * p.scale};
  f32x4 mx;
#pragma unroll
  for (int h = 0; h < kHeadsPerGroup; ++h) {
    if (lane >= n) sc[h] = neg_inf;
    mx[h] = wave_max(sc[h]);
  }
  if (lane < n) w4[lane] = f32x4{det_exp(sc[0] - mx[0]), det_exp(sc[1] - mx[1]), det_exp(sc[2] - mx[2]), det_exp(sc[3] - mx[3])};
  __syncthreads();
  float* rec = p.scratch + (static_cast<int64_t>(j * p.n_kv + g) * p.max_pages + page) * p.rec_floats;
  float* v_out = rec + 8;
  const float* wflat = reinterpret_cast<const float*>(w4);
  float den = 0.0f;  // head (lane & 3)
#pragma unroll
  for (int it = 0; it < (D + 63) / 64; ++it) {
    const int d = lane + 64 * it;
    if (d >= D) continue;
    f32x4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll 4
    for (int i = 0; i < n; ++i) {
      float v;
      if constexpr (kEl == 8) v = f32_of(static_cast<uint32_t>(vs[i][d]) << 16);
      else v = vs[i][d];
      const f32x4 wi = w4[i];
#pragma unroll
      for (int h = 0; h < kHeadsPerGroup; ++h) acc[h] = __builtin_fmaf(wi[h], v, acc[h]);
      if (it == 0) den = den + wflat[i * kHeadsPerGroup + (lane & 3)];
    }
#pragma unroll
    for (int h = 0; h < kHeadsPerGroup; ++h) v_out[h * D + d] = acc[h];
  }
  if (lane < kHeadsPerGroup) {
    rec[lane] = mx[lane];
    rec[4 + lane] = den;
  }
}

// Ascending-page combine of one row's records for one KV group, written as bf16
// x tiles (src/kernel_common.h:252-309, writer src/kernels_tc.cu:658-666) or,
// for the exact path, as fp32 dim-major out[idx * stride + row] (LaneWriter,
// src/kernels.cu:287-291). All
// of the row's records come into LDS in one coalesced pass; threads 0..3 derive
// each head's page factors and denominator (pages in order); thread (h, d) then
// folds the weighted values of head h, dim d over the pages in order.
template <int D, bool kExact>
__global__ __launch_bounds__(256) void k_attn_combine(StrideAttentionParams p) {
  extern __shared__ float recs[];  // [pages][rec_floats], then f[4][pages]
  __shared__ float den[kHeadsPerGroup];
  const int j = blockIdx.x / p.n_kv;
  const int g = blockIdx.x % p.n_kv;
  const int t = threadIdx.x;
  const int pages = min((p.row_pos[j] >> kAttnPageShift) + 1, p.max_pages);  // row_pos < 64 * max_pages
  const int rf = p.rec_floats;
  const float* src = p.scratch + static_cast<int64_t>(j * p.n_kv + g) * p.max_pages * rf;
  for (int i = t; i < pages * rf; i += 256) recs[i] = src[i];
  float* f = recs + pages * rf;
  __syncthreads();
  if (t < kHeadsPerGroup) {
    float m = f32_of(0xFF800000u);
    for (int c = 0; c < pages; ++c) {
      const float mc = recs[c * rf + t];
      if (mc > m) m = mc;
    }
    float d = 0.0f;
    for (int c = 0; c < pages; ++c) {
      const float e = det_exp(recs[c * rf + t] - m);
      f[t * pages + c] = e;
      d = __builtin_fmaf(e, recs[c * rf + 4 + t], d);
    }
    den[t] = d;
  }
  __syncthreads();
  const int col_tiles = p.out_cols >> 4;
  uint16_t* out = static_cast<uint16_t*>(p.out);
  const int64_t lane0 = static_cast<int64_t>(j >> 4) * col_tiles * kTileElems + (j & 15) * 16;
  for (int hd = t; hd < p.n_q * D; hd += 256) {
    const int qh = hd / D, d = hd % D;
    float acc = 0.0f;
    for (int c = 0; c < pages; ++c) acc = __builtin_fmaf(f[qh * pages + c], recs[c * rf + 8 + qh * D + d], acc);
    const int idx = (g * p.n_q + qh) * D + d;
    if constexpr (kExact) static_cast<float*>(p.out)[static_cast<int64_t>(idx) * p.l.stride + j] = acc / den[qh];
    else out[lane0 + static_cast<int64_t>(idx >> 4) * kTileElems + (idx & 15)] = static_cast<uint16_t>(bf16_rne(acc / den[qh]));
  }
}

// Pages and combine in one kernel. One workgroup per (row, KV group): its NWV
// waves take the row's 64-position pages round robin, each summing a page
// exactly as k_attn_page does (the same expressions in the same order) into a
// record kept in LDS; after a barrier the workgroup combines the records in
// ascending page order exactly as k_attn_combine does and writes the bf16 x
// tiles (KvT = uint16_t: bf16 KV, the tensor-core path) or the fp32 dim-major
// output (KvT = float, kExact: the exact path's fp32 KV). No second launch is
// needed.
//
// LIST = false: item_count == -1, every page of every row is computed.
// LIST = true: the caller's (row, page) item list decides, with the semantics of
// the page + combine pair (listed pages are summed now, the others are combined
// from the records `scratch` holds). The list the reference's engine builds
// (src/engine.cpp:93-103: rows ascending, each row's pages 0 .. last ascending)
// puts row j's items at offset sum_{i<j} pages_i; the workgroup computes that
// offset from row_pos and checks its row's stretch of the list. When it matches
// (every page listed) the records stay in LDS and scratch is not touched.
// Otherwise the workgroup scans the whole list for its row, sums the listed
// pages, reads the unlisted pages' records from scratch and stores the records
// it summed there, as k_attn_page would.
constexpr int kListMaxPages = 320;  // pages a LIST workgroup tracks (the LDS bound is lower)

template <int D, int NWV, bool LIST, class KvT = uint16_t, bool kExact = false>
__global__ __launch_bounds__(64 * NWV) void k_attn_fused(StrideAttentionParams p, int page_shift) {
  constexpr int kEl = 16 / static_cast<int>(sizeof(KvT));  // KV elements per 16-byte piece
  constexpr int kPer = kAttnPage * D / kEl / 64;  // V pieces per lane
  constexpr int kKey = D / kEl;                 // 16-byte pieces of one K row
  constexpr int RF = 8 + kHeadsPerGroup * D;    // record floats
  extern __shared__ float recs[];  // [max_pages][RF], f[4][max_pages], then the row's KV page numbers
  __shared__ f32x4 w4[NWV][kAttnPage];
  __shared__ KvT vs[NWV][kAttnPage][D];
  __shared__ uint32_t listed[LIST ? kListMaxPages / 32 : 1];
  __shared__ int part[NWV];
  const int j = blockIdx.x / p.n_kv;
  const int g = blockIdx.x % p.n_kv;
  const int t = threadIdx.x, wave = t >> 6, lane = t & 63;
  const int slot = p.row_slot[j];
  const int visible = p.row_pos[j] + 1;
  const int last = visible - 1;
  // A row must satisfy row_pos < max_pages * 64 (the caller sizes max_pages for
  // its longest row); the clamp keeps a row past it inside this workgroup's LDS.
  const int pages = min((last >> kAttnPageShift) + 1, p.max_pages);
  // The row's KV page numbers, read once: every K/V address below then comes
  // from LDS, so a page's loads never wait on a dependent page-table load.
  int32_t* btab = reinterpret_cast<int32_t*>(recs + p.max_pages * (RF + kHeadsPerGroup));
  const int nblk = min((last >> page_shift) + 1, (p.max_pages * kAttnPage + (1 << page_shift) - 1) >> page_shift);
  for (int i = t; i < nblk; i += 64 * NWV) btab[i] = p.kv.table[static_cast<int64_t>(slot) * p.kv.max_blocks + i];
  const KvT* kv_base = static_cast<const KvT*>(p.kv.arena) + p.layer * p.kv.layer_elems + g * p.kv.group_elems;
  auto kv_at = [&](int which, int pos) {
    return kv_base + btab[pos >> page_shift] * p.kv.block_elems + which * p.kv.which_elems +
           static_cast<int64_t>(pos & ((1 << page_shift) - 1)) * D;
  };
  __syncthreads();
  const float* qrow = p.q + static_cast<int64_t>(j) * p.q_stride + static_cast<int64_t>(g * kHeadsPerGroup) * D;
  // The query row is the same for every lane: read through the scalar cache into
  // SGPRs, so the scores take their query operands without LDS reads.
  typedef const __attribute__((address_space(4))) float ConstF;
  ConstF* cq = (ConstF*)(qrow);
  const float neg_inf = f32_of(0xFF800000u);
  const int rounds = (pages + NWV - 1) / NWV;  // the same for every wave: barriers stay uniform
  // K and V of the wave's next page are loaded into registers one round ahead:
  // they stream in while the current page is scored and mixed.
  u32x4 vr[kPer], kr[kKey];
  auto fetch = [&](int page) {
    const int p0 = page << kAttnPageShift;
#pragma unroll
    for (int k = 0; k < kPer; ++k) {
      const int P = k * 64 + lane, i = P / (D / kEl), c = P % (D / kEl);
      vr[k] = ld_kv(kv_at(1, min(p0 + i, last)) + c * kEl);
    }
    const KvT* key = kv_at(0, min(p0 + lane, last));
#pragma unroll
    for (int c = 0; c < kKey; ++c) kr[c] = load16(key + kEl * c);
  };
  // LIST: does the item list hold row j's pages where the engine's list puts them?
  // (The page counts of the rows before j are loaded before the first page, so
  // the check's loads overlap that page's.)
  int s = 0;
  if constexpr (LIST)
    for (int i = t; i < j; i += 64 * NWV) s += (p.row_pos[i] >> kAttnPageShift) + 1;
  if (wave < pages) fetch(wave);
  // Round 0 runs before the list check completes and sums whichever pages it
  // takes; if the check then fails, the unlisted pages' records are replaced
  // from scratch before anything reads them.
  bool whole = true, checked = !LIST;
  int list_ok = 1, off_list = 0;
  int32_t item_row = 0, item_page = 0;
  auto is_listed = [&](int page) { return !checked || whole || ((listed[page >> 5] >> (page & 31)) & 1u); };
  for (int it = 0; it < rounds; ++it) {
    const int page = it * NWV + wave;
    const bool active = page < pages && is_listed(page);
    const int p0 = page << kAttnPageShift;
    const int n = active ? min(visible - p0, kAttnPage) : 0;
    if (active) {
#pragma unroll
      for (int k = 0; k < kPer; ++k) {
        const int P = k * 64 + lane;
        *reinterpret_cast<u32x4*>(&vs[wave][P / (D / kEl)][(P % (D / kEl)) * kEl]) = vr[k];
      }
    }
    if constexpr (LIST) {
      if (it == 0) {
#pragma unroll
        for (int off = 32; off > 0; off >>= 1) s += __shfl_xor(s, off);
        if (lane == 0) part[wave] = s;
      }
    }
    __syncthreads();  // this wave's V rows
    if constexpr (LIST) {
      if (it == 0) {  // row j's stretch of the list: loads issued now, compared at the end of the round
#pragma unroll
        for (int w = 0; w < NWV; ++w) off_list += part[w];
        list_ok = off_list + pages <= p.item_count;
        if (list_ok && t < pages) {
          item_row = p.items[2 * (off_list + t)];
          item_page = p.items[2 * (off_list + t) + 1];
        } else {
          item_row = j;
          item_page = t;
        }
      }
    }
    f32x4 mx = {0.f, 0.f, 0.f, 0.f};
    float sc[kHeadsPerGroup] = {0.f, 0.f, 0.f, 0.f};
    if (active) {
      float a0 = 0.0f, a1 = 0.0f, a2 = 0.0f, a3 = 0.0f;
#pragma unroll
      for (int c = 0; c < kKey; ++c) {
#pragma unroll
        for (int e = 0; e < kEl; ++e) {
          float k;
          if constexpr (kEl == 8) k = f32_of(e & 1 ? kr[c][e >> 1] & 0xFFFF0000u : kr[c][e >> 1] << 16);
          else k = f32_of(kr[c][e]);
          const int d = kEl * c + e;
          const f32x4 qd = f32x4{cq[d], cq[D + d], cq[2 * D + d], cq[3 * D + d]};
          a0 = __builtin_fmaf(qd[0], k, a0);
          a1 = __builtin_fmaf(qd[1], k, a1);
          a2 = __builtin_fmaf(qd[2], k, a2);
          a3 = __builtin_fmaf(qd[3], k, a3);
        }
        __builtin_amdgcn_sched_barrier(0);
      }
      sc[0] = a0 * p.scale;
      sc[1] = a1 * p.scale;
      sc[2] = a2 * p.scale;
      sc[3] = a3 * p.scale;
    }
    if (page + NWV < pages) fetch(page + NWV);  // registers are free again
    if (active) {
#pragma unroll
      for (int h = 0; h < kHeadsPerGroup; ++h) {
        if (lane >= n) sc[h] = neg_inf;
        mx[h] = wave_max(sc[h]);
      }
      if (lane < n)
        w4[wave][lane] = f32x4{det_exp(sc[0] - mx[0]), det_exp(sc[1] - mx[1]), det_exp(sc[2] - mx[2]), det_exp(sc[3] - mx[3])};
    }
    __syncthreads();  // this wave's weights
    if (active) {
      float* rec = recs + page * RF;
      const float* wflat = reinterpret_cast<const float*>(w4[wave]);
      float dn = 0.0f;  // head (lane & 3)
#pragma unroll
      for (int itd = 0; itd < (D + 63) / 64; ++itd) {
        const int d = lane + 64 * itd;
        if (d >= D) continue;
        f32x4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll 8
        for (int i = 0; i < n; ++i) {
          float v;
          if constexpr (kEl == 8) v = f32_of(static_cast<uint32_t>(vs[wave][i][d]) << 16);
          else v = vs[wave][i][d];
          const f32x4 wi = w4[wave][i];
#pragma unroll
          for (int h = 0; h < kHeadsPerGroup; ++h) acc[h] = __builtin_fmaf(wi[h], v, acc[h]);
          if (itd == 0) dn = dn + wflat[i * kHeadsPerGroup + (lane & 3)];
        }
#pragma unroll
        for (int h = 0; h < kHeadsPerGroup; ++h) rec[8 + h * D + d] = acc[h];
      }
      if (lane < kHeadsPerGroup) {
        rec[lane] = mx[lane];
        rec[4 + lane] = dn;
      }
    }
    __syncthreads();  // the staging buffers are reused by the next round
    if constexpr (LIST) {
      if (it == 0) {
        int ok = list_ok && item_row == j && item_page == t;
        for (int c = t + 64 * NWV; ok && c < pages; c += 64 * NWV)  // rows of more pages than threads
          ok = p.items[2 * (off_list + c)] == j && p.items[2 * (off_list + c) + 1] == c;
        whole = __syncthreads_and(ok) != 0;
        checked = true;
        if (!whole) {
          for (int i = t; i < kListMaxPages / 32; i += 64 * NWV) listed[i] = 0u;
          __syncthreads();
          for (int i = t; i < p.item_count; i += 64 * NWV) {
            const int c = p.items[2 * i + 1];
            if (p.items[2 * i] == j && c >= 0 && c < pages) atomicOr(&listed[c >> 5], 1u << (c & 31));
          }
          __syncthreads();
          // unlisted pages: the records an earlier call left in scratch (over
          // whatever round 0 summed for them)
          const float* src = p.scratch + static_cast<int64_t>(j * p.n_kv + g) * p.max_pages * p.rec_floats;
          for (int u = t; u < pages * RF; u += 64 * NWV) {
            const int c = u / RF, e = u % RF;
            if (!((listed[c >> 5] >> (c & 31)) & 1u)) recs[c * RF + e] = src[static_cast<int64_t>(c) * p.rec_floats + e];
          }
          __syncthreads();
        }
      }
    }
  }
  if constexpr (LIST) {
    if (!whole) {  // store the summed records, as the page kernel does
      float* dst = p.scratch + static_cast<int64_t>(j * p.n_kv + g) * p.max_pages * p.rec_floats;
      for (int u = t; u < pages * RF; u += 64 * NWV) {
        const int c = u / RF, e = u % RF;
        if ((listed[c >> 5] >> (c & 31)) & 1u) dst[static_cast<int64_t>(c) * p.rec_floats + e] = recs[c * RF + e];
      }
    }
  }
  // Combine in ascending page order (k_attn_combine's expressions). Each page
  // factor is computed by its own thread; every thread derives the head maximum
  // with the same ascending loop, so all agree; each output thread then forms
  // its head's denominator and its dim's sum over the pages in order.
  float* f = recs + pages * RF;
  for (int u = t; u < kHeadsPerGroup * pages; u += 64 * NWV) {
    const int h = u & 3, c = u >> 2;
    float m = neg_inf;
    for (int c2 = 0; c2 < pages; ++c2) {
      const float mc = recs[c2 * RF + h];
      if (mc > m) m = mc;
    }
    f[h * pages + c] = det_exp(recs[c * RF + h] - m);
  }
  __syncthreads();
  const int col_tiles = p.out_cols >> 4;
  uint16_t* out = static_cast<uint16_t*>(p.out);
  const int64_t lane0 = kExact ? 0 : static_cast<int64_t>(j >> 4) * col_tiles * kTileElems + (j & 15) * 16;
  for (int hd = t; hd < kHeadsPerGroup * D; hd += 64 * NWV) {
    const int qh = hd / D, d = hd % D;
    float acc = 0.0f, dn = 0.0f;
    for (int c = 0; c < pages; ++c) {
      const float e = f[qh * pages + c];
      dn = __builtin_fmaf(e, recs[c * RF + 4 + qh], dn);
      acc = __builtin_fmaf(e, recs[c * RF + 8 + qh * D + d], acc);
    }
    const int idx = (g * kHeadsPerGroup + qh) * D + d;
    if constexpr (kExact) static_cast<float*>(p.out)[static_cast<int64_t>(idx) * p.l.stride + j] = acc / dn;
    else out[lane0 + static_cast<int64_t>(idx >> 4) * kTileElems + (idx & 15)] = static_cast<uint16_t>(bf16_rne(acc / dn));
  }
}

bool lanes_valid(const StrideLanes& l) { return l.rows >= 0 && l.lane_groups == (l.rows + 15) / 16; }

}  // namespace
}  // namespace stride_tc

using namespace stride_tc;

static_assert(sizeof(StrideTcEmbedParams) == 48, "TcEmbedParams layout");
static_assert(sizeof(StrideTcNormParams) == 48, "TcNormParams layout");
static_assert(sizeof(StrideTcCompactParams) == 48, "TcCompactParams layout");
static_assert(offsetof(StrideAttentionParams, kv) == 48 && sizeof(StrideAttentionParams) == 176,
              "AttentionParams layout");

static int launched(const char* what);

// The combine keeps a row's records in LDS; past the default 64 KiB of dynamic
// LDS (long contexts at head_dim 128) the kernel's limit is raised once.
// (The kernel's own static LDS shares the 160 KiB, hence the margin.)
constexpr size_t kCombineLdsMax = 159 * 1024;

template <int D, bool kExact>
static int combine(dim3 grid, size_t lds, hipStream_t st, const StrideAttentionParams& p) {
  static size_t raised = 64 * 1024;
  if (lds > raised) {
    const hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(&k_attn_combine<D, kExact>),
                                             hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(lds));
    if (e != hipSuccess) return fail(static_cast<int>(e), std::string("tc_attention: raising the LDS limit failed: ") + hipGetErrorString(e));
    raised = lds;
  }
  hipLaunchKernelGGL((k_attn_combine<D, kExact>), grid, dim3(256), lds, st, p);
  return launched("attention (combine)");
}

// One-kernel attention; its static LDS (staging for up to four waves) and the
// row's records share the 160 KiB.
template <int D, int NWV, class KvT>
constexpr size_t fused_static_lds() {
  return NWV * 64 * 16 + NWV * 64 * D * sizeof(KvT) + kListMaxPages / 8 + 4 * NWV;
}

template <int D, int NWV, bool LIST, class KvT, bool kExact>
static int fused_nwv(dim3 grid, size_t lds, hipStream_t st, const StrideAttentionParams& p, int page_shift) {
  if (lds + fused_static_lds<D, NWV, KvT>() > kCombineLdsMax)
    return fail(STRIDE_TC_EINVAL, "tc_attention: max_pages too large for the one-kernel form (use an item list)");
  static size_t raised = 64 * 1024;
  if (lds > raised) {
    const hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(&k_attn_fused<D, NWV, LIST, KvT, kExact>),
                                             hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(lds));
    if (e != hipSuccess) return fail(static_cast<int>(e), std::string("tc_attention: raising the LDS limit failed: ") + hipGetErrorString(e));
    raised = lds;
  }
  hipLaunchKernelGGL((k_attn_fused<D, NWV, LIST, KvT, kExact>), grid, dim3(64 * NWV), lds, st, p, page_shift);
  return launched("attention (one kernel)");
}

// Waves per workgroup of the one-kernel form, from measurements of the full
// decode step at position 383 (six pages per row): with many (row, group)
// workgroups (batch 128, 1024 of them) two waves per workgroup (three rounds of
// pages) measured best (30.9 us against 32.4 with three and 33+ with four); with
// fewer (batch 64) four waves finish a row sooner.
template <int D, bool LIST, class KvT = uint16_t, bool kExact = false>
static int fused(dim3 grid, size_t lds, hipStream_t st, const StrideAttentionParams& p, int page_shift) {
  if (grid.x >= 768) return fused_nwv<D, 2, LIST, KvT, kExact>(grid, lds, st, p, page_shift);
  return fused_nwv<D, 4, LIST, KvT, kExact>(grid, lds, st, p, page_shift);
}

// Does the one-kernel form serve a call with this dynamic LDS? (4 waves: the
// larger static staging.)
template <int D, class KvT = uint16_t>
static bool fused_fits(size_t lds) {
  return lds + fused_static_lds<D, 4, KvT>() <= kCombineLdsMax;
}

// Item-list calls run the one-kernel form (which checks the list on the device)
// for up to this many rows: each workgroup sums the page counts of the rows
// before its own to find its stretch of the list, which grows with the row count.
constexpr int kListFusedMaxRows = 512;

static int launched(const char* what) {
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(static_cast<int>(e), std::string(what) + " launch failed: " + hipGetErrorString(e));
  return 0;
}

extern "C" {

int stride_tc_embed(const StrideTcEmbedParams* p, void* stream) {
  if (!p || !lanes_valid(p->l) || p->dim <= 0 || p->dim % 16 != 0 || (p->l.rows > 0 && (!p->embed || !p->tokens || !p->h)))
    return fail(STRIDE_TC_EINVAL, "tc_embed: need rows >= 0, lane_groups = ceil(rows/16), dim a positive multiple of 16 and pointers");
  if (p->l.rows == 0) return 0;
  hipLaunchKernelGGL(k_embed, dim3(p->l.rows), dim3(256), 0, static_cast<hipStream_t>(stream), *p);
  return launched("tc_embed");
}

int stride_tc_norm(const StrideTcNormParams* p, int per_lane, void* stream) {
  if (!p || !lanes_valid(p->l) || p->dim <= 0 || p->dim % 16 != 0 ||
      (p->l.rows > 0 && (!p->h || !p->x || !p->weight)))
    return fail(STRIDE_TC_EINVAL, "tc_norm: need rows >= 0, lane_groups = ceil(rows/16), dim a positive multiple of 16 and pointers");
  if (p->l.rows == 0) return 0;
  const dim3 grid(p->l.lane_groups * 16);
  hipStream_t st = static_cast<hipStream_t>(stream);
  const int pl = per_lane ? 1 : 0;
  switch (p->dim) {
    case 512: hipLaunchKernelGGL(k_norm<1>, grid, dim3(64), 0, st, *p, pl); break;
    case 1024: hipLaunchKernelGGL(k_norm<2>, grid, dim3(64), 0, st, *p, pl); break;
    case 2048: hipLaunchKernelGGL(k_norm<4>, grid, dim3(64), 0, st, *p, pl); break;
    case 4096: hipLaunchKernelGGL(k_norm<8>, grid, dim3(64), 0, st, *p, pl); break;
    default: hipLaunchKernelGGL(k_norm<0>, grid, dim3(64), 0, st, *p, pl); break;
  }
  return launched("tc_norm");
}

int stride_tc_compact(const StrideTcCompactParams* p, void* stream) {
  if (!p || p->lm_count < 0 || p->col_tiles <= 0 || (p->lm_count > 0 && (!p->in || !p->out || !p->lm_rows)))
    return fail(STRIDE_TC_EINVAL, "tc_compact: need lm_count >= 0, col_tiles > 0 and pointers");
  if (p->lm_count == 0) return 0;
  hipLaunchKernelGGL(k_compact, dim3(p->lm_count), dim3(64), 0, static_cast<hipStream_t>(stream), *p);
  return launched("tc_compact");
}

}  // extern "C"

// Shared checks and launches of the tensor-core (bf16 KV, bf16 x-tile output)
// and exact (fp32 KV, fp32 dim-major output) attention.
template <bool kExact>
static int attention(const StrideAttentionParams* p, void* stream, const char* name) {
  if (!p) return fail(STRIDE_TC_EINVAL, std::string(name) + ": null parameters");
  const int D = p->head_dim;
  const int64_t page_tokens = D > 0 ? p->kv.group_elems / D : 0;
  int page_shift = 0;
  while (page_shift < 30 && (int64_t{1} << page_shift) < page_tokens) ++page_shift;
  std::string why;
  if (kExact ? (p->l.rows < 0 || p->l.stride < p->l.rows) : !lanes_valid(p->l))
    why = kExact ? "need rows >= 0 and stride >= rows" : "lane_groups must equal ceil(rows/16)";
  else if ((D != 32 && D != 64 && D != 128) || p->kv.head_dim != D) why = "head_dim must be 32, 64 or 128 and match kv.head_dim";
  else if (p->n_q != kHeadsPerGroup) why = "four query heads per KV group are required (the reference packs them in a float4)";
  else if (p->n_kv <= 0 || p->rec_floats < 8 + 4 * D || p->max_pages <= 0 || p->item_count < (kExact ? 0 : -1))
    why = "bad n_kv, rec_floats, max_pages or item_count";
  else if (page_tokens <= 0 || (int64_t{1} << page_shift) != page_tokens) why = "the KV storage page (group_elems / head_dim) must be a power of two";
  else if (!kExact && (p->out_cols % 16 != 0 || p->out_cols < p->n_kv * p->n_q * D)) why = "out_cols must be a multiple of 16 covering every head";
  else if (p->l.rows > 0 && (!p->q || !p->out || !p->kv.arena || !p->kv.table || !p->row_slot || !p->row_pos ||
                             (p->item_count >= 0 && !p->scratch) || (p->item_count > 0 && !p->items)))
    why = "missing pointer";
  else if (static_cast<size_t>(p->max_pages) * (p->rec_floats + kHeadsPerGroup) * sizeof(float) > kCombineLdsMax)
    why = "max_pages * rec_floats too large for the combine's LDS (159 KiB)";
  if (!why.empty()) return fail(STRIDE_TC_EINVAL, std::string(name) + ": " + why);
  if (p->l.rows == 0) return 0;
  hipStream_t st = static_cast<hipStream_t>(stream);
  using KvT = typename std::conditional<kExact, float, uint16_t>::type;
  {
    // records and page factors, then the row's KV page numbers
    const size_t blocks = (static_cast<size_t>(p->max_pages) * kAttnPage + page_tokens - 1) / page_tokens;
    const size_t lds = static_cast<size_t>(p->max_pages) * (8 + 4 * D + kHeadsPerGroup) * sizeof(float) + blocks * 4;
    const dim3 grid(p->l.rows * p->n_kv);
    if constexpr (!kExact) {
      if (p->item_count == -1) {
        if (D == 32) return fused<32, false>(grid, lds, st, *p, page_shift);
        if (D == 64) return fused<64, false>(grid, lds, st, *p, page_shift);
        return fused<128, false>(grid, lds, st, *p, page_shift);
      }
    }
    const bool fits = D == 32 ? fused_fits<32, KvT>(lds) : (D == 64 ? fused_fits<64, KvT>(lds) : fused_fits<128, KvT>(lds));
    if (fits && p->max_pages <= kListMaxPages && p->l.rows <= kListFusedMaxRows) {
      if (D == 32) return fused<32, true, KvT, kExact>(grid, lds, st, *p, page_shift);
      if (D == 64) return fused<64, true, KvT, kExact>(grid, lds, st, *p, page_shift);
      return fused<128, true, KvT, kExact>(grid, lds, st, *p, page_shift);
    }
  }
  if (p->item_count > 0) {
    const dim3 grid(p->item_count * p->n_kv);
    if (D == 32) hipLaunchKernelGGL((k_attn_page<32, KvT>), grid, dim3(64), 0, st, *p, page_shift);
    else if (D == 64) hipLaunchKernelGGL((k_attn_page<64, KvT>), grid, dim3(64), 0, st, *p, page_shift);
    else hipLaunchKernelGGL((k_attn_page<128, KvT>), grid, dim3(64), 0, st, *p, page_shift);
    if (int rc = launched("attention (pages)")) return rc;
  }
  const size_t lds = static_cast<size_t>(p->max_pages) * (p->rec_floats + kHeadsPerGroup) * sizeof(float);
  const dim3 cgrid(p->l.rows * p->n_kv);
  if (D == 32) return combine<32, kExact>(cgrid, lds, st, *p);
  if (D == 64) return combine<64, kExact>(cgrid, lds, st, *p);
  return combine<128, kExact>(cgrid, lds, st, *p);
}

extern "C" int stride_tc_attention(const StrideAttentionParams* p, void* stream) {
  return attention<false>(p, stream, "tc_attention");
}

// Exact path (src/kernels.cu:474-485): fp32 KV, fp32 dim-major output.
extern "C" int stride_k_attention(const StrideAttentionParams* p, void* stream) {
  return attention<true>(p, stream, "k_attention");
}
