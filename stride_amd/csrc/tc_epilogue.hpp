// Problem geometry and the epilogues shared by every GEMM kernel family.
// Epilogues receive one finished 16x16 output tile per matrix in MFMA fragment
// layout (lane l holds batch lane l%16, rows 4*(l/16)+i) and write it in the
// reference's output layout; every kernel variant calls the same functions, so
// the output bits do not depend on which variant ran.
#pragma once

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
  // Cross-workgroup split partials (k_stream with XS): fp32 fragments indexed
  // ((tile * part_splits + split) * mats + m) * 64 + lane, tile = segment tile
  // base + rt * lane_groups + lt, and one arrival counter per (row block, lane
  // group) unit, zero between launches. Unused (null) otherwise.
  float* part;
  int32_t* split_cnt;
  int32_t part_splits;
};

// Spread consecutive logical blocks over one XCD: hardware hands workgroup i to
// XCD i % 8, so logical neighbours (which share weight or activation tiles) are
// made to land on the same L2. Bijective on [0, n).
__device__ __forceinline__ int xcd_remap(int i, int n) {
  const int full = n & ~7;
  if (i >= full) return i;
  return (i & 7) * (full >> 3) + (i >> 3);
}

// Segment i of g with i known only at run time. Selecting among the three by
// value keeps the kernel argument in registers (indexing the argument array with
// a run-time index makes the compiler copy it to scratch memory).
__device__ __forceinline__ Segment seg_at(const Geometry& g, int i) {
  return i == 0 ? g.seg[0] : (i == 1 ? g.seg[1] : g.seg[2]);
}

// Row tile rt of the segments laid end to end: its segment, and its index there.
__device__ __forceinline__ int flat_segment(const Geometry& g, int rt, int& local) {
  const int r0 = g.seg[0].row_tiles, r1 = g.seg[1].row_tiles;
  if (rt < r0) {
    local = rt;
    return 0;
  }
  if (rt < r0 + r1) {
    local = rt - r0;
    return 1;
  }
  local = rt - r0 - r1;
  return 2;
}

// Segment of logical row block rb (made segment-relative), with `per` logical
// blocks per row block of a segment's count.
__device__ __forceinline__ int locate_segment(const Geometry& g, int& rb, int per = 1) {
  int s = 0;
#pragma unroll
  for (int k = 0; k < 2; ++k) {
    if (s == k && k + 1 < g.nseg && rb >= g.seg[k].blocks * per) {
      rb -= g.seg[k].blocks * per;
      s = k + 1;
    }
  }
  return s;
}

// ---------------------------------------------------------------------------
// Epilogues. Each receives one finished 16x16 tile y (fragment layout: lane l
// holds lane l%16, rows 4*(l/16)+i) per matrix and writes it out. They are
// called by whole wavefronts (QKV and the argmax exchange values across lanes).

struct EpiResidual {  // h <- h + W x   (reference src/kernels_tc.cu:438-501)
  static constexpr int kMats = 1;
  static constexpr bool kReduce = false;
  static constexpr bool kInitFromOutput = true;
  struct Out {
    float* h;
    int32_t h_tiles;
  };
  __device__ __forceinline__ static float* at(const Out& o, int rt, int lt, int lane) {
    return o.h + (static_cast<int64_t>(lt) * o.h_tiles + rt) * kTileElems + (lane & 15) * 16 + (lane >> 4) * 4;
  }
  __device__ __forceinline__ static f32x4 init(const Out& o, int rt, int lt, int lane) {
    return *reinterpret_cast<const f32x4*>(at(o, rt, lt, lane));
  }
  __device__ __forceinline__ static void apply(const Out& o, const Geometry&, int, int rt, int lt, const f32x4* y, int lane) {
    *reinterpret_cast<f32x4*>(at(o, rt, lt, lane)) = y[0];
  }
};

struct EpiLogits {  // logits tiles [rt][lt][16 rows][16 lanes]  (src/kernels_tc.cu:632-655)
  static constexpr int kMats = 1;
  static constexpr bool kReduce = false;
  static constexpr bool kInitFromOutput = false;
  struct Out {
    float* logits;
  };
  __device__ __forceinline__ static f32x4 init(const Out&, int, int, int) { return f32x4{0.f, 0.f, 0.f, 0.f}; }
  __device__ __forceinline__ static void apply(const Out& o, const Geometry& g, int, int rt, int lt, const f32x4* y, int lane) {
    float* base = o.logits + (static_cast<int64_t>(rt) * g.lane_groups + lt) * kTileElems + (lane >> 4) * 64 + (lane & 15);
    base[0] = y[0][0];
    base[16] = y[0][1];
    base[32] = y[0][2];
    base[48] = y[0][3];
  }
};

struct EpiGateUp {  // z = bf16(det_silu(W1 x) * (W3 x))  (src/kernels_tc.cu:505-564)
  static constexpr int kMats = 2;
  static constexpr bool kReduce = false;
  static constexpr bool kInitFromOutput = false;
  struct Out {
    uint16_t* z;
    int32_t z_tiles;
  };
  __device__ __forceinline__ static f32x4 init(const Out&, int, int, int) { return f32x4{0.f, 0.f, 0.f, 0.f}; }
  __device__ __forceinline__ static void apply(const Out& o, const Geometry&, int, int rt, int lt, const f32x4* y, int lane) {
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

// Lexicographic merge of argmax candidates (larger value, then smaller index;
// index -1 = none). Associative and commutative, so any merge order gives the
// same result.
__device__ __forceinline__ void arg_merge(float& bv, int32_t& bi, float ov, int32_t oi) {
  if (oi >= 0 && (bi < 0 || better_than(ov, oi, bv, bi))) {
    bv = ov;
    bi = oi;
  }
}

struct EpiArgmax {  // per-lane greedy argmax  (src/kernels_tc.cu:590-630)
  static constexpr int kMats = 1;
  static constexpr bool kInitFromOutput = false;
  // Kernels reduce the candidates of all row tiles a workgroup owns before they
  // touch `best`, so each lane sees one compare-and-swap per workgroup instead
  // of one per row tile (thousands of racing updates otherwise serialise).
  static constexpr bool kReduce = true;
  struct Out {
    StrideBestEntry* best;
    int32_t vocab;
    // When set, a workgroup stores its per-lane candidate to cand[lane * nrb +
    // row block] instead of updating `best`; k_argmax_finish then reduces the
    // row blocks of each lane (contiguous) and merges once into `best`.
    unsigned long long* cand;
    int32_t nrb;
  };
  __device__ __forceinline__ static f32x4 init(const Out&, int, int, int) { return f32x4{0.f, 0.f, 0.f, 0.f}; }
  // Merge tile (rt, *) into this lane column's candidate (bv, bi); after the call
  // every lane l holds the candidate of batch lane l % 16. Whole-wave call.
  __device__ __forceinline__ static void merge_tile(const Out& o, int rt, const f32x4& y, int lane, float& bv, int32_t& bi) {
    float tv = f32_of(0xFF800000u);
    int32_t ti = -1;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int index = rt * 16 + (lane >> 4) * 4 + i;
      if (index < o.vocab && y[i] > tv) {  // ascending rows, strict '>' (ties keep the smaller index)
        tv = y[i];
        ti = index;
      }
    }
#pragma unroll
    for (int sh = 16; sh <= 32; sh <<= 1) {
      const float ov = __shfl_xor(tv, sh);
      const int32_t oi = __shfl_xor(ti, sh);
      arg_merge(tv, ti, ov, oi);
    }
    arg_merge(bv, bi, tv, ti);
  }
  __device__ __forceinline__ static void commit(const Out& o, const Geometry& g, int lt, int lane, float bv, int32_t bi, int rb) {
    const int j = lt * 16 + (lane & 15);
    if (lane >= 16 || j >= g.rows) return;
    if (o.cand) {
      o.cand[static_cast<int64_t>(j) * o.nrb + rb] =
          (static_cast<unsigned long long>(static_cast<uint32_t>(bi)) << 32) | u32_of(bv);
    } else if (bi >= 0) {
      best_update(&o.best[j], bv, bi);
    }
  }
  __device__ __forceinline__ static void apply(const Out& o, const Geometry& g, int, int rt, int lt, const f32x4* y, int lane) {
    float bv = f32_of(0xFF800000u);
    int32_t bi = -1;
    merge_tile(o, rt, y[0], lane, bv, bi);
    const int j = lt * 16 + (lane & 15);
    if (lane < 16 && j < g.rows && bi >= 0) best_update(&o.best[j], bv, bi);
  }
};

// Second pass of the greedy LM head: lane j reduces the candidates of all nrb
// row blocks (any order gives the same lexicographic max) and merges the winner
// into best[j] (the caller's initial entry takes part, as in the reference).
// Internal linkage: every translation unit that includes this header gets its own copy.
static __global__ __launch_bounds__(256) void k_argmax_finish(const unsigned long long* __restrict__ cand, int nrb, int rows,
                                                       StrideBestEntry* best) {
  const int j = blockIdx.x;
  float bv = f32_of(0xFF800000u);
  int32_t bi = -1;
  for (int rb = threadIdx.x; rb < nrb; rb += 256) {
    const unsigned long long c = cand[static_cast<int64_t>(j) * nrb + rb];
    arg_merge(bv, bi, f32_of(static_cast<uint32_t>(c)), static_cast<int32_t>(c >> 32));
  }
  __shared__ float sv[256];
  __shared__ int32_t si[256];
  sv[threadIdx.x] = bv;
  si[threadIdx.x] = bi;
  __syncthreads();
  for (int h = 128; h > 0; h >>= 1) {
    if (threadIdx.x < h) {
      float v = sv[threadIdx.x];
      int32_t i = si[threadIdx.x];
      arg_merge(v, i, sv[threadIdx.x + h], si[threadIdx.x + h]);
      sv[threadIdx.x] = v;
      si[threadIdx.x] = i;
    }
    __syncthreads();
  }
  if (threadIdx.x == 0 && si[0] >= 0) best_update(&best[j], sv[0], si[0]);
}

struct EpiQkv {  // RoPE + q store + bf16 KV append  (src/kernels_tc.cu:347-432)
  static constexpr int kMats = 1;
  static constexpr bool kReduce = false;
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
  __device__ __forceinline__ static f32x4 init(const Out&, int, int, int) { return f32x4{0.f, 0.f, 0.f, 0.f}; }
  __device__ __forceinline__ static uint16_t* kv_row(const Out& o, int which, int head, int slot, int pos) {
    const StrideKvRef& kv = o.kv;
    const int64_t block = kv.table[static_cast<int64_t>(slot) * kv.max_blocks + (pos >> o.page_shift)];
    const int token = pos & ((1 << o.page_shift) - 1);
    return static_cast<uint16_t*>(kv.arena) + block * kv.block_elems + o.layer * kv.layer_elems + which * kv.which_elems +
           head * kv.group_elems + static_cast<int64_t>(token) * kv.head_dim;
  }
  __device__ __forceinline__ static void apply(const Out& o, const Geometry& g, int kind, int rt, int lt, const f32x4* y, int lane) {
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
    // This lane holds dims d..d+3 (rows 4*(lane/16)+i of the tile) and, from
    // its partner, d+half..d+half+3: each half is written as one vector when
    // the destination is aligned for it.
    const int d = d0 + (lane >> 4) * 4;
    float lo[4], hi[4];
    if (kind == 2) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        lo[i] = y[0][i];
        hi[i] = partner[i];
      }
    } else {
      const float* cs = o.rope + (static_cast<int64_t>(pos) * half + d) * 2;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float co = cs[2 * i], si = cs[2 * i + 1];
        const float a = y[0][i], b = partner[i];
        lo[i] = a * co - b * si;
        hi[i] = b * co + a * si;
      }
    }
    if (kind == 0) {
      float* q = o.q_out + static_cast<int64_t>(j) * o.q_stride + static_cast<int64_t>(head) * D + d;
      if ((reinterpret_cast<uintptr_t>(q) & 15) == 0 && (half & 3) == 0) {
        *reinterpret_cast<f32x4*>(q) = f32x4{lo[0], lo[1], lo[2], lo[3]};
        *reinterpret_cast<f32x4*>(q + half) = f32x4{hi[0], hi[1], hi[2], hi[3]};
      } else {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          q[i] = lo[i];
          q[half + i] = hi[i];
        }
      }
    } else {
      uint16_t* dst = kv_row(o, kind == 2 ? 1 : 0, head, slot, pos) + d;
      const uint32_t b0 = bf16_rne(lo[0]), b1 = bf16_rne(lo[1]), b2 = bf16_rne(lo[2]), b3 = bf16_rne(lo[3]);
      const uint32_t c0 = bf16_rne(hi[0]), c1 = bf16_rne(hi[1]), c2 = bf16_rne(hi[2]), c3 = bf16_rne(hi[3]);
      if ((reinterpret_cast<uintptr_t>(dst) & 7) == 0 && (half & 3) == 0) {
        *reinterpret_cast<u32x2*>(dst) = u32x2{b0 | (b1 << 16), b2 | (b3 << 16)};
        *reinterpret_cast<u32x2*>(dst + half) = u32x2{c0 | (c1 << 16), c2 | (c3 << 16)};
      } else {
        dst[0] = static_cast<uint16_t>(b0);
        dst[1] = static_cast<uint16_t>(b1);
        dst[2] = static_cast<uint16_t>(b2);
        dst[3] = static_cast<uint16_t>(b3);
        dst[half] = static_cast<uint16_t>(c0);
        dst[half + 1] = static_cast<uint16_t>(c1);
        dst[half + 2] = static_cast<uint16_t>(c2);
        dst[half + 3] = static_cast<uint16_t>(c3);
      }
    }
  }
};

}  // namespace stride_tc
