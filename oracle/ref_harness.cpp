// TEST INFRASTRUCTURE ONLY. A C-ABI harness around the reference's own CPU exact
// path. oracle/Makefile compiles this file together with the reference sources
// where they lie (/root/reference/src/kernels.cu and device.cu, built as C++) into
// oracle/_ref/libstride_ref.so. No reference source is copied into this repository.
//
// The harness converts plain row-major operands into the exact path's layouts:
//   weights  W[group][col][4 rows]           (pack, src/model.cpp:94-111)
//   RoPE rows (d0, d0+1, d0+D/2, d0+D/2+1)   (rope_rows, src/model.cpp:168-174)
//   activations dim-major A[dim*stride+lane] (src/kernels.h:3-8, lane_shape
//                                             src/engine.cpp:24-28)
// and calls k_lm_full / k_gemm_residual / k_mlp13 / k_lm_greedy / k_qkv, and
// k_embed / k_norm / k_attention for the non-GEMM operators (src/kernels.h:146-155). Signatures mirror oracle/exact.cpp so the two can be
// compared element for element.
#include <cstdint>
#include <cstring>
#include <vector>

#include "kernels.h"
#include "numerics.h"

using namespace stride;

namespace {

struct Shape {
  int J, lane_groups, stride;
};

Shape lane_shape(int rows) {
  if (rows == 1) return {1, 1, 1};
  const int g = (rows + 3) / 4;
  return {4, g, g * 4};
}

std::vector<uint16_t> pack4(const uint16_t* w, int n, int k, int groups, const std::vector<int>& row_of) {
  std::vector<uint16_t> out(static_cast<size_t>(groups) * k * 4, 0);
  for (int g = 0; g < groups; ++g)
    for (int s = 0; s < 4; ++s) {
      const int row = row_of[g * 4 + s];
      if (row < 0 || row >= n) continue;
      for (int c = 0; c < k; ++c) out[(static_cast<size_t>(g) * k + c) * 4 + s] = w[static_cast<size_t>(row) * k + c];
    }
  return out;
}

std::vector<int> plain_rows(int groups) {
  std::vector<int> r(groups * 4);
  for (int i = 0; i < groups * 4; ++i) r[i] = i;
  return r;
}

std::vector<int> rope_rows(int groups, int D) {
  std::vector<int> r(groups * 4);
  for (int g = 0; g < groups; ++g) {
    const int head = g / (D / 4);
    const int d0 = 2 * (g % (D / 4));
    const int off[4] = {d0, d0 + 1, d0 + D / 2, d0 + D / 2 + 1};
    for (int s = 0; s < 4; ++s) r[g * 4 + s] = head * D + off[s];
  }
  return r;
}

std::vector<float> dim_major(const float* x, int m, int k, const Shape& s) {
  std::vector<float> out(static_cast<size_t>(k) * s.stride + 16, 0.0f);
  for (int j = 0; j < m; ++j)
    for (int c = 0; c < k; ++c) out[static_cast<size_t>(c) * s.stride + j] = x[static_cast<size_t>(j) * k + c];
  return out;
}

Lanes lanes_of(int m, const Shape& s) { return Lanes{m, s.lane_groups, s.stride, 0}; }

}  // namespace

extern "C" {

float ref_det_exp(float x) { return det_exp(x); }
float ref_det_silu(float x) { return det_silu(x); }

int ref_gemm(const uint16_t* w, int n, int k, const float* x, int m, float* y) {
  const int groups = (n + 3) / 4;
  const Shape s = lane_shape(m);
  std::vector<uint16_t> wp = pack4(w, n, k, groups, plain_rows(groups));
  std::vector<float> xd = dim_major(x, m, k, s);
  std::vector<float> logits(static_cast<size_t>(groups) * 4 * s.stride, 0.0f);
  LmFullParams p{};
  p.l = lanes_of(m, s);
  p.x = xd.data();
  p.m = GemmMat{wp.data(), groups, k};
  p.logits = logits.data();
  k_lm_full(p, s.J);
  for (int j = 0; j < m; ++j)
    for (int r = 0; r < n; ++r) y[static_cast<size_t>(j) * n + r] = logits[static_cast<size_t>(r) * s.stride + j];
  return 0;
}

int ref_gemm_residual(const uint16_t* w, int n, int k, const float* x, int m, float* h) {
  const int groups = n / 4;
  const Shape s = lane_shape(m);
  std::vector<uint16_t> wp = pack4(w, n, k, groups, plain_rows(groups));
  std::vector<float> xd = dim_major(x, m, k, s);
  std::vector<float> hd = dim_major(h, m, n, s);
  GemmResidualParams p{};
  p.l = lanes_of(m, s);
  p.x = xd.data();
  p.m = GemmMat{wp.data(), groups, k};
  p.h = hd.data();
  k_gemm_residual(p, s.J);
  for (int j = 0; j < m; ++j)
    for (int r = 0; r < n; ++r) h[static_cast<size_t>(j) * n + r] = hd[static_cast<size_t>(r) * s.stride + j];
  return 0;
}

int ref_mlp13(const uint16_t* w1, const uint16_t* w3, int n, int k, const float* x, int m, float* z) {
  const int groups = n / 4;
  const Shape s = lane_shape(m);
  std::vector<uint16_t> p1 = pack4(w1, n, k, groups, plain_rows(groups));
  std::vector<uint16_t> p3 = pack4(w3, n, k, groups, plain_rows(groups));
  std::vector<float> xd = dim_major(x, m, k, s);
  std::vector<float> zd(static_cast<size_t>(n) * s.stride + 16, 0.0f);
  Mlp13Params p{};
  p.l = lanes_of(m, s);
  p.x = xd.data();
  p.w1 = GemmMat{p1.data(), groups, k};
  p.w3 = GemmMat{p3.data(), groups, k};
  p.z = zd.data();
  k_mlp13(p, s.J);
  for (int j = 0; j < m; ++j)
    for (int r = 0; r < n; ++r) z[static_cast<size_t>(j) * n + r] = zd[static_cast<size_t>(r) * s.stride + j];
  return 0;
}

int ref_lm_greedy(const uint16_t* w, int n, int vocab, int k, const float* x, int m, float* best_value, int32_t* best_index) {
  const int groups = (vocab + 3) / 4;
  const Shape s = lane_shape(m);
  std::vector<int> rows(groups * 4);
  for (int i = 0; i < groups * 4; ++i) rows[i] = i < vocab ? i : -1;
  std::vector<uint16_t> wp = pack4(w, n, k, groups, rows);
  std::vector<float> xd = dim_major(x, m, k, s);
  std::vector<BestEntry> best(m);
  for (auto& b : best) {
    const uint32_t ninf = 0xFF800000u;
    std::memcpy(&b.value, &ninf, 4);
    b.index = -1;
  }
  LmGreedyParams p{};
  p.l = lanes_of(m, s);
  p.x = xd.data();
  p.m = GemmMat{wp.data(), groups, k};
  p.vocab = vocab;
  p.best = best.data();
  k_lm_greedy(p, s.J);
  for (int j = 0; j < m; ++j) {
    best_value[j] = best[j].value;
    best_index[j] = best[j].index;
  }
  return 0;
}

// Each activation row j gets KV slot j; slot j's blocks are laid out contiguously.
int ref_qkv(const uint16_t* wq, const uint16_t* wk, const uint16_t* wv, int nq, int nkv, int k, const float* x, int m,
            int head_dim, const float* rope, const int32_t* row_pos, float* q_out, float* k_out, float* v_out) {
  const int D = head_dim;
  const Shape s = lane_shape(m);
  const int gq = nq / 4, gk = nkv / 4;
  std::vector<uint16_t> pq = pack4(wq, nq, k, gq, rope_rows(gq, D));
  std::vector<uint16_t> pk = pack4(wk, nkv, k, gk, rope_rows(gk, D));
  std::vector<uint16_t> pv = pack4(wv, nkv, k, gk, rope_rows(gk, D));
  std::vector<float> xd = dim_major(x, m, k, s);
  int max_pos = 0;
  for (int j = 0; j < m; ++j) max_pos = row_pos[j] > max_pos ? row_pos[j] : max_pos;
  const int max_blocks = (max_pos >> kKvBlockShift) + 1;
  const int kv_heads = nkv / D;
  KvRef kv{};
  kv.group_elems = static_cast<int64_t>(kKvBlockTokens) * D;
  kv.which_elems = kv.group_elems * kv_heads;
  kv.layer_elems = kv.which_elems * 2;
  kv.block_elems = kv.layer_elems;  // one layer
  kv.max_blocks = max_blocks;
  kv.head_dim = D;
  std::vector<int32_t> table(static_cast<size_t>(m) * max_blocks);
  for (size_t i = 0; i < table.size(); ++i) table[i] = static_cast<int32_t>(i);
  std::vector<float> arena(table.size() * kv.block_elems, 0.0f);
  kv.arena = arena.data();
  kv.table = table.data();
  std::vector<int32_t> slots(m);
  for (int j = 0; j < m; ++j) slots[j] = j;
  QkvParams p{};
  p.l = lanes_of(m, s);
  p.x = xd.data();
  p.q = GemmMat{pq.data(), gq, k};
  p.k = GemmMat{pk.data(), gk, k};
  p.v = GemmMat{pv.data(), gk, k};
  p.q_out = q_out;
  p.q_stride = nq;
  p.kv = kv;
  p.rope = rope;
  p.row_slot = slots.data();
  p.row_pos = row_pos;
  p.layer = 0;
  p.head_dim = D;
  k_qkv(p, s.J);
  for (int j = 0; j < m; ++j) {
    const int pos = row_pos[j];
    const int64_t blk = table[static_cast<size_t>(j) * max_blocks + (pos >> kKvBlockShift)];
    const int tok = pos & (kKvBlockTokens - 1);
    for (int hd = 0; hd < kv_heads; ++hd)
      for (int d = 0; d < D; ++d) {
        const int64_t base = blk * kv.block_elems + hd * kv.group_elems + tok * D + d;
        k_out[static_cast<size_t>(j) * nkv + hd * D + d] = arena[base];
        v_out[static_cast<size_t>(j) * nkv + hd * D + d] = arena[base + kv.which_elems];
      }
  }
  return 0;
}


// Exact-path embedding (src/kernels.cu:98-117) of plain bf16 rows emb[vocab][dim]
// (packed into the exact path's [vocab/4][dim][4] layout) into h[m][dim].
int ref_embed(const uint16_t* emb, int vocab, int dim, const int32_t* tokens, int m, float* h) {
  const int groups = (vocab + 3) / 4;
  const Shape s = lane_shape(m);
  std::vector<uint16_t> ep = pack4(emb, vocab, dim, groups, plain_rows(groups));
  std::vector<float> hd(static_cast<size_t>(dim) * s.stride + 16, 0.0f);
  EmbedParams p{};
  p.l = lanes_of(m, s);
  p.embed = ep.data();
  p.tokens = tokens;
  p.h = hd.data();
  p.dim = dim;
  k_embed(p);
  for (int j = 0; j < m; ++j)
    for (int c = 0; c < dim; ++c) h[static_cast<size_t>(j) * dim + c] = hd[static_cast<size_t>(c) * s.stride + j];
  return 0;
}

// Exact-path RMSNorm (src/kernels.cu:119-200), fp32 out[m][dim].
int ref_norm(const float* h, int m, int dim, const float* weight, float eps, float* out) {
  const Shape s = lane_shape(m);
  std::vector<float> hd = dim_major(h, m, dim, s);
  std::vector<float> od(hd.size(), 0.0f);
  NormParams p{};
  p.l = lanes_of(m, s);
  p.in = hd.data();
  p.out = od.data();
  p.weight = weight;
  p.dim = dim;
  p.eps = eps;
  k_norm(p, s.J);
  for (int j = 0; j < m; ++j)
    for (int c = 0; c < dim; ++c) out[static_cast<size_t>(j) * dim + c] = od[static_cast<size_t>(c) * s.stride + j];
  return 0;
}

// Exact-path attention (src/kernels.cu:474-485, src/kernel_common.h:84-309) over
// fp32 KV holding the widened bf16 values k, v [slot][g][pos][hd] (cap positions
// per slot), laid out in the reference's 64-token KV blocks; fp32 out[m][heads*hd].
int ref_attention(const float* q, const uint16_t* k, const uint16_t* v, int slots, int cap, const int32_t* row_slot,
                  const int32_t* row_pos, int m, int n_kv, int hd, float scale, float* out) {
  const Shape s = lane_shape(m);
  const int heads = n_kv * 4;
  const int max_blocks = (cap + kKvBlockTokens - 1) / kKvBlockTokens;
  const int64_t group_elems = static_cast<int64_t>(kKvBlockTokens) * hd;
  const int64_t which_elems = n_kv * group_elems;
  const int64_t block_elems = 2 * which_elems;
  std::vector<float> arena(static_cast<size_t>(slots) * max_blocks * block_elems, 0.0f);
  std::vector<int32_t> table(static_cast<size_t>(slots) * max_blocks);
  for (int sl = 0; sl < slots; ++sl)
    for (int b = 0; b < max_blocks; ++b) table[static_cast<size_t>(sl) * max_blocks + b] = sl * max_blocks + b;
  for (int sl = 0; sl < slots; ++sl)
    for (int g = 0; g < n_kv; ++g)
      for (int pos = 0; pos < cap; ++pos)
        for (int which = 0; which < 2; ++which) {
          const uint16_t* src = (which ? v : k) + ((static_cast<int64_t>(sl) * n_kv + g) * cap + pos) * hd;
          float* dst = arena.data() + (static_cast<int64_t>(sl) * max_blocks + pos / kKvBlockTokens) * block_elems +
                       which * which_elems + g * group_elems + static_cast<int64_t>(pos % kKvBlockTokens) * hd;
          for (int d = 0; d < hd; ++d) {
            const uint32_t bits = static_cast<uint32_t>(src[d]) << 16;
            std::memcpy(&dst[d], &bits, 4);
          }
        }
  std::vector<int32_t> items;
  for (int j = 0; j < m; ++j)
    for (int page = 0; page <= (row_pos[j] >> kKvBlockShift); ++page) {
      items.push_back(j);
      items.push_back(page);
    }
  const int rec_floats = 4 * hd + 8;
  std::vector<float> scratch(static_cast<size_t>(m) * n_kv * max_blocks * rec_floats, 0.0f);
  std::vector<float> od(static_cast<size_t>(heads) * hd * s.stride + 16, 0.0f);
  AttentionParams p{};
  p.l = lanes_of(m, s);
  p.q = q;
  p.q_stride = heads * hd;
  p.out = od.data();
  p.out_cols = heads * hd;
  p.kv = KvRef{arena.data(), table.data(), block_elems, block_elems, which_elems, group_elems, max_blocks, hd};
  p.row_slot = row_slot;
  p.row_pos = row_pos;
  p.items = items.data();
  p.item_count = static_cast<int32_t>(items.size() / 2);
  p.scratch = scratch.data();
  p.max_pages = max_blocks;
  p.rec_floats = rec_floats;
  p.layer = 0;
  p.n_kv = n_kv;
  p.n_q = 4;
  p.head_dim = hd;
  p.scale = scale;
  k_attention(p);
  for (int j = 0; j < m; ++j)
    for (int c = 0; c < heads * hd; ++c) out[static_cast<size_t>(j) * heads * hd + c] = od[static_cast<size_t>(c) * s.stride + j];
  return 0;
}

}  // extern "C"

// CPU baseline timing: packs once, then times `reps` calls of the reference's
// k_lm_full (the exact-path GEMM, src/kernels.cu:427-452) over the same operands.
// Returns wall seconds for all reps.
#include <chrono>
extern "C" double ref_bench_gemm(const uint16_t* w, int n, int k, const float* x, int m, int reps) {
  const int groups = (n + 3) / 4;
  const Shape s = lane_shape(m);
  std::vector<uint16_t> wp = pack4(w, n, k, groups, plain_rows(groups));
  std::vector<float> xd = dim_major(x, m, k, s);
  std::vector<float> logits(static_cast<size_t>(groups) * 4 * s.stride, 0.0f);
  LmFullParams p{};
  p.l = lanes_of(m, s);
  p.x = xd.data();
  p.m = GemmMat{wp.data(), groups, k};
  p.logits = logits.data();
  const auto t0 = std::chrono::steady_clock::now();
  for (int r = 0; r < reps; ++r) k_lm_full(p, s.J);
  const auto t1 = std::chrono::steady_clock::now();
  return std::chrono::duration<double>(t1 - t0).count();
}

// The reference's exact-path entry points themselves, taking its own parameter
// blocks (pointers into host memory: the CPU build's "device" is the host). An
// exact-path engine step driven through these on the CPU is the reference's
// Engine::step_exact (src/engine.cpp:144-297) operator for operator.
extern "C" {
void ref_k_embed(const EmbedParams* p) { k_embed(*p); }
void ref_k_norm(const NormParams* p, int J) { k_norm(*p, J); }
void ref_k_qkv(const QkvParams* p, int J) { k_qkv(*p, J); }
void ref_k_attention(const AttentionParams* p) { k_attention(*p); }
void ref_k_gemm_residual(const GemmResidualParams* p, int J) { k_gemm_residual(*p, J); }
void ref_k_mlp13(const Mlp13Params* p, int J) { k_mlp13(*p, J); }
void ref_k_compact(const CompactParams* p) { k_compact(*p); }
void ref_k_lm_greedy(const LmGreedyParams* p, int J) { k_lm_greedy(*p, J); }
void ref_k_lm_full(const LmFullParams* p, int J) { k_lm_full(*p, J); }
}  // extern "C"
