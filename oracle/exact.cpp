// TEST INFRASTRUCTURE ONLY. This is the CPU oracle for the stride tensor-core GEMM
// path: a restatement of stride's CPU "exact path" (src/kernels.cu), written from
// scratch on plain row-major operands. Only tests/, __graft_entry__.smoke() and
// bench.py's cpu_baseline leg may load it, and only as the checker. The product
// (stride_amd/) never links or calls it.
//
// Arithmetic contract restated here (reference file:line):
//   * dot product of weight row n and activation row m is split over 32 partial
//     chains; chain t owns the 8-column lines l == t (mod 32) and runs
//     acc = fmaf(w[c], x[c], acc) over those columns in ascending order
//     (src/kernels.cu:63-94, 22-58);
//   * the 32 partials are combined left to right, ((P0 + P1) + P2) + ... + P31
//     (src/kernels.cu:311-318, 350-355, 403-404, 445-446, 239-242);
//   * residual: h = h + y (src/kernels.cu:321-322);
//   * gate/up: z = det_silu(a) * b (src/kernels.cu:359-360, src/numerics.h:16-33);
//   * LM greedy: per lane, scan rows ascending with strict '>' then the
//     order-independent lexicographic max of (value, -index)
//     (src/kernels.cu:407-423, src/kernel_common.h:58-82);
//   * QKV RoPE: ra = a*c - b*s, rb = b*c + a*s on pairs (d, d + D/2)
//     (src/kernels.cu:254-267).
// And the tensor-core path's non-GEMM operators, whose trees differ from the
// exact path's in places (see the comments at oracle_tc_norm and
// oracle_tc_attention).
// Rows are independent, so any split of the work over threads gives the same bits
// (the fork-join pool of src/cpu_pool.h:24-49 only changes who computes a row).
//
// Parity pins: bit-exact against the reference kernels.cu compiled as C++
// (oracle/_ref, built by oracle/Makefile) and against the golden fixtures under
// tests/golden/, plus closed-form checks in tests/test_oracle.py.
//
// Build flags matter: -ffp-contract=off -fno-fast-math so that only the explicit
// fmaf calls fuse (the reference's CMakeLists.txt:24-27 uses the same discipline).
#include <atomic>
#include <cmath>
#include <cstdint>
#include <cstring>
#include <thread>
#include <vector>

namespace {

inline float f32_of_bits(uint32_t u) {
  float f;
  std::memcpy(&f, &u, 4);
  return f;
}
inline uint32_t bits_of_f32(float f) {
  uint32_t u;
  std::memcpy(&u, &f, 4);
  return u;
}
inline float widen_bf16(uint16_t b) { return f32_of_bits(static_cast<uint32_t>(b) << 16); }

// Deterministic exp: reduce by k = floor(x*log2(e) + 1/2) with ln2 split in two
// parts (Cody-Waite), then a degree-6 polynomial in Horner/FMA form and an
// exponent-field scale. The constants are the Cephes expf coefficients and the
// two-part ln 2 split; they fix the bits, so they must be these exact floats
// (src/numerics.h:16-30).
float det_exp(float x) {
  if (x < -87.0f) return 0.0f;
  if (x > 88.0f) return f32_of_bits(0x7F800000u);
  const float kf = std::floor(std::fma(x, 1.44269504088896341f, 0.5f));
  float r = std::fma(-kf, 0.693359375f, x);
  r = std::fma(-kf, -2.12194440e-4f, r);
  static const float c[6] = {1.9875691500e-4f, 1.3981999507e-3f, 8.3334519073e-3f,
                             4.1665795894e-2f, 1.6666665459e-1f, 5.0000001201e-1f};
  float p = c[0];
  for (int i = 1; i < 6; ++i) p = std::fma(p, r, c[i]);
  const float y = std::fma(std::fma(p, r, 1.0f), r, 1.0f);
  const uint32_t scale = static_cast<uint32_t>(static_cast<int32_t>(kf)) << 23;
  return f32_of_bits(bits_of_f32(y) + scale);
}

float det_silu(float x) { return x / (1.0f + det_exp(-x)); }

// Round-to-nearest-even FP32 -> BF16 on the bit pattern (no NaN special case),
// src/kernel_common.h:29-32.
uint16_t bf16_rne(float f) {
  const uint32_t u = bits_of_f32(f);
  return static_cast<uint16_t>((u + 0x7FFFu + ((u >> 16) & 1u)) >> 16);
}

// The exact-path dot product of one bf16 weight row and one fp32 activation row.
float exact_dot(const uint16_t* w, const float* x, int k) {
  float part[32];
  for (int t = 0; t < 32; ++t) part[t] = 0.0f;
  const int lines = k / 8;
  for (int line = 0; line < lines; ++line) {
    float& acc = part[line & 31];
    const int c0 = line * 8;
    for (int c = 0; c < 8; ++c) acc = std::fma(widen_bf16(w[c0 + c]), x[c0 + c], acc);
  }
  float y = part[0];
  for (int t = 1; t < 32; ++t) y = y + part[t];
  return y;
}

template <class F>
void parallel_rows(int n, int threads, F&& body) {
  if (threads <= 1 || n <= 1) {
    for (int i = 0; i < n; ++i) body(i);
    return;
  }
  std::atomic<int> next{0};
  std::vector<std::thread> pool;
  for (int i = 0; i < threads; ++i) {
    pool.emplace_back([&] {
      for (;;) {
        const int r = next.fetch_add(1);
        if (r >= n) return;
        body(r);
      }
    });
  }
  for (auto& th : pool) th.join();
}

int resolve_threads(int threads) {
  if (threads > 0) return threads;
  const unsigned hc = std::thread::hardware_concurrency();
  return hc ? static_cast<int>(hc) : 1;
}

}  // namespace

extern "C" {

float oracle_det_exp(float x) { return det_exp(x); }
float oracle_det_silu(float x) { return det_silu(x); }
uint16_t oracle_bf16_rne(float f) { return bf16_rne(f); }

// y[m][n] = W[n] . x[m]; W row-major [n][k] bf16, x row-major [m][k] fp32.
// Work is split over weight rows. Returns 0, or -1 on a bad shape.
int oracle_gemm(const uint16_t* w, int n, int k, const float* x, int m, float* y, int threads) {
  if (n < 0 || m < 0 || k <= 0 || k % 8 != 0) return -1;
  parallel_rows(n, resolve_threads(threads), [&](int r) {
    const uint16_t* wr = w + static_cast<int64_t>(r) * k;
    for (int j = 0; j < m; ++j) y[static_cast<int64_t>(j) * n + r] = exact_dot(wr, x + static_cast<int64_t>(j) * k, k);
  });
  return 0;
}

// h[m][n] = h[m][n] + W[n] . x[m]  (output / down projection, src/kernels.cu:294-325).
int oracle_gemm_residual(const uint16_t* w, int n, int k, const float* x, int m, float* h, int threads) {
  if (n < 0 || m < 0 || k <= 0 || k % 8 != 0) return -1;
  parallel_rows(n, resolve_threads(threads), [&](int r) {
    const uint16_t* wr = w + static_cast<int64_t>(r) * k;
    for (int j = 0; j < m; ++j) {
      float* hp = h + static_cast<int64_t>(j) * n + r;
      *hp = *hp + exact_dot(wr, x + static_cast<int64_t>(j) * k, k);
    }
  });
  return 0;
}

// z[m][n] = det_silu(W1[n] . x[m]) * (W3[n] . x[m])  (src/kernels.cu:329-363).
// Optionally also returns the two pre-activations a (gate) and b (up).
int oracle_mlp13(const uint16_t* w1, const uint16_t* w3, int n, int k, const float* x, int m, float* z, float* a_out,
                 float* b_out, int threads) {
  if (n < 0 || m < 0 || k <= 0 || k % 8 != 0) return -1;
  parallel_rows(n, resolve_threads(threads), [&](int r) {
    const uint16_t* w1r = w1 + static_cast<int64_t>(r) * k;
    const uint16_t* w3r = w3 + static_cast<int64_t>(r) * k;
    for (int j = 0; j < m; ++j) {
      const float* xj = x + static_cast<int64_t>(j) * k;
      const float a = exact_dot(w1r, xj, k);
      const float b = exact_dot(w3r, xj, k);
      const int64_t at = static_cast<int64_t>(j) * n + r;
      z[at] = det_silu(a) * b;
      if (a_out) a_out[at] = a;
      if (b_out) b_out[at] = b;
    }
  });
  return 0;
}

// Greedy LM head: for each activation row m, the index of the largest logit over
// rows [0, vocab), ties to the smaller index (src/kernels.cu:383-425,
// src/kernel_common.h:58-82). W has n >= vocab rows.
int oracle_lm_greedy(const uint16_t* w, int n, int vocab, int k, const float* x, int m, float* best_value,
                     int32_t* best_index, int threads) {
  if (vocab > n || m < 0 || k <= 0 || k % 8 != 0) return -1;
  std::vector<float> logits(static_cast<size_t>(m) * vocab);
  parallel_rows(vocab, resolve_threads(threads), [&](int r) {
    const uint16_t* wr = w + static_cast<int64_t>(r) * k;
    for (int j = 0; j < m; ++j) logits[static_cast<size_t>(j) * vocab + r] = exact_dot(wr, x + static_cast<int64_t>(j) * k, k);
  });
  for (int j = 0; j < m; ++j) {
    float best = f32_of_bits(0xFF800000u);
    int32_t bi = -1;
    const float* row = &logits[static_cast<size_t>(j) * vocab];
    for (int r = 0; r < vocab; ++r) {
      if (row[r] > best) {
        best = row[r];
        bi = r;
      }
    }
    best_value[j] = best;
    best_index[j] = bi;
  }
  return 0;
}

// Fused QKV with RoPE (src/kernels.cu:204-284). Weights are row-major in the
// Hugging Face order (head-major, d in [0, D)); rope is [pos][D/2][cos, sin].
// Outputs are dense: q_out[m][nq], k_out[m][nkv], v_out[m][nkv].
int oracle_qkv(const uint16_t* wq, const uint16_t* wk, const uint16_t* wv, int nq, int nkv, int k, const float* x, int m,
               int head_dim, const float* rope, const int32_t* row_pos, float* q_out, float* k_out, float* v_out,
               int threads) {
  if (k <= 0 || k % 8 != 0 || head_dim <= 0 || head_dim % 2 != 0 || nq % head_dim != 0 || nkv % head_dim != 0) return -1;
  const int half = head_dim / 2;
  // One work item per (matrix, head, d < half): a RoPE pair.
  const int q_pairs = nq / 2, kv_pairs = nkv / 2;
  const int items = q_pairs + 2 * kv_pairs;
  parallel_rows(items, resolve_threads(threads), [&](int it) {
    int kind, pair;
    if (it < q_pairs) {
      kind = 0;
      pair = it;
    } else if (it < q_pairs + kv_pairs) {
      kind = 1;
      pair = it - q_pairs;
    } else {
      kind = 2;
      pair = it - q_pairs - kv_pairs;
    }
    const uint16_t* wm = kind == 0 ? wq : (kind == 1 ? wk : wv);
    const int n = kind == 0 ? nq : nkv;
    float* out = kind == 0 ? q_out : (kind == 1 ? k_out : v_out);
    const int head = pair / half;
    const int d = pair % half;
    const int ra_row = head * head_dim + d, rb_row = ra_row + half;
    for (int j = 0; j < m; ++j) {
      const float* xj = x + static_cast<int64_t>(j) * k;
      const float a = exact_dot(wm + static_cast<int64_t>(ra_row) * k, xj, k);
      const float b = exact_dot(wm + static_cast<int64_t>(rb_row) * k, xj, k);
      float oa = a, ob = b;
      if (kind != 2) {
        const float* cs = rope + (static_cast<int64_t>(row_pos[j]) * half + d) * 2;
        const float co = cs[0], si = cs[1];
        oa = a * co - b * si;
        ob = b * co + a * si;
      }
      out[static_cast<int64_t>(j) * n + ra_row] = oa;
      out[static_cast<int64_t>(j) * n + rb_row] = ob;
    }
  });
  return 0;
}

// RMSNorm of the tensor-core path (src/kernels_tc.cu:205-271; the per-lane
// variant :276-340 has the same bits): 32 partials, partial t = fmaf(v, v, acc)
// over the 16 columns of each column tile ct == t (mod 32), tiles ascending;
// sum = ((p0 + p1) + ...) + p31; r = 1 / sqrtf(sum / dim + eps);
// x = bf16(g * (v * r)). (The exact path's RmsNorm, src/kernels.cu:119-200,
// groups four columns per unit instead of sixteen, so its sum can differ in the
// last bit.) h and x are row-major [m][dim].
int oracle_tc_norm(const float* h, int m, int dim, const float* weight, float eps, uint16_t* x) {
  const int col_tiles = dim / 16;
  for (int j = 0; j < m; ++j) {
    const float* v = h + static_cast<int64_t>(j) * dim;
    float part[32];
    for (int t = 0; t < 32; ++t) {
      float acc = 0.0f;
      for (int ct = t; ct < col_tiles; ct += 32)
        for (int c = 0; c < 16; ++c) acc = std::fma(v[ct * 16 + c], v[ct * 16 + c], acc);
      part[t] = acc;
    }
    float sum = part[0];
    for (int t = 1; t < 32; ++t) sum = sum + part[t];
    const float r = 1.0f / std::sqrt(sum / static_cast<float>(dim) + eps);
    for (int c = 0; c < dim; ++c) x[static_cast<int64_t>(j) * dim + c] = bf16_rne(weight[c] * (v[c] * r));
  }
  return 0;
}

// Paged attention of the tensor-core path over bf16 KV (src/kernel_common.h:
// 84-309 with KvT = uint16_t, writer src/kernels_tc.cu:658-666), for groups of
// four query heads sharing KV group g. For row j, positions 0..row_pos[j] in
// 64-position pages: per page and head, score_i = (fmaf chain over d ascending
// of q[d] * k_i[d]) * scale; mp = max score; e_i = det_exp(score_i - mp);
// den = e_0 + e_1 + ... (left to right); v[d] = fmaf chain over i ascending of
// e_i * v_i[d]. Then over pages c ascending: M = max mp_c; f_c =
// det_exp(mp_c - M); D = fmaf chain of f_c * den_c; out[d] = (fmaf chain of
// f_c * v_c[d]) / D, rounded to bf16. Operands are plain: q [m][n_kv*4][hd] fp32,
// k and v [slot][g][pos][hd] bf16 bits with `cap` positions per slot,
// out [m][n_kv*4*hd] bf16 bits.
int oracle_tc_attention(const float* q, const uint16_t* k, const uint16_t* v, int cap, const int32_t* row_slot,
                        const int32_t* row_pos, int m, int n_kv, int hd, float scale, uint16_t* out) {
  const int heads = n_kv * 4;
  const float neg_inf = f32_of_bits(0xFF800000u);
  for (int j = 0; j < m; ++j) {
    const int pages = (row_pos[j] >> 6) + 1;
    const int visible = row_pos[j] + 1;
    for (int g = 0; g < n_kv; ++g) {
      const uint16_t* kg = k + (static_cast<int64_t>(row_slot[j]) * n_kv + g) * cap * hd;
      const uint16_t* vg = v + (static_cast<int64_t>(row_slot[j]) * n_kv + g) * cap * hd;
      std::vector<float> mp(static_cast<size_t>(pages) * 4), den(static_cast<size_t>(pages) * 4),
          vs(static_cast<size_t>(pages) * 4 * hd);
      for (int c = 0; c < pages; ++c) {
        const int p0 = c * 64;
        const int n = visible - p0 < 64 ? visible - p0 : 64;
        for (int h = 0; h < 4; ++h) {
          const float* qh = q + (static_cast<int64_t>(j) * heads + g * 4 + h) * hd;
          float sc[64];
          float mx = neg_inf;
          for (int i = 0; i < n; ++i) {
            float a = 0.0f;
            for (int d = 0; d < hd; ++d) a = std::fma(qh[d], widen_bf16(kg[static_cast<int64_t>(p0 + i) * hd + d]), a);
            sc[i] = a * scale;
            if (sc[i] > mx) mx = sc[i];
          }
          float e[64];
          for (int i = 0; i < n; ++i) e[i] = det_exp(sc[i] - mx);
          float dn = 0.0f;
          for (int i = 0; i < n; ++i) dn = dn + e[i];
          mp[c * 4 + h] = mx;
          den[c * 4 + h] = dn;
          for (int d = 0; d < hd; ++d) {
            float a = 0.0f;
            for (int i = 0; i < n; ++i) a = std::fma(e[i], widen_bf16(vg[static_cast<int64_t>(p0 + i) * hd + d]), a);
            vs[(static_cast<size_t>(c) * 4 + h) * hd + d] = a;
          }
        }
      }
      for (int h = 0; h < 4; ++h) {
        float M = neg_inf;
        for (int c = 0; c < pages; ++c)
          if (mp[c * 4 + h] > M) M = mp[c * 4 + h];
        std::vector<float> f(pages);
        float dn = 0.0f;
        for (int c = 0; c < pages; ++c) {
          f[c] = det_exp(mp[c * 4 + h] - M);
          dn = std::fma(f[c], den[c * 4 + h], dn);
        }
        for (int d = 0; d < hd; ++d) {
          float acc = 0.0f;
          for (int c = 0; c < pages; ++c) acc = std::fma(f[c], vs[(static_cast<size_t>(c) * 4 + h) * hd + d], acc);
          out[static_cast<int64_t>(j) * heads * hd + (g * 4 + h) * hd + d] = bf16_rne(acc / dn);
        }
      }
    }
  }
  return 0;
}

// RoPE table (src/model.cpp:54-88; model.cpp itself needs nlohmann/json, which
// this image lacks, so it is restated here): base = fp32(pow(theta, double(fp32(2i)
// / fp32(dim)))), f = 1 / base in fp32, llama3 band scaling on the wavelength
// 2*pi/f in fp32; entry (pos, i) = (fp32(cos(double(fp32(f_i * fp32(pos))))),
// fp32(sin(...))) with the C library's double cos/sin. table is
// [max_positions][dim/2][2].
int oracle_rope_table(int dim, double theta, int llama3, double factor, double low, double high, double orig_ctx,
                      int max_positions, float* table) {
  if (dim <= 0 || dim % 2 != 0 || max_positions <= 0) return 1;
  const int half = dim / 2;
  std::vector<float> inv(half);
  const float pi2 = static_cast<float>(2.0 * M_PI);
  for (int i = 0; i < half; ++i) {
    const float e = static_cast<float>(2 * i) / static_cast<float>(dim);
    float f = 1.0f / static_cast<float>(std::pow(theta, static_cast<double>(e)));
    if (llama3) {
      const float fac = static_cast<float>(factor);
      const float low_wave = static_cast<float>(orig_ctx / low);
      const float high_wave = static_cast<float>(orig_ctx / high);
      const float wave = pi2 / f;
      const float smooth = (static_cast<float>(orig_ctx) / wave - static_cast<float>(low)) / static_cast<float>(high - low);
      if (wave > low_wave)
        f = f / fac;
      else if (!(wave < high_wave))
        f = (1.0f - smooth) * (f / fac) + smooth * f;
    }
    inv[i] = f;
  }
  for (int pos = 0; pos < max_positions; ++pos)
    for (int i = 0; i < half; ++i) {
      const double a = static_cast<double>(inv[i] * static_cast<float>(pos));
      table[(static_cast<int64_t>(pos) * half + i) * 2] = static_cast<float>(std::cos(a));
      table[(static_cast<int64_t>(pos) * half + i) * 2 + 1] = static_cast<float>(std::sin(a));
    }
  return 0;
}

}  // extern "C"
