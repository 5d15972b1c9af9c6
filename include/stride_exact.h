/* C ABI of the exact path on MI355X (libstride_tc.so): the reference's fused
 * FP32 kernels (src/kernels.h:146-155, src/kernels.cu) as HIP kernels that give
 * the same bits as the reference's CPU exact path, so a CPU run and a GPU run of
 * the engine produce byte-identical ledgers.
 *
 * Layouts (src/kernels.h:3-10): activations dim-major fp32 A[dim * stride +
 * lane] (J = 1: one lane, stride 1; J = 4: lanes in groups of four, lane_groups
 * = ceil(rows / 4)); weights bf16 in four-row groups W[group][col][4]; KV fp32
 * [block][layer][K|V][group][token][dim] with the block size given by
 * group_elems / head_dim (the reference uses 64).
 *
 * Arithmetic (src/kernels.cu:1-12): a dot product is split over 32 chains, chain
 * t owning the 8-column lines l == t (mod 32) with fmaf in ascending column
 * order; the 32 partials are added left to right. Every entry point returns 0
 * or a nonzero code with stride_tc_last_error() set, and launches on `stream`
 * (a hipStream_t, or NULL). The shared structs (StrideLanes, StrideGemmMat,
 * StrideKvRef, StrideBestEntry, StrideAttentionParams) come from stride_tc.h. */
#ifndef STRIDE_EXACT_H
#define STRIDE_EXACT_H

#include <stdint.h>

#include "stride_tc.h"

#ifdef __cplusplus
extern "C" {
#endif

/* EmbedParams, src/kernels.h:48-54. h[k * stride + row] = widen(embed[token]). */
typedef struct {
  StrideLanes l;
  const uint16_t* embed;
  const int32_t* tokens;
  float* h;
  int32_t dim;
} StrideEmbedParams;

/* NormParams, src/kernels.h:56-63. */
typedef struct {
  StrideLanes l;
  const float* in;
  float* out;
  const float* weight;
  int32_t dim;
  float eps;
} StrideNormParams;

/* QkvParams, src/kernels.h:65-77: q/k/v weights use the four-row RoPE groups
 * (d, d+1, d+D/2, d+D/2+1), src/model.cpp:168-174. */
typedef struct {
  StrideLanes l;
  const float* x;
  StrideGemmMat q, k, v;
  float* q_out;
  int32_t q_stride;
  StrideKvRef kv;
  const float* rope;
  const int32_t* row_slot;
  const int32_t* row_pos;
  int32_t layer;
  int32_t head_dim;
} StrideQkvParams;

/* GemmResidualParams, src/kernels.h:100-105: h += W x. */
typedef struct {
  StrideLanes l;
  const float* x;
  StrideGemmMat m;
  float* h;
} StrideGemmResidualParams;

/* Mlp13Params, src/kernels.h:107-112: z = det_silu(W1 x) * (W3 x). */
typedef struct {
  StrideLanes l;
  const float* x;
  StrideGemmMat w1, w3;
  float* z;
} StrideMlp13Params;

/* CompactParams, src/kernels.h:114-122. */
typedef struct {
  StrideLanes l;
  const float* in;
  float* out;
  const int32_t* lm_rows;
  int32_t lm_count;
  int32_t lm_stride;
  int32_t dim;
} StrideCompactParams;

/* LmGreedyParams, src/kernels.h:130-136; best[] pre-initialised to {-inf, -1}. */
typedef struct {
  StrideLanes l;
  const float* x;
  StrideGemmMat m;
  int32_t vocab;
  StrideBestEntry* best;
} StrideLmGreedyParams;

/* LmFullParams, src/kernels.h:138-143: logits[row * stride + lane]. */
typedef struct {
  StrideLanes l;
  const float* x;
  StrideGemmMat m;
  float* logits;
} StrideLmFullParams;

/* The reference's k_* entry points (src/kernels.h:146-155); J is 1 or 4. */
int stride_k_embed(const StrideEmbedParams* p, void* stream);
int stride_k_norm(const StrideNormParams* p, int32_t J, void* stream);
int stride_k_qkv(const StrideQkvParams* p, int32_t J, void* stream);
/* Attention over fp32 KV, output dim-major fp32 out[(head * D + d) * stride + row]
 * (src/kernels.cu:474-485, LaneWriter :287-291); scratch and items as for
 * stride_tc_attention. */
int stride_k_attention(const StrideAttentionParams* p, void* stream);
int stride_k_gemm_residual(const StrideGemmResidualParams* p, int32_t J, void* stream);
int stride_k_mlp13(const StrideMlp13Params* p, int32_t J, void* stream);
int stride_k_compact(const StrideCompactParams* p, void* stream);
int stride_k_lm_greedy(const StrideLmGreedyParams* p, int32_t J, void* stream);
int stride_k_lm_full(const StrideLmFullParams* p, int32_t J, void* stream);

#ifdef __cplusplus
}
#endif

#endif
