/* C ABI of the MI355X (gfx950) batch-invariant BF16 linear-layer GEMM library
 * (libstride_tc.so). It replaces the GEMM entry points of stride's tensor-core
 * path, declared in the reference at src/kernels_tc.h:81-87 and defined at
 * src/kernels_tc.cu:677-710.
 *
 * Structs are byte-compatible with the reference's POD parameter blocks
 * (src/kernels.h:23-46, 79-98, 125-128 and src/kernels_tc.h:10-77): same field order,
 * int32 fields, 8-byte pointers, BestEntry 8-byte aligned. A caller that already
 * fills stride::TcGemmResidualParams can pass its address here unchanged.
 *
 * Layouts (the reference's tile conventions, src/kernels_tc.cu:8-11):
 *   weights  W[row tile][col tile][16 rows][16 cols]  bf16 (pack_tiles, src/model.cpp:114-133)
 *   x / z    X[lane tile][col tile][16 lanes][16 cols] bf16
 *   h        fp32, same tile grid as x: h[lane tile][row tile][16 lanes][16 rows]
 *   logits   fp32 [row tile][lane tile][16 rows][16 lanes]
 * Shapes: cols (K) must be a multiple of 16 (the reference's 16-column tiles,
 * src/model.cpp:114-120); lane_groups must equal ceil(rows/16);
 * lanes past `rows` inside the last lane tile must hold zeros (the engine
 * zero-fills its tile buffers, src/engine.cpp:72-80).
 *
 * Batch invariance: every output element is computed by the same sequence of
 * operations whatever `rows`, the lane position, the stream or the (r, lt)
 * blocking hint: K is consumed in 32-column chunks in ascending order by one
 * v_mfma_f32_16x16x32_bf16 chain per split, the split count S depends only on
 * the weight shape (stride_tc_split_count), and the S partial sums combine left
 * to right, split 0 starting from the residual where there is one. When K is
 * 16 (mod 32) the last split's chain ends with one more MFMA over the trailing
 * 16 columns, whose upper 16 k are zero; such launches always run the
 * register-streaming kernel (correct for any M, not tuned for prefill).
 *
 * Errors: every entry point returns 0 on success or a nonzero code (a hipError_t
 * value, or STRIDE_TC_EINVAL for rejected arguments); stride_tc_last_error()
 * describes the last failure on the calling thread. Launches are asynchronous on
 * `stream` (NULL = the default stream); nothing here synchronizes or allocates.
 *
 * Shared device state: GEMM launches that combine splits across workgroups, and
 * the greedy LM head, use a 16 MiB device-global scratch array and a set of
 * arrival counters. There are four such sets per device, each bound to the
 * stream that last used it (a new stream takes a free set, else the least
 * recently used one), so launches on up to four streams of one device may
 * overlap; with more streams in flight at once, order them (the reference
 * keeps every launch on one stream, src/kernels.cu:457-460). A launch captured
 * in a HIP graph keeps the set of its capture stream for every replay, and a
 * fifth stream used at any time later (not only at once) may be given that same
 * set: order eager launches on such a stream with the graph's replays. Built
 * with -DSTRIDE_TC_DEBUG, a launch that would take over a set whose stream still
 * has work queued fails with STRIDE_TC_EINVAL instead. The configuration hooks
 * below are process-wide and meant for tuning sweeps, not for concurrent
 * callers.
 */
#ifndef STRIDE_TC_H
#define STRIDE_TC_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define STRIDE_TC_EINVAL 0x5354 /* argument rejected before any launch */

/* src/kernels.h:23-27 */
typedef struct StrideGemmMat {
  const uint16_t* w;
  int32_t groups; /* row tiles (N / 16) */
  int32_t cols;   /* K */
} StrideGemmMat;

/* src/kernels.h:30-39. The page size in tokens is group_elems / head_dim
 * (64 in the reference's KvCache; any power of two here). */
typedef struct StrideKvRef {
  void* arena;
  const int32_t* table;
  int64_t block_elems;
  int64_t layer_elems;
  int64_t which_elems;
  int64_t group_elems;
  int32_t max_blocks;
  int32_t head_dim;
} StrideKvRef;

/* src/kernels.h:41-46 (stride and bug are ignored by this library) */
typedef struct StrideLanes {
  int32_t rows;
  int32_t lane_groups;
  int32_t stride;
  int32_t bug;
} StrideLanes;

/* src/kernels.h:125-128 */
typedef struct StrideBestEntry {
  float value;
  int32_t index;
} __attribute__((aligned(8))) StrideBestEntry;

/* src/kernels_tc.h:27-39 */
typedef struct StrideTcQkvParams {
  StrideLanes l;
  const uint16_t* x;
  StrideGemmMat q, k, v;
  float* q_out;
  int32_t q_stride;
  StrideKvRef kv;
  const float* rope;
  const int32_t* row_slot;
  const int32_t* row_pos;
  int32_t layer;
  int32_t head_dim;
} StrideTcQkvParams;

/* src/kernels_tc.h:41-46 */
typedef struct StrideTcGemmResidualParams {
  StrideLanes l;
  const uint16_t* x;
  StrideGemmMat m;
  float* h;
} StrideTcGemmResidualParams;

/* src/kernels_tc.h:48-53 */
typedef struct StrideTcMlp13Params {
  StrideLanes l;
  const uint16_t* x;
  StrideGemmMat w1, w3;
  uint16_t* z;
} StrideTcMlp13Params;

/* src/kernels_tc.h:64-70 */
typedef struct StrideTcLmGreedyParams {
  StrideLanes l;
  const uint16_t* x;
  StrideGemmMat m;
  int32_t vocab;
  StrideBestEntry* best;
} StrideTcLmGreedyParams;

/* src/kernels_tc.h:72-77 */
typedef struct StrideTcLmFullParams {
  StrideLanes l;
  const uint16_t* x;
  StrideGemmMat m;
  float* logits;
} StrideTcLmFullParams;

/* No reference counterpart: parameters of stride_tc_gemm_f32x. */
typedef struct StrideTcGemmF32xParams {
  StrideLanes l;
  const float* x;      /* fp32 activations, row-major [rows][cols] */
  StrideGemmMat m;
  float* y;            /* fp32 output tiles [lt][rt][16 lanes][16 rows] (the h layout), overwritten */
  uint16_t* workspace; /* caller-owned, 2 * lane_groups * 16 * cols bf16 elements */
} StrideTcGemmF32xParams;

/* src/kernels_tc.h:10-16 */
typedef struct StrideTcEmbedParams {
  StrideLanes l;
  const uint16_t* embed; /* tied embedding as weight tiles [rt][ct][16][16] bf16 */
  const int32_t* tokens; /* [rows] */
  float* h;              /* fp32 tiles [lt][ct][16 lanes][16 cols] */
  int32_t dim;
} StrideTcEmbedParams;

/* src/kernels_tc.h:18-25 */
typedef struct StrideTcNormParams {
  StrideLanes l;
  const float* h;       /* fp32 tiles [lt][ct][16 lanes][16 cols] */
  uint16_t* x;          /* bf16 tiles, same grid */
  const float* weight;  /* [dim] gains */
  int32_t dim;
  float eps;
} StrideTcNormParams;

/* src/kernels_tc.h:55-62 */
typedef struct StrideTcCompactParams {
  StrideLanes l;
  const uint16_t* in;     /* bf16 tiles [lt][ct][16][16] */
  uint16_t* out;          /* bf16 tiles, lane l = in lane lm_rows[l] */
  const int32_t* lm_rows;
  int32_t lm_count;
  int32_t col_tiles;
} StrideTcCompactParams;

/* src/kernels.h:79-98 */
typedef struct StrideAttentionParams {
  StrideLanes l;
  const float* q; /* [row][head][dim] fp32 (tc_qkv's q_out) */
  int32_t q_stride;
  void* out;      /* bf16 x tiles [lt][ct][16][16], out_cols columns */
  int32_t out_cols;
  StrideKvRef kv;
  const int32_t* row_slot;
  const int32_t* row_pos;
  const int32_t* items; /* (row, page) pairs to compute this call */
  int32_t item_count;
  float* scratch;       /* caller-owned page records */
  int32_t max_pages;
  int32_t rec_floats;   /* >= 8 + 4 * head_dim */
  int32_t layer;
  int32_t n_kv;
  int32_t n_q;
  int32_t head_dim;
  float scale;
} StrideAttentionParams;

/* Replaces stride::tc_qkv (src/kernels_tc.h:81, src/kernels_tc.cu:677-679):
 * q = Wq x, k = Wk x, v = Wv x with RoPE on q and k (row tiles hold RoPE pairs
 * (d0+i, d0+D/2+i), src/model.cpp:178-183); q -> fp32 q_out[row*q_stride +
 * head*D + d]; k, v -> bf16 (round to nearest even) into the paged KV arena. */
int stride_tc_qkv(const StrideTcQkvParams* p, void* stream);

/* Replaces stride::tc_gemm_residual (src/kernels_tc.h:83, src/kernels_tc.cu:692-695):
 * h <- h + W x (output and MLP-down projections). row_tiles_per_warp and
 * lane_tiles_per_warp are the reference's register-blocking hints; they are
 * accepted for interface compatibility and never change results. */
int stride_tc_gemm_residual(const StrideTcGemmResidualParams* p, int row_tiles_per_warp, int lane_tiles_per_warp,
                            void* stream);

/* Replaces stride::tc_mlp13 (src/kernels_tc.h:84, src/kernels_tc.cu:696-700):
 * z = bf16(det_silu(W1 x) * (W3 x)) written as x-layout tiles. */
int stride_tc_mlp13(const StrideTcMlp13Params* p, int row_tiles_per_warp, int lane_tiles_per_warp, void* stream);

/* Replaces stride::tc_lm_greedy (src/kernels_tc.h:86, src/kernels_tc.cu:702-706):
 * per lane, best[lane] <- lexicographic max of (logit, -index) over rows < vocab,
 * merged into the caller-initialised entries (value -inf, index -1). */
int stride_tc_lm_greedy(const StrideTcLmGreedyParams* p, int row_tiles_per_warp, int lane_tiles_per_warp,
                        void* stream);

/* Replaces stride::tc_lm_full (src/kernels_tc.h:87, src/kernels_tc.cu:707-710):
 * logits tiles [row tile][lane tile][16 rows][16 lanes], fp32. */
int stride_tc_lm_full(const StrideTcLmFullParams* p, int lane_tiles_per_block, void* stream);

/* No reference counterpart (the reference's tensor-core path consumes bf16 x
 * only): y = W x for fp32 activations, for callers that keep them in fp32 (a
 * projection compared against the CPU exact path, which reads fp32 x). x is split
 * into hi = bf16(x) and lo = bf16(x - hi); then y = (0 + W hi) + W lo, each term
 * computed like stride_tc_gemm_residual, so every row is batch invariant. The
 * part of x below lo is under 2^-16 of |x|. */
int stride_tc_gemm_f32x(const StrideTcGemmF32xParams* p, void* stream);

/* No reference counterpart: stride_tc_gemm_f32x for callers that cannot
 * allocate device memory (code under HIP graph capture, serving loops that
 * forbid hipMalloc). Same result bits as stride_tc_gemm_f32x; p->workspace must
 * be NULL: hi and lo are staged in a 16 MiB file-scope device array (each GPU
 * the library runs on holds one until the process ends), so
 * 2 * 16 * lane_groups * cols must not exceed stride_tc_f32x_scratch_elems()
 * (for example M <= 256 at K = 8192 or M <= 2048 at K = 2048); larger calls are
 * rejected with STRIDE_TC_EINVAL. Calls that overlap on one GPU (other streams,
 * other threads) share that array and race; order them on one stream. Nothing
 * here calls hipMalloc or hipFree. */
int stride_tc_gemm_f32x_noalloc(const StrideTcGemmF32xParams* p, void* stream);

/* Capacity of the scratch stride_tc_gemm_f32x_noalloc stages into, in bf16 elements. */
int stride_tc_f32x_scratch_elems(void);

/* Replaces stride::tc_embed (src/kernels_tc.h:79, src/kernels_tc.cu:179-203):
 * h tile row of lane j <- the fp32 widening of embedding row tokens[j]. */
int stride_tc_embed(const StrideTcEmbedParams* p, void* stream);

/* Replaces stride::tc_norm (src/kernels_tc.h:80, src/kernels_tc.cu:205-340):
 * x = bf16(weight * (h * r)), r = 1 / sqrtf(sum / dim + eps), where sum is the
 * reference's fixed tree: 32 partials (partial t = fmaf over the 16 columns of
 * column tiles ct == t mod 32, ascending), added left to right. per_lane = 0
 * also writes zeros to the padding lanes of the last lane tile. */
int stride_tc_norm(const StrideTcNormParams* p, int per_lane, void* stream);

/* Replaces stride::tc_attention (src/kernels_tc.h:82, src/kernels_tc.cu:668-679,
 * src/kernel_common.h:84-309): paged attention over bf16 KV for groups of four
 * query heads sharing one KV head. Each (row, 64-position page) item is summed
 * on its own into a record (max, denominator, weighted values) in `scratch`;
 * then each row's pages are combined in ascending order and the output is
 * written as bf16 x tiles. The KV storage page (group_elems / head_dim tokens,
 * a power of two) is independent of the 64-position summation page. head_dim
 * must be 32, 64 or 128; n_q must be 4.
 * The library picks the form. With the item list the reference's engine
 * always builds (src/engine.cpp:93-103: rows ascending, each row's pages 0 ..
 * last ascending), up to 512 rows and when the row's records fit the LDS (below),
 * pages and combine run as one kernel that checks each row's stretch of the list
 * on the device; such rows keep their records in LDS and leave `scratch` as it
 * was. Any other list gets the page + combine semantics exactly: listed pages
 * are summed and stored in `scratch`, the rest are combined from what `scratch`
 * holds. Extension (no reference counterpart): item_count == -1 means every page
 * of every row with no list and no scratch. The one-kernel form needs
 * max_pages * (12 + 4 * head_dim) floats plus the row's KV page numbers (4 bytes
 * each) and its staging within 159 KiB of LDS: with 16-token KV pages up to 115
 * pages (7360 positions) at head_dim 64, 44 at head_dim 128; item_count == -1
 * beyond that is rejected, item lists beyond it run the page + combine pair.
 * Every row must satisfy row_pos < 64 * max_pages. */
int stride_tc_attention(const StrideAttentionParams* p, void* stream);

/* Replaces stride::tc_compact (src/kernels_tc.h:85, src/kernels_tc.cu:566-587):
 * out lane l <- in lane lm_rows[l], for l < lm_count. */
int stride_tc_compact(const StrideTcCompactParams* p, void* stream);

/* No reference counterpart (a property the reference fixes in code,
 * src/kernels_tc.cu:29-32): the number of K splits used for a weight matrix
 * of n rows and k columns. Depends on (n, k) only. */
int stride_tc_split_count(int32_t n, int32_t k);

/* Tuning hook, no reference counterpart: force the register-streaming kernel
 * configuration `index` (0 .. stride_tc_stream_config_count()-1) for launches of
 * at most 8 lane tiles, or the LDS-pipelined configuration -3-i for every launch
 * it can serve, or the register-streamed weight / LDS-ring activation
 * configuration 1000+i, or -1 for the automatic choice. Every configuration computes
 * identical bits; this only changes speed. A configuration that cannot serve a
 * launch is ignored for it. */
int stride_tc_set_stream_config(int32_t index);
int stride_tc_stream_config_count(void);
/* Number of LDS-pipelined configurations (selected as -3-i above). */
int stride_tc_pipe_config_count(void);
/* Number of register-streamed weight / LDS-ring activation configurations
 * (selected as 1000+i above). */
int stride_tc_dec_config_count(void);
/* Configuration used by the last launch in this process, in the numbering of
 * stride_tc_set_stream_config (-2: the fallback tile kernel, -1: none yet). */
int stride_tc_last_stream_config(void);
/* Writes (R, LT, WS, WR, U, flags) of configuration `index` into out6; flags bit 0:
 * activations staged in LDS, bit 1: one K split per workgroup (the last workgroup
 * of each tile group to finish combines the partials). */
int stride_tc_stream_config(int32_t index, int32_t* out6);

/* Message for the last nonzero return on this thread ("" if none). */
const char* stride_tc_last_error(void);

/* Library version string. */
const char* stride_tc_version(void);

#ifdef __cplusplus
}
#endif

#endif /* STRIDE_TC_H */
