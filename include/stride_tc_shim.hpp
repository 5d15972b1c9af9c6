// C++ drop-in for the GEMM entry points of stride's tensor-core path, for an
// engine build that links libstride_tc.so instead of compiling kernels_tc.cu.
// Include it from ONE translation unit of the engine, after the engine's own
// "kernels_tc.h" (reference src/kernels_tc.h), e.g. a file tc_gemm_hip.cpp:
//
//     #include "kernels_tc.h"          // stride::TcQkvParams, ... (unchanged)
//     #include "stride_tc_shim.hpp"    // defines stride::tc_qkv, ... over the C ABI
//
// It defines the nine functions with the reference signatures
// (src/kernels_tc.h:79-87). The parameter structs are passed by address: the
// static_asserts below check that the engine's PODs have exactly the layout the
// C ABI expects. Launches go on stride::tc_stream(), which the engine defines
// (the counterpart of the reference's kernel_stream(), src/kernels.cu:457-460).
// A nonzero return becomes std::runtime_error, as the reference's device check()
// throws (src/device.cu:16-21).
#pragma once

#include <cstddef>
#include <stdexcept>
#include <string>

#include "stride_tc.h"

namespace stride {

// Provided by the engine's HIP backend: the one stream all kernels go on.
void* tc_stream();

namespace tc_shim {

template <class Ref, class Abi>
const Abi* as_abi(const Ref& p) {
  static_assert(sizeof(Ref) == sizeof(Abi), "engine parameter block differs from the C ABI layout");
  static_assert(alignof(Ref) <= alignof(Abi), "engine parameter block alignment differs from the C ABI");
  return reinterpret_cast<const Abi*>(&p);
}

inline void check(int rc, const char* what) {
  if (rc != 0) throw std::runtime_error(std::string(what) + ": " + stride_tc_last_error());
}

static_assert(sizeof(BestEntry) == sizeof(StrideBestEntry) && alignof(BestEntry) == alignof(StrideBestEntry),
              "BestEntry layout");
static_assert(offsetof(TcQkvParams, kv) == offsetof(StrideTcQkvParams, kv), "TcQkvParams.kv offset");
static_assert(offsetof(TcQkvParams, head_dim) == offsetof(StrideTcQkvParams, head_dim), "TcQkvParams.head_dim offset");
static_assert(offsetof(TcLmGreedyParams, best) == offsetof(StrideTcLmGreedyParams, best), "TcLmGreedyParams.best offset");
static_assert(offsetof(TcNormParams, eps) == offsetof(StrideTcNormParams, eps), "TcNormParams.eps offset");
static_assert(offsetof(TcCompactParams, col_tiles) == offsetof(StrideTcCompactParams, col_tiles), "TcCompactParams offset");
static_assert(offsetof(AttentionParams, kv) == offsetof(StrideAttentionParams, kv), "AttentionParams.kv offset");
static_assert(offsetof(AttentionParams, scale) == offsetof(StrideAttentionParams, scale), "AttentionParams.scale offset");

}  // namespace tc_shim

void tc_qkv(const TcQkvParams& p) {
  tc_shim::check(stride_tc_qkv(tc_shim::as_abi<TcQkvParams, StrideTcQkvParams>(p), tc_stream()), "tc_qkv");
}

void tc_gemm_residual(const TcGemmResidualParams& p, int r, int lt) {
  tc_shim::check(stride_tc_gemm_residual(tc_shim::as_abi<TcGemmResidualParams, StrideTcGemmResidualParams>(p), r, lt,
                                         tc_stream()),
                 "tc_gemm_residual");
}

void tc_mlp13(const TcMlp13Params& p, int r, int lt) {
  tc_shim::check(stride_tc_mlp13(tc_shim::as_abi<TcMlp13Params, StrideTcMlp13Params>(p), r, lt, tc_stream()), "tc_mlp13");
}

void tc_lm_greedy(const TcLmGreedyParams& p, int r, int lt) {
  tc_shim::check(stride_tc_lm_greedy(tc_shim::as_abi<TcLmGreedyParams, StrideTcLmGreedyParams>(p), r, lt, tc_stream()),
                 "tc_lm_greedy");
}

void tc_lm_full(const TcLmFullParams& p, int lt) {
  tc_shim::check(stride_tc_lm_full(tc_shim::as_abi<TcLmFullParams, StrideTcLmFullParams>(p), lt, tc_stream()), "tc_lm_full");
}

void tc_embed(const TcEmbedParams& p) {
  tc_shim::check(stride_tc_embed(tc_shim::as_abi<TcEmbedParams, StrideTcEmbedParams>(p), tc_stream()), "tc_embed");
}

void tc_norm(const TcNormParams& p, bool per_lane) {
  tc_shim::check(stride_tc_norm(tc_shim::as_abi<TcNormParams, StrideTcNormParams>(p), per_lane ? 1 : 0, tc_stream()),
                 "tc_norm");
}

void tc_attention(const AttentionParams& p) {
  tc_shim::check(stride_tc_attention(tc_shim::as_abi<AttentionParams, StrideAttentionParams>(p), tc_stream()),
                 "tc_attention");
}

void tc_compact(const TcCompactParams& p) {
  tc_shim::check(stride_tc_compact(tc_shim::as_abi<TcCompactParams, StrideTcCompactParams>(p), tc_stream()), "tc_compact");
}

}  // namespace stride
