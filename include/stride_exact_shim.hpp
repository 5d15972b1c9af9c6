// C++ drop-in for the exact path's entry points (src/kernels.h:146-155), for an
// engine HIP build that links libstride_tc.so instead of compiling kernels.cu for
// the GPU. Include it from ONE translation unit of the engine, after the engine's
// own "kernels.h", next to stride_tc_shim.hpp:
//
//     #include "kernels.h"               // stride::EmbedParams, ... (unchanged)
//     #include "stride_exact_shim.hpp"   // defines stride::k_embed, ... over the C ABI
//
// The nine functions keep the reference signatures; the engine's PODs are passed
// by address after static_asserts on their layout. Launches go on
// stride::tc_stream() (defined by the engine, as for stride_tc_shim.hpp); a
// nonzero return becomes std::runtime_error, as the reference's check() throws
// (src/device.cu:16-21).
#pragma once

#include <cstddef>
#include <stdexcept>
#include <string>

#include "stride_exact.h"

namespace stride {

void* tc_stream();

namespace exact_shim {

template <class Ref, class Abi>
const Abi* as_abi(const Ref& p) {
  static_assert(sizeof(Ref) == sizeof(Abi), "engine parameter block differs from the C ABI layout");
  static_assert(alignof(Ref) <= alignof(Abi), "engine parameter block alignment differs from the C ABI");
  return reinterpret_cast<const Abi*>(&p);
}

inline void check(int rc, const char* what) {
  if (rc != 0) throw std::runtime_error(std::string(what) + ": " + stride_tc_last_error());
}

static_assert(offsetof(QkvParams, kv) == offsetof(StrideQkvParams, kv), "QkvParams.kv offset");
static_assert(offsetof(QkvParams, rope) == offsetof(StrideQkvParams, rope), "QkvParams.rope offset");
static_assert(offsetof(NormParams, eps) == offsetof(StrideNormParams, eps), "NormParams.eps offset");
static_assert(offsetof(LmGreedyParams, best) == offsetof(StrideLmGreedyParams, best), "LmGreedyParams.best offset");
static_assert(offsetof(CompactParams, dim) == offsetof(StrideCompactParams, dim), "CompactParams.dim offset");

}  // namespace exact_shim

void k_embed(const EmbedParams& p) {
  exact_shim::check(stride_k_embed(exact_shim::as_abi<EmbedParams, StrideEmbedParams>(p), tc_stream()), "k_embed");
}

void k_norm(const NormParams& p, int J) {
  exact_shim::check(stride_k_norm(exact_shim::as_abi<NormParams, StrideNormParams>(p), J, tc_stream()), "k_norm");
}

void k_qkv(const QkvParams& p, int J) {
  exact_shim::check(stride_k_qkv(exact_shim::as_abi<QkvParams, StrideQkvParams>(p), J, tc_stream()), "k_qkv");
}

void k_attention(const AttentionParams& p) {
  exact_shim::check(stride_k_attention(exact_shim::as_abi<AttentionParams, StrideAttentionParams>(p), tc_stream()),
                    "k_attention");
}

void k_gemm_residual(const GemmResidualParams& p, int J) {
  exact_shim::check(
      stride_k_gemm_residual(exact_shim::as_abi<GemmResidualParams, StrideGemmResidualParams>(p), J, tc_stream()),
      "k_gemm_residual");
}

void k_mlp13(const Mlp13Params& p, int J) {
  exact_shim::check(stride_k_mlp13(exact_shim::as_abi<Mlp13Params, StrideMlp13Params>(p), J, tc_stream()), "k_mlp13");
}

void k_compact(const CompactParams& p) {
  exact_shim::check(stride_k_compact(exact_shim::as_abi<CompactParams, StrideCompactParams>(p), tc_stream()),
                    "k_compact");
}

void k_lm_greedy(const LmGreedyParams& p, int J) {
  exact_shim::check(stride_k_lm_greedy(exact_shim::as_abi<LmGreedyParams, StrideLmGreedyParams>(p), J, tc_stream()),
                    "k_lm_greedy");
}

void k_lm_full(const LmFullParams& p, int J) {
  exact_shim::check(stride_k_lm_full(exact_shim::as_abi<LmFullParams, StrideLmFullParams>(p), J, tc_stream()),
                    "k_lm_full");
}

}  // namespace stride
