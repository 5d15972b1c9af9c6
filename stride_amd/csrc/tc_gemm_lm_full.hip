// stride_tc_lm_full (C ABI of include/stride_tc.h): argument checks and the launch through
// run<EpiLogits> (tc_gemm_run.hpp). A translation unit of its own so that the library's
// kernel instantiations compile in parallel.
#include "tc_gemm_run.hpp"

using namespace stride_tc;

extern "C" {

int stride_tc_lm_full(const StrideTcLmFullParams* p, int, void* stream) {
  std::string why;
  if (!p) return fail(STRIDE_TC_EINVAL, "lm_full: null params");
  if (!lanes_ok(p->l, why) || !mat_ok(p->m, "lm_full.m", why)) return fail(STRIDE_TC_EINVAL, "lm_full: " + why);
  if (!p->x || !p->logits) return fail(STRIDE_TC_EINVAL, "lm_full: null x or logits");
  Geometry g = single(p->l, p->x, p->m, nullptr);
  EpiLogits::Out o{p->logits};
  return run<EpiLogits>(g, o, static_cast<hipStream_t>(stream));
}

}  // extern "C"
