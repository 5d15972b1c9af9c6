// stride_tc_lm_greedy (C ABI of include/stride_tc.h): argument checks and the launch through
// run<EpiArgmax> (tc_gemm_run.hpp). A translation unit of its own so that the library's
// kernel instantiations compile in parallel.
#include "tc_gemm_run.hpp"

using namespace stride_tc;

extern "C" {

int stride_tc_lm_greedy(const StrideTcLmGreedyParams* p, int, int, void* stream) {
  std::string why;
  if (!p) return fail(STRIDE_TC_EINVAL, "lm_greedy: null params");
  if (!lanes_ok(p->l, why) || !mat_ok(p->m, "lm_greedy.m", why)) return fail(STRIDE_TC_EINVAL, "lm_greedy: " + why);
  if (!p->x || !p->best) return fail(STRIDE_TC_EINVAL, "lm_greedy: null x or best");
  if (p->vocab <= 0 || p->vocab > p->m.groups * 16) return fail(STRIDE_TC_EINVAL, "lm_greedy: vocab must be in (0, groups*16]");
  Geometry g = single(p->l, p->x, p->m, nullptr);
  EpiArgmax::Out o{p->best, p->vocab, nullptr, 0};
  return run<EpiArgmax>(g, o, static_cast<hipStream_t>(stream));
}

}  // extern "C"
