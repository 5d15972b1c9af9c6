// stride_tc_mlp13 (C ABI of include/stride_tc.h): argument checks and the launch through
// run<EpiGateUp> (tc_gemm_run.hpp). A translation unit of its own so that the library's
// kernel instantiations compile in parallel.
#include "tc_gemm_run.hpp"

using namespace stride_tc;

extern "C" {

int stride_tc_mlp13(const StrideTcMlp13Params* p, int, int, void* stream) {
  std::string why;
  if (!p) return fail(STRIDE_TC_EINVAL, "mlp13: null params");
  if (!lanes_ok(p->l, why) || !mat_ok(p->w1, "mlp13.w1", why) || !mat_ok(p->w3, "mlp13.w3", why))
    return fail(STRIDE_TC_EINVAL, "mlp13: " + why);
  if (p->w1.groups != p->w3.groups || p->w1.cols != p->w3.cols) return fail(STRIDE_TC_EINVAL, "mlp13: w1 and w3 shapes differ");
  if (!p->x || !p->z) return fail(STRIDE_TC_EINVAL, "mlp13: null x or z");
  Geometry g = single(p->l, p->x, p->w1, p->w3.w);
  EpiGateUp::Out o{p->z, p->w1.groups};
  return run<EpiGateUp>(g, o, static_cast<hipStream_t>(stream));
}

}  // extern "C"
