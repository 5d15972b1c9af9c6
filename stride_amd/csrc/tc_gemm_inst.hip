// Explicit instantiation of one epilogue's configuration table of one kernel
// family (tc_gemm_run.hpp). The build compiles this file once per (epilogue,
// family) pair, with STRIDE_TC_EPI naming the epilogue and STRIDE_TC_FAMILY
// selecting the register-streaming (0), register-streamed weight / LDS-ring (1)
// or LDS-pipelined (2) table, so that the library's kernels compile in parallel.
#include "tc_gemm_run.hpp"

#ifndef STRIDE_TC_EPI
#error "STRIDE_TC_EPI must name an epilogue"
#endif

namespace stride_tc {

#if STRIDE_TC_FAMILY == 0
template void launch_decode_cfg<STRIDE_TC_EPI>(int, const Geometry&, const STRIDE_TC_EPI::Out&, hipStream_t);
#elif STRIDE_TC_FAMILY == 1
template void launch_dec_cfg<STRIDE_TC_EPI>(int, const Geometry&, const STRIDE_TC_EPI::Out&, hipStream_t);
#elif STRIDE_TC_FAMILY == 2
template void launch_pipe_cfg<STRIDE_TC_EPI>(int, const Geometry&, const STRIDE_TC_EPI::Out&, int, hipStream_t);
#else
#error "STRIDE_TC_FAMILY must be 0, 1 or 2"
#endif

}  // namespace stride_tc
