// Batch-invariant BF16 linear-layer GEMMs for MI355X (gfx950), behind the C ABI
// of include/stride_tc.h. These replace the GEMM kernels of stride's tensor-core
// path (reference src/kernels_tc.cu:347-655): fused QKV + RoPE + KV append,
// GEMM + residual (output / down), paired gate/up + SiLU, LM head + argmax and
// LM head full logits.
//
// Arithmetic contract (identical for every kernel variant below, hence batch
// invariant): for a weight matrix with K columns, K is read in 32-column chunks
// (one v_mfma_f32_16x16x32_bf16 each). The chunks are divided into S contiguous
// splits, S = split_count(N, K) depending on the weight shape only. Each split s
// chains its chunks in ascending order into an fp32 accumulator that starts at
// zero, except split 0 of a residual GEMM, which starts from h. The result is
// y = ((c0 + c1) + c2) + ... + c(S-1), then the epilogue. The reference fixes the
// same kind of tree with kFewRowsWarps (src/kernels_tc.cu:29-32, 462-496).
//
// Kernel families evaluating that expression (tc_stream.hpp, tc_pipe.hpp):
//   k_stream  weight streaming. A workgroup owns WR*R row tiles and LT lane
//             tiles; its WS split waves run the splits side by side, stream
//             weight chunks straight from HBM into registers with 16-byte loads,
//             and combine the split partials through LDS in ascending order. With
//             XS, each workgroup runs one split and the last one to finish a tile
//             group folds the partials in order. Serves decode batches and, for
//             matrices with four splits, prefill up to about a thousand rows.
//   k_pipe    LDS pipeline. WM x WN waves own a block of tiles; every stage's
//             chunks are copied HBM->LDS by global_load_lds in fragment order
//             through an NS-deep ring; splits are walked in order and folded in
//             registers. Serves prefill, and with small blocks the LM head and
//             gate/up from two to eight lane tiles.
//   k_tile    the first LDS-staged kernel, kept as the fallback when a split
//             length is not a multiple of the pipeline's chunks per stage.
// All call the same chunk order, the same MFMA instruction and the same
// epilogue functions, so every output row has the same bits for any M and any
// configuration; run() picks the configuration from measured sweeps.
#include <mutex>

#include "tc_gemm_run.hpp"

namespace stride_tc {

thread_local std::string g_last_error;

int fail(int code, const std::string& msg) {
  g_last_error = msg;
  return code;
}

// Device scratch for the split partials of cross-workgroup split launches and
// the greedy LM head's candidates, with the split arrival counters: kScratchSets
// file-scope sets, so no entry point allocates. Each stream that launches such
// kernels is given a set of its own (the first free set, else the set its device
// used least recently), so launches on up to kScratchSets streams of one device
// may overlap; ordering is only needed beyond that. Counters are left at zero by
// every launch. Addresses come from hipGetSymbolAddress once per device.
__device__ __align__(256) unsigned long long g_scratch[kScratchSets][kScratchBytes / 8];
__device__ __align__(256) int32_t g_split_cnt[kScratchSets][kSplitUnits];

namespace {
struct DeviceScratch {
  unsigned long long* scratch = nullptr;
  int32_t* counters = nullptr;
  hipStream_t owner[kScratchSets] = {};
  bool used[kScratchSets] = {};
  uint64_t last_use[kScratchSets] = {};
  uint64_t tick = 0;
};
std::mutex g_scratch_mu;
DeviceScratch g_dev_scratch[64];
}  // namespace

ScratchSet scratch_for(hipStream_t st) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return {};
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  DeviceScratch& d = g_dev_scratch[dev];
  if (!d.scratch) {
    void* p = nullptr;
    void* c = nullptr;
    if (hipGetSymbolAddress(&p, HIP_SYMBOL(g_scratch)) != hipSuccess) return {};
    if (hipGetSymbolAddress(&c, HIP_SYMBOL(g_split_cnt)) != hipSuccess) return {};
    d.scratch = static_cast<unsigned long long*>(p);
    d.counters = static_cast<int32_t*>(c);
  }
  int pick = -1;
  for (int i = 0; i < kScratchSets && pick < 0; ++i)
    if (d.used[i] && d.owner[i] == st) pick = i;
  for (int i = 0; i < kScratchSets && pick < 0; ++i)
    if (!d.used[i]) pick = i;
  if (pick < 0) {
    pick = 0;
    for (int i = 1; i < kScratchSets; ++i)
      if (d.last_use[i] < d.last_use[pick]) pick = i;
#ifdef STRIDE_TC_DEBUG
    // A fifth stream takes over the least recently used set. In debug builds that
    // is refused while the set's previous stream still has work queued (which
    // would race on the partials and counters). The previous stream must still
    // exist, which release builds cannot assume, hence no such check there.
    if (hipStreamQuery(d.owner[pick]) == hipErrorNotReady) {
      fail(STRIDE_TC_EINVAL, "scratch set of another stream is still in use (more than four streams in flight)");
      return {};
    }
#endif
  }
  d.used[pick] = true;
  d.owner[pick] = st;
  d.last_use[pick] = ++d.tick;
  return {d.scratch + static_cast<int64_t>(pick) * (kScratchBytes / 8), d.counters + static_cast<int64_t>(pick) * kSplitUnits};
}

int g_forced_cfg = -1;
int g_forced_dec = -1;
int g_forced_pipe = -1;
int g_last_cfg = -1;

// fp32 activations rows [rows][cols] -> two bf16 lane-tile sets, hi = bf16(x) and
// lo = bf16(x - hi), both round to nearest even; lanes past `rows` are zero.
// Thread i converts 8 consecutive columns of one lane.
__global__ __launch_bounds__(256) void k_split_f32x(const float* x, int rows, int cols, int lane_groups, uint16_t* hi,
                                                    uint16_t* lo) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  const int per_lane = cols / 8;
  if (i >= static_cast<int64_t>(lane_groups) * 16 * per_lane) return;
  const int lane = static_cast<int>(i / per_lane), c8 = static_cast<int>(i % per_lane) * 8;
  uint32_t h[4] = {0u, 0u, 0u, 0u}, l[4] = {0u, 0u, 0u, 0u};
  if (lane < rows) {
    const f32x4* src = reinterpret_cast<const f32x4*>(x + static_cast<int64_t>(lane) * cols + c8);
    const f32x4 a = src[0], b = src[1];
    const float v[8] = {a[0], a[1], a[2], a[3], b[0], b[1], b[2], b[3]};
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      const uint32_t hb = bf16_rne(v[k]);
      const uint32_t lb = bf16_rne(v[k] - f32_of(hb << 16));
      h[k / 2] |= hb << (16 * (k & 1));
      l[k / 2] |= lb << (16 * (k & 1));
    }
  }
  // lane tile layout [lt][ct][16 lanes][16 cols]
  const int64_t at = (static_cast<int64_t>(lane >> 4) * (cols / 16) + c8 / 16) * kTileElems + (lane & 15) * 16 + (c8 & 15);
  *reinterpret_cast<u32x4*>(hi + at) = u32x4{h[0], h[1], h[2], h[3]};
  *reinterpret_cast<u32x4*>(lo + at) = u32x4{l[0], l[1], l[2], l[3]};
}

// Zero-fill of fp32 output (a kernel, so a captured graph holds no memset node).
__global__ __launch_bounds__(256) void k_zero_f32(float* y, int64_t n) {
  const int64_t i = (static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x) * 4;
  if (i + 3 < n) *reinterpret_cast<f32x4*>(y + i) = f32x4{0.f, 0.f, 0.f, 0.f};
  else for (int64_t k = i; k < n; ++k) y[k] = 0.f;
}

// Staging of stride_tc_gemm_f32x_noalloc: the hi and lo bf16 lane tiles live in
// this file-scope array instead of a caller workspace. Every GPU the library runs
// on holds its own copy (16 MiB) until the process ends.
constexpr int64_t kF32xScratchElems = int64_t{8} << 20;  // bf16 elements: hi + lo
__device__ __align__(256) uint16_t scratch[kF32xScratchElems];

// Device address of `scratch` on the current device, resolved once per device
// with hipGetSymbolAddress (the array's name is only a host-side stand-in).
uint16_t* f32x_scratch(std::string& why) {
  static std::once_flag once[64];
  static uint16_t* addr[64] = {};
  static hipError_t err[64] = {};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) {
    why = "no current HIP device";
    return nullptr;
  }
  std::call_once(once[dev], [dev] {
    void* p = nullptr;
    err[dev] = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    addr[dev] = err[dev] == hipSuccess ? static_cast<uint16_t*>(p) : nullptr;
  });
  if (!addr[dev]) why = std::string("hipGetSymbolAddress(scratch) failed: ") + hipGetErrorString(err[dev]);
  return addr[dev];
}

// The launches of stride_tc_gemm_f32x with hi/lo staged at `hi` (2 * lane
// elements, caller-owned or the file-scope scratch).
int gemm_f32x_launch(const StrideTcGemmF32xParams& p, uint16_t* hi, hipStream_t st) {
  const int64_t lane_elems = static_cast<int64_t>(p.l.lane_groups) * 16 * p.m.cols;
  uint16_t* lo = hi + lane_elems;
  const int64_t pieces = static_cast<int64_t>(p.l.lane_groups) * 16 * (p.m.cols / 8);
  hipLaunchKernelGGL(k_split_f32x, dim3(static_cast<unsigned>((pieces + 255) / 256)), dim3(256), 0, st, p.x, p.l.rows,
                     p.m.cols, p.l.lane_groups, hi, lo);
  const int64_t y_elems = static_cast<int64_t>(p.l.lane_groups) * p.m.groups * kTileElems;
  hipLaunchKernelGGL(k_zero_f32, dim3(static_cast<unsigned>((y_elems / 4 + 255) / 256)), dim3(256), 0, st, p.y, y_elems);
  if (hipError_t e = hipGetLastError(); e != hipSuccess)
    return fail(static_cast<int>(e), std::string("gemm_f32x: launch failed: ") + hipGetErrorString(e));
  EpiResidual::Out o{p.y, p.m.groups};
  if (int rc = run<EpiResidual>(single(p.l, hi, p.m, nullptr), o, st)) return rc;
  return run<EpiResidual>(single(p.l, lo, p.m, nullptr), o, st);
}

}  // namespace stride_tc

using namespace stride_tc;

// Layout guards: these structs cross the ABI by address and must match the
// reference's PODs (src/kernels.h, src/kernels_tc.h) byte for byte.
static_assert(sizeof(StrideGemmMat) == 16, "GemmMat layout");
static_assert(sizeof(StrideKvRef) == 56, "KvRef layout");
static_assert(sizeof(StrideLanes) == 16, "Lanes layout");
static_assert(sizeof(StrideBestEntry) == 8 && alignof(StrideBestEntry) == 8, "BestEntry layout");
static_assert(offsetof(StrideTcQkvParams, kv) == 88 && sizeof(StrideTcQkvParams) == 176, "TcQkvParams layout");
static_assert(sizeof(StrideTcGemmResidualParams) == 48, "TcGemmResidualParams layout");
static_assert(sizeof(StrideTcMlp13Params) == 64, "TcMlp13Params layout");
static_assert(sizeof(StrideTcLmGreedyParams) == 56, "TcLmGreedyParams layout");
static_assert(sizeof(StrideTcLmFullParams) == 48, "TcLmFullParams layout");

extern "C" {

int stride_tc_set_stream_config(int32_t index) {
  if (index <= -3 && -3 - index < kNumPipeCfgs) {
    g_forced_pipe = -3 - index;
    g_forced_cfg = g_forced_dec = -1;
    return 0;
  }
  if (index >= kDecIndexBase && index - kDecIndexBase < kNumDecCfgs) {
    g_forced_dec = index - kDecIndexBase;
    g_forced_cfg = g_forced_pipe = -1;
    return 0;
  }
  if (index < -1 || index >= kNumDecodeCfgs) return fail(STRIDE_TC_EINVAL, "config index out of range");
  g_forced_cfg = index;
  g_forced_pipe = g_forced_dec = -1;
  return 0;
}

int stride_tc_dec_config_count(void) { return kNumDecCfgs; }

int stride_tc_stream_config_count(void) { return kNumDecodeCfgs; }

int stride_tc_pipe_config_count(void) { return kNumPipeCfgs; }

int stride_tc_last_stream_config(void) { return g_last_cfg; }

int stride_tc_stream_config(int32_t index, int32_t* out6) {
  if (index < 0 || index >= kNumDecodeCfgs || !out6) return fail(STRIDE_TC_EINVAL, "decode config index out of range");
  const DecodeCfg& c = kDecodeCfgs[index];
  out6[0] = c.r;
  out6[1] = c.lt;
  out6[2] = c.ws;
  out6[3] = c.wr;
  out6[4] = c.u;
  out6[5] = (c.xl ? 1 : 0) | (c.xs ? 2 : 0);
  return 0;
}

int stride_tc_split_count(int32_t n, int32_t k) {
  if (n <= 0 || k <= 0 || k % 16 != 0) return fail(-1, "split_count: need n > 0 and k a positive multiple of 16"), -1;
  return split_count(n, k);
}

const char* stride_tc_last_error(void) { return g_last_error.c_str(); }

const char* stride_tc_version(void) { return "stride_tc 0.1 gfx950 mfma_f32_16x16x32_bf16"; }

int stride_tc_gemm_residual(const StrideTcGemmResidualParams* p, int, int, void* stream) {
  std::string why;
  if (!p) return fail(STRIDE_TC_EINVAL, "gemm_residual: null params");
  if (!lanes_ok(p->l, why) || !mat_ok(p->m, "gemm_residual.m", why)) return fail(STRIDE_TC_EINVAL, "gemm_residual: " + why);
  if (!p->x || !p->h) return fail(STRIDE_TC_EINVAL, "gemm_residual: null x or h");
  Geometry g = single(p->l, p->x, p->m, nullptr);
  EpiResidual::Out o{p->h, p->m.groups};
  return run<EpiResidual>(g, o, static_cast<hipStream_t>(stream));
}

int stride_tc_gemm_f32x(const StrideTcGemmF32xParams* p, void* stream) {
  std::string why;
  if (!p) return fail(STRIDE_TC_EINVAL, "gemm_f32x: null params");
  if (!lanes_ok(p->l, why) || !mat_ok(p->m, "gemm_f32x.m", why)) return fail(STRIDE_TC_EINVAL, "gemm_f32x: " + why);
  if (!p->x || !p->y || !p->workspace) return fail(STRIDE_TC_EINVAL, "gemm_f32x: null x, y or workspace");
  if (p->l.rows == 0) return 0;
  return gemm_f32x_launch(*p, p->workspace, static_cast<hipStream_t>(stream));
}

int stride_tc_gemm_f32x_noalloc(const StrideTcGemmF32xParams* p, void* stream) {
  std::string why;
  if (!p) return fail(STRIDE_TC_EINVAL, "gemm_f32x_noalloc: null params");
  if (!lanes_ok(p->l, why) || !mat_ok(p->m, "gemm_f32x_noalloc.m", why))
    return fail(STRIDE_TC_EINVAL, "gemm_f32x_noalloc: " + why);
  if (!p->x || !p->y) return fail(STRIDE_TC_EINVAL, "gemm_f32x_noalloc: null x or y");
  if (p->workspace) return fail(STRIDE_TC_EINVAL, "gemm_f32x_noalloc: workspace must be null (the library's scratch is used)");
  const int64_t need = 2 * static_cast<int64_t>(p->l.lane_groups) * 16 * p->m.cols;
  if (need > kF32xScratchElems)
    return fail(STRIDE_TC_EINVAL, "gemm_f32x_noalloc: 2 * 16 * lane_groups * cols = " + std::to_string(need) +
                                      " bf16 elements exceeds the scratch of " + std::to_string(kF32xScratchElems));
  if (p->l.rows == 0) return 0;
  uint16_t* hi = f32x_scratch(why);
  if (!hi) return fail(STRIDE_TC_EINVAL, "gemm_f32x_noalloc: " + why);
  return gemm_f32x_launch(*p, hi, static_cast<hipStream_t>(stream));
}

int stride_tc_f32x_scratch_elems(void) { return static_cast<int>(kF32xScratchElems); }

}  // extern "C"
