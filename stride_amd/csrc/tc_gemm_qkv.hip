// stride_tc_qkv (C ABI of include/stride_tc.h): argument checks and the launch through
// run<EpiQkv> (tc_gemm_run.hpp). A translation unit of its own so that the library's
// kernel instantiations compile in parallel.
#include "tc_gemm_run.hpp"

using namespace stride_tc;

extern "C" {

int stride_tc_qkv(const StrideTcQkvParams* p, void* stream) {
  std::string why;
  if (!p) return fail(STRIDE_TC_EINVAL, "qkv: null params");
  if (!lanes_ok(p->l, why) || !mat_ok(p->q, "qkv.q", why) || !mat_ok(p->k, "qkv.k", why) || !mat_ok(p->v, "qkv.v", why))
    return fail(STRIDE_TC_EINVAL, "qkv: " + why);
  if (p->q.cols != p->k.cols || p->q.cols != p->v.cols || p->k.groups != p->v.groups)
    return fail(STRIDE_TC_EINVAL, "qkv: q, k, v must share cols and k, v must have equal groups");
  const int D = p->head_dim;
  if (D <= 0 || D % 16 != 0 || (p->q.groups * 16) % D != 0 || (p->k.groups * 16) % D != 0)
    return fail(STRIDE_TC_EINVAL, "qkv: head_dim must be a multiple of 16 dividing the q and k rows");
  if (!p->x || !p->q_out || !p->rope || !p->row_slot || !p->row_pos || !p->kv.arena || !p->kv.table)
    return fail(STRIDE_TC_EINVAL, "qkv: null pointer argument");
  if (p->kv.head_dim != D || p->kv.group_elems <= 0 || p->kv.group_elems % D != 0)
    return fail(STRIDE_TC_EINVAL, "qkv: kv.head_dim must equal head_dim and kv.group_elems must be tokens*head_dim");
  const int64_t page = p->kv.group_elems / D;
  int shift = 0;
  while ((int64_t{1} << shift) < page) ++shift;
  if ((int64_t{1} << shift) != page) return fail(STRIDE_TC_EINVAL, "qkv: KV page size (group_elems/head_dim) must be a power of two");
  Geometry g{};
  g.x = p->x;
  g.col_tiles = p->q.cols / 16;
  g.rows = p->l.rows;
  g.lane_groups = p->l.lane_groups;
  g.nseg = 3;
  const StrideGemmMat* mats[3] = {&p->q, &p->k, &p->v};
  for (int i = 0; i < 3; ++i) {
    g.seg[i].w[0] = mats[i]->w;
    g.seg[i].w[1] = nullptr;
    g.seg[i].row_tiles = mats[i]->groups;
    g.seg[i].splits = split_count(mats[i]->groups * 16, mats[i]->cols);
  }
  EpiQkv::Out o{};
  o.q_out = p->q_out;
  o.q_stride = p->q_stride;
  o.layer = p->layer;
  o.head_dim = D;
  o.page_shift = shift;
  o.kv = p->kv;
  o.rope = p->rope;
  o.row_slot = p->row_slot;
  o.row_pos = p->row_pos;
  return run<EpiQkv>(g, o, static_cast<hipStream_t>(stream));
}

}  // extern "C"
