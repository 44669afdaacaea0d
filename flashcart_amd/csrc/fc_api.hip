// C ABI of the tensor product and library metadata.
#include "fc_tp_impl.h"

namespace fc {

int segment_sum(int64_t n_seg, int64_t width, const float* src, const int32_t* perm, const int32_t* ptr, float* dst,
                hipStream_t s);
int colsum(int64_t rows, int64_t cols, const float* src, float* dst, hipStream_t s);

// Runtime mirror of PathList (same order, used for validation and sizes).
static int count_paths(int l1m, int l2m, int lom, bool sym, int* per_lo) {
  const int lp = l1m > l2m ? l1m : l2m;
  int n = 0;
  for (int lo = 0; lo <= lom; ++lo) {
    int q = 0;
    for (int l1 = 0; l1 <= lp; ++l1)
      for (int l2 = 0; l2 <= l1; ++l2)
        if (allowed(l1, l2, lo) && l1 <= l1m && l2 <= l2m) ++q;
    if (!sym)
      for (int l1 = 0; l1 <= lp; ++l1)
        for (int l2 = 0; l2 < l1; ++l2)
          if (allowed(l1, l2, lo) && l1 <= l2m && l2 <= l1m) ++q;
    if (per_lo) per_lo[lo] = q;
    n += q;
  }
  return n;
}

static int check_tp(const fc_tp_desc* d) {
  if (!d) return FC_ERR_NULL;
  if (d->in1_l_max < 0 || d->in2_l_max < 0 || d->out_l_max < 0) return FC_ERR_BAD_DESC;
  if (d->in1_l_max > FC_KERNEL_L_MAX || d->in2_l_max > FC_KERNEL_L_MAX || d->out_l_max > FC_KERNEL_L_MAX)
    return FC_ERR_UNSUPPORTED_L;
  const int f1 = d->in1_features, f2 = d->in2_features;
  if (f1 < 1 || f2 < 1 || !(f1 == f2 || f1 == 1 || f2 == 1)) return FC_ERR_BAD_DESC;
  if (d->symmetric_product && (d->in1_l_max != d->in2_l_max || f1 != f2)) return FC_ERR_BAD_DESC;
  return FC_OK;
}

static int64_t out_width(const fc_tp_desc* d) {
  int per[FC_MAX_RANKS] = {0};
  count_paths(d->in1_l_max, d->in2_l_max, d->out_l_max, d->symmetric_product != 0, per);
  const int64_t C = d->in1_features > d->in2_features ? d->in1_features : d->in2_features;
  int64_t w = 0;
  for (int lo = 0; lo <= d->out_l_max; ++lo)
    w += (int64_t)(2 * lo + 1) * (d->reduce_paths ? (per[lo] > 0 ? 1 : 0) : per[lo]) * C;
  return w;
}

static TPArgs make_args(const fc_tp_desc* d, int64_t n_rows) {
  TPArgs g{};
  g.n_rows = n_rows;
  g.F1 = d->in1_features;
  g.F2 = d->in2_features;
  g.C = g.F1 > g.F2 ? g.F1 : g.F2;
  g.shared_w = d->shared_weights;
  g.reduced = d->reduce_paths;
  g.alpha = 1.0f;
  g.alpha_div = d->alpha_div;
  return g;
}

static int dispatch(const fc_tp_desc* d, const TPArgs& g, bool conv, bool bwd, hipStream_t s) {
  const bool sym = d->symmetric_product != 0;
  switch (d->in1_l_max) {
    case 0: return dispatch_tp_l0(d->in2_l_max, d->out_l_max, sym, g, conv, bwd, s);
    case 1: return dispatch_tp_l1(d->in2_l_max, d->out_l_max, sym, g, conv, bwd, s);
    case 2: return dispatch_tp_l2(d->in2_l_max, d->out_l_max, sym, g, conv, bwd, s);
    case 3: return dispatch_tp_l3(d->in2_l_max, d->out_l_max, sym, g, conv, bwd, s);
#if FC_KERNEL_L_MAX >= 4
    case 4: return dispatch_tp_l4(d->in2_l_max, d->out_l_max, sym, g, conv, bwd, s);
#endif
  }
  return FC_ERR_UNSUPPORTED_L;
}

}  // namespace fc

using namespace fc;

extern "C" int fc_version(void) { return 100; }
extern "C" int fc_kernel_l_max(void) { return FC_KERNEL_L_MAX; }

extern "C" const char* fc_status_string(int st) {
  switch (st) {
    case FC_OK: return "ok";
    case FC_ERR_BAD_DESC: return "inconsistent descriptor";
    case FC_ERR_UNSUPPORTED_L: return "tensor rank above the compiled kernel limit (3)";
    case FC_ERR_LAUNCH: return "HIP kernel launch failed";
    case FC_ERR_SHAPE: return "unsupported sizes";
    case FC_ERR_NULL: return "required pointer is NULL";
    case FC_ERR_WORKSPACE: return "workspace missing or too small";
    case FC_ERR_SCRATCH_LIMIT: return "input exceeds the fixed scratch of an allocation-free entry point";
  }
  return "unknown status";
}

extern "C" int fc_tp_num_paths(const fc_tp_desc* d) {
  const int st = check_tp(d);
  if (st != FC_OK) return -st;
  return count_paths(d->in1_l_max, d->in2_l_max, d->out_l_max, d->symmetric_product != 0, nullptr);
}

extern "C" int64_t fc_tp_out_dim(const fc_tp_desc* d) {
  const int st = check_tp(d);
  if (st != FC_OK) return -st;
  return out_width(d);
}

extern "C" int fc_tp_fwd(const fc_tp_desc* d, const fc_csr* graph, int64_t n_rows, const float* in1,
                         const float* in2, const float* w, float alpha, float* out, void* stream) {
  int st = check_tp(d);
  if (st != FC_OK) return st;
  const bool conv = graph != nullptr;
  const int64_t rows = conv ? graph->n_nodes : n_rows;
  if (rows < 0) return FC_ERR_SHAPE;
  if (rows == 0) return FC_OK;
  if (!out) return FC_ERR_NULL;
  if (conv && (!graph->rowptr || !graph->idx_j)) return FC_ERR_NULL;
  const int64_t items = conv ? graph->n_edges : rows;
  if (items > 0 && (!in1 || !in2 || !w)) return FC_ERR_NULL;
  if (conv && graph->pair_slot && d->shared_weights) return FC_ERR_BAD_DESC;
  TPArgs g = make_args(d, rows);
  g.in1 = in1; g.in2 = in2; g.w = w; g.out = out; g.alpha = alpha;
  if (conv) { g.idx_j = graph->idx_j; g.rowptr = graph->rowptr; g.wslot = graph->pair_slot; g.n_edges = graph->n_edges; }
  return dispatch(d, g, conv, false, (hipStream_t)stream);
}

extern "C" int64_t fc_tp_bwd_workspace(const fc_tp_desc* d, const fc_csr* graph, int64_t n_rows, int need_in1,
                                       int need_w) {
  const int st = check_tp(d);
  if (st != FC_OK) return -st;
  const bool conv = graph != nullptr;
  const int64_t items = conv ? graph->n_edges : n_rows;
  const int64_t C = d->in1_features > d->in2_features ? d->in1_features : d->in2_features;
  int64_t ws = 0;
  if (conv && need_in1) ws += items * (int64_t)ncomp(d->in1_l_max) * d->in1_features;
  if (need_w && d->shared_weights)
    ws += items * (int64_t)count_paths(d->in1_l_max, d->in2_l_max, d->out_l_max, d->symmetric_product != 0, nullptr) * C;
  return ws;
}

extern "C" int fc_tp_bwd(const fc_tp_desc* d, const fc_csr* graph, int64_t n_rows, const float* go, const float* in1,
                         const float* in2, const float* w, float alpha, float* gin1, float* gin2, float* gw,
                         float* ws, int64_t ws_floats, void* stream) {
  int st = check_tp(d);
  if (st != FC_OK) return st;
  const bool conv = graph != nullptr;
  const int64_t rows = conv ? graph->n_nodes : n_rows;
  if (rows < 0) return FC_ERR_SHAPE;
  hipStream_t s = (hipStream_t)stream;
  const int64_t items = conv ? graph->n_edges : rows;
  const int64_t need_ws = fc_tp_bwd_workspace(d, graph, n_rows, gin1 != nullptr, gw != nullptr);
  if (need_ws > 0 && (!ws || ws_floats < need_ws)) return FC_ERR_WORKSPACE;
  if (conv && (!graph->rowptr || !graph->idx_j)) return FC_ERR_NULL;
  if (conv && gin1 && (!graph->sender_perm || !graph->sender_ptr)) return FC_ERR_NULL;
  if (rows > 0 && !go) return FC_ERR_NULL;
  if (items > 0 && (!in1 || !in2 || !w)) return FC_ERR_NULL;
  if (conv && graph->pair_slot && d->shared_weights) return FC_ERR_BAD_DESC;

  TPArgs g = make_args(d, rows);
  g.in1 = in1; g.in2 = in2; g.w = w; g.grad_out = go; g.alpha = alpha;
  // all three gradients of an interaction-layer convolution with few channels: in sender order
  // (no per-edge messages, no segmented sum) when the configuration has a sender-order kernel
  if (conv && gin1 && gin2 && gw && graph->idx_i && !d->shared_weights && graph->n_sender_rows > 0) {
    TPArgs gs = g;
    gs.n_rows = graph->n_sender_rows;
    gs.grad_in1 = gin1; gs.grad_in2 = gin2; gs.grad_w = gw;
    gs.idx_j = graph->idx_j; gs.rowptr = graph->rowptr; gs.wslot = graph->pair_slot; gs.n_edges = graph->n_edges;
    gs.idx_i = graph->idx_i; gs.sperm = graph->sender_perm; gs.sptr = graph->sender_ptr;
    gs.sender_major = 1;
    st = dispatch(d, gs, true, true, s);
    if (st != kSendNotApplicable) return st;
  }
  const int np = count_paths(d->in1_l_max, d->in2_l_max, d->out_l_max, d->symmetric_product != 0, nullptr);
  float* msg = nullptr;
  float* wtmp = nullptr;
  float* cursor = ws;
  if (conv && gin1) { msg = cursor; cursor += items * (int64_t)ncomp(d->in1_l_max) * d->in1_features; }
  if (gw && d->shared_weights) wtmp = cursor;
  g.grad_in1 = conv ? msg : gin1;
  g.grad_in2 = gin2;
  g.grad_w = (gw && d->shared_weights) ? wtmp : gw;
  if (conv) { g.idx_j = graph->idx_j; g.rowptr = graph->rowptr; g.wslot = graph->pair_slot; g.n_edges = graph->n_edges; }
  if (rows > 0) {
    st = dispatch(d, g, conv, true, s);
    if (st != FC_OK) return st;
  }
  if (conv && gin1) {
    const int64_t width = (int64_t)ncomp(d->in1_l_max) * d->in1_features;
    st = segment_sum(graph->n_sender_rows, width, msg, graph->sender_perm, graph->sender_ptr, gin1, s);
    if (st != FC_OK) return st;
  }
  if (gw && d->shared_weights) {
    const int64_t C = g.C;
    st = colsum(items, (int64_t)np * C, wtmp, gw, s);
    if (st != FC_OK) return st;
  }
  return FC_OK;
}

extern "C" int fc_tp_bwd_rows_acc(const fc_tp_desc* d, int64_t n_rows, const float* go, const float* in1,
                                  const float* in2, const float* w, float alpha, const float* res1,
                                  int32_t res1_comps, const float* res2, int32_t res2_comps, float* gin1,
                                  float* gin2, void* stream) {
  int st = check_tp(d);
  if (st != FC_OK) return st;
  if (d->in1_features != d->in2_features || d->reduce_paths) return FC_ERR_BAD_DESC;
  if (n_rows < 0) return FC_ERR_SHAPE;
  if ((res1 && (res1_comps < 0 || res1_comps > ncomp(d->in1_l_max))) ||
      (res2 && (res2_comps < 0 || res2_comps > ncomp(d->in2_l_max))))
    return FC_ERR_SHAPE;
  if (n_rows == 0 || (!gin1 && !gin2)) return FC_OK;
  if (!go || !in1 || !in2 || !w) return FC_ERR_NULL;
  TPArgs g = make_args(d, n_rows);
  g.in1 = in1; g.in2 = in2; g.w = w; g.grad_out = go; g.alpha = alpha;
  g.grad_in1 = gin1;
  g.grad_in2 = gin2;
  g.res1 = res1; g.res1_comps = res1 ? res1_comps : 0;
  g.res2 = res2; g.res2_comps = res2 ? res2_comps : 0;
  return dispatch(d, g, false, true, (hipStream_t)stream);
}
