// Float64 equivariant linear map: forward, input gradient and weight gradients.
//
// The reference's linear ops run float64 tensors with float64 accumulation (use_fp64 = True,
// src/flashcart/o3/_linear.py:328-343,382, chosen by dtype in src/flashcart/o3/utils.py:36-50).
// gfx950 issues fp64 FMAs on its vector units at the rate of its fp64 matrix cores (78.6
// TFLOP/s either way), so these are LDS-tiled vector GEMMs: a 64 x 64 output tile per
// 256-thread workgroup, 4 x 4 outputs per thread (rows ty + 16 i, columns tx + 16 j: the LDS
// reads of a wave are broadcasts or 16 consecutive doubles), the reduction in steps of 16
// through LDS. Each output element is written once; the weight gradient's row reduction is
// split over workgroups into partial tiles that a second kernel adds in a fixed order, so
// results are the same run to run.
#include "fc_common.h"

namespace fc {
namespace {

constexpr int F64_T = 64;      // output tile edge
constexpr int F64_KS = 16;     // reduction step
constexpr int F64_MAXB = FC_MAX_RANKS * FC_MAX_RANKS;  // (rank, component) blocks: sum over l of 2l + 1
constexpr int F64_MAXPARTS = 256;

// One (rank l, component c) block of the forward or the input gradient:
//   D[n, j] = s * sum_q A[n, q] B(q, j) (+ R[n, j])
// over the node rows n; node n's row of the block starts at a + n * a_ld in A (and at
// d + n * d_ld, r + n * d_ld in D and R). B(q, j) = w[j * Q + q] when WT (forward: W_l is
// (J, Q) row-major), w[q * J + j] otherwise (input gradient: W_l is (Q, J)).
struct F64Block {
  const double* a;
  const double* w;
  const double* r;  // residual block, or null
  double* d;
  int32_t Q, J;
  double s;
};

struct F64Batch {
  F64Block b[F64_MAXB];
  int64_t n, a_ld, d_ld;
};

template <bool WT>
__global__ void __launch_bounds__(256) linear_f64_kernel(F64Batch bt) {
  const F64Block& B = bt.b[blockIdx.z];
  const int j0 = blockIdx.y * F64_T;
  if (j0 >= B.J) return;  // uniform: a block narrower than the widest one
  const int64_t n0 = (int64_t)blockIdx.x * F64_T;
  __shared__ double As[F64_KS][F64_T + 1];
  __shared__ double Bs[F64_KS][F64_T + 1];
  const int t = threadIdx.x, tx = t & 15, ty = t >> 4;
  double acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = 0.0;
  for (int q0 = 0; q0 < B.Q; q0 += F64_KS) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {  // A: 64 rows x 16 q, consecutive q contiguous
      const int e = t + 256 * i, rr = e >> 4, qq = e & 15;
      const int64_t row = n0 + rr;
      const int q = q0 + qq;
      As[qq][rr] = (row < bt.n && q < B.Q) ? B.a[row * bt.a_ld + q] : 0.0;
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {  // B: 16 q x 64 j, read along the contiguous index
      const int e = t + 256 * i;
      const int qq = WT ? (e & 15) : (e >> 6), jj = WT ? (e >> 4) : (e & 63);
      const int q = q0 + qq, j = j0 + jj;
      double v = 0.0;
      if (q < B.Q && j < B.J) v = WT ? B.w[(int64_t)j * B.Q + q] : B.w[(int64_t)q * B.J + j];
      Bs[qq][jj] = v;
    }
    __syncthreads();
#pragma unroll
    for (int qq = 0; qq < F64_KS; ++qq) {
      double a[4], b[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) a[i] = As[qq][ty + 16 * i];
#pragma unroll
      for (int j = 0; j < 4; ++j) b[j] = Bs[qq][tx + 16 * j];
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = fma(a[i], b[j], acc[i][j]);
    }
    __syncthreads();
  }
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int64_t row = n0 + ty + 16 * i;
    if (row >= bt.n) continue;
    double* drow = B.d + row * bt.d_ld;
    const double* rrow = B.r ? B.r + row * bt.d_ld : nullptr;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int col = j0 + tx + 16 * j;
      if (col < B.J) drow[col] = B.s * acc[i][j] + (rrow ? rrow[col] : 0.0);  // rrow may alias drow
    }
  }
}

// Weight gradient of one rank: G[o, q] = sum over the rows (node n, component c < m) of
// g[n * g_ld + c * O + o] * x[n * x_ld + c * Q + q], O x Q row-major. Part p of `parts`
// covers rows [p R / parts, (p + 1) R / parts) of the R = n m rows (row = n m + c) and
// writes s * G to dw (parts == 1) or its partial G to ws + p O Q.
struct F64WRank {
  const double* g;
  const double* x;
  double* dw;
  double* ws;
  int32_t O, Q, m, tiles_q;
  int32_t tile0;  // first tile of this rank in the grid's x dimension
  double s;
};

struct F64WBatch {
  F64WRank r[FC_MAX_RANKS];
  int32_t n_ranks, parts;
  int64_t n, g_ld, x_ld;
};

__global__ void __launch_bounds__(256) linear_wgrad_f64_kernel(F64WBatch bt) {
  int ri = 0;
  for (int k = 1; k < bt.n_ranks; ++k)
    if ((int)blockIdx.x >= bt.r[k].tile0) ri = k;
  const F64WRank& R = bt.r[ri];
  const int tile = (int)blockIdx.x - R.tile0;
  const int o0 = (tile / R.tiles_q) * F64_T, q0 = (tile % R.tiles_q) * F64_T;
  const int64_t rows = bt.n * R.m;
  const int64_t r_begin = rows * blockIdx.y / bt.parts, r_end = rows * (blockIdx.y + 1) / bt.parts;
  __shared__ double Gs[F64_KS][F64_T + 1];
  __shared__ double Xs[F64_KS][F64_T + 1];
  const int t = threadIdx.x, tx = t & 15, ty = t >> 4;
  double acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = 0.0;
  for (int64_t r0 = r_begin; r0 < r_end; r0 += F64_KS) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {  // 16 rows x 64 columns of each operand, columns contiguous
      const int e = t + 256 * i, rr = e >> 6, cc = e & 63;
      const int64_t row = r0 + rr;
      double gv = 0.0, xv = 0.0;
      if (row < r_end) {
        const int64_t node = row / R.m;
        const int c = (int)(row - node * R.m);
        if (o0 + cc < R.O) gv = R.g[node * bt.g_ld + (int64_t)c * R.O + o0 + cc];
        if (q0 + cc < R.Q) xv = R.x[node * bt.x_ld + (int64_t)c * R.Q + q0 + cc];
      }
      Gs[rr][cc] = gv;
      Xs[rr][cc] = xv;
    }
    __syncthreads();
#pragma unroll
    for (int rr = 0; rr < F64_KS; ++rr) {
      double a[4], b[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) a[i] = Gs[rr][ty + 16 * i];
#pragma unroll
      for (int j = 0; j < 4; ++j) b[j] = Xs[rr][tx + 16 * j];
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = fma(a[i], b[j], acc[i][j]);
    }
    __syncthreads();
  }
  double* const part = bt.parts > 1 ? R.ws + (int64_t)blockIdx.y * R.O * R.Q : nullptr;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int o = o0 + ty + 16 * i;
    if (o >= R.O) continue;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int q = q0 + tx + 16 * j;
      if (q >= R.Q) continue;
      if (part) part[(int64_t)o * R.Q + q] = acc[i][j];
      else R.dw[(int64_t)o * R.Q + q] = R.s * acc[i][j];
    }
  }
}

// dw[k] = s * sum over p = 0, 1, ... of ws[p * size + k]
__global__ void wgrad_f64_reduce_kernel(const double* __restrict__ ws, int parts, int64_t size, double s,
                                        double* __restrict__ dw) {
  const int64_t k = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (k >= size) return;
  double v = 0.0;
  for (int p = 0; p < parts; ++p) v += ws[(int64_t)p * size + k];
  dw[k] = s * v;
}

// dst[r, off:off+width] = src ? src[r, off:off+width] : 0 (row stride row_stride)
__global__ void fill_rows_f64_kernel(int64_t rows, int64_t row_stride, int64_t off, int64_t width,
                                     const double* __restrict__ src, double* __restrict__ dst) {
  const int64_t r = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (r >= rows) return;
  const int64_t base = r * row_stride + off;
  for (int64_t c = threadIdx.x & 63; c < width; c += 64) dst[base + c] = src ? src[base + c] : 0.0;
}

int fill_f64(int64_t rows, int64_t row_stride, int64_t off, int64_t width, const double* src, double* dst,
             hipStream_t s) {
  if (rows * width == 0 || src == dst) return FC_OK;
  hipLaunchKernelGGL(fill_rows_f64_kernel, dim3((unsigned)((rows + 3) / 4)), dim3(256), 0, s, rows, row_stride, off,
                     width, src, dst);
  FC_LAUNCH_CHECK();
  return FC_OK;
}

int check_f64(const fc_linear_desc_f64* d) {
  if (!d) return FC_ERR_NULL;
  if (d->in_l_max < 0 || d->out_l_max < 0) return FC_ERR_BAD_DESC;
  if (d->in_l_max >= FC_MAX_RANKS || d->out_l_max >= FC_MAX_RANKS) return FC_ERR_UNSUPPORTED_L;
  if (d->in_features < 1 || d->out_features < 1) return FC_ERR_BAD_DESC;
  const int common = d->in_l_max < d->out_l_max ? d->in_l_max : d->out_l_max;
  for (int l = 0; l <= d->in_l_max; ++l)
    if (d->in_paths[l] < 1) return FC_ERR_BAD_DESC;
  for (int l = 0; l <= common; ++l)
    if (!d->weight[l]) return FC_ERR_NULL;
  return FC_OK;
}

struct F64Layout {
  int64_t in_dim, out_dim, in_off[FC_MAX_RANKS], out_off[FC_MAX_RANKS];
  int common;
};

F64Layout layout_f64(const fc_linear_desc_f64* d) {
  F64Layout L{};
  L.common = d->in_l_max < d->out_l_max ? d->in_l_max : d->out_l_max;
  int64_t o = 0;
  for (int l = 0; l <= d->in_l_max; ++l) {
    L.in_off[l] = o;
    o += (int64_t)(2 * l + 1) * d->in_features * d->in_paths[l];
  }
  L.in_dim = o;
  o = 0;
  for (int l = 0; l <= d->out_l_max; ++l) {
    L.out_off[l] = o;
    o += (int64_t)(2 * l + 1) * d->out_features;
  }
  L.out_dim = o;
  return L;
}

// Forward (fwd) or input gradient (!fwd) of every shared rank and component in one launch.
int launch_blocks(const fc_linear_desc_f64* d, const F64Layout& L, int64_t n, const double* a, double alpha,
                  const double* residual, double* out, bool fwd, hipStream_t s) {
  F64Batch bt{};
  bt.n = n;
  bt.a_ld = fwd ? L.in_dim : L.out_dim;
  bt.d_ld = fwd ? L.out_dim : L.in_dim;
  int nb = 0, max_j = 0;
  for (int l = 0; l <= L.common; ++l) {
    const int Kin = d->in_features * d->in_paths[l], O = d->out_features;
    for (int c = 0; c < 2 * l + 1; ++c) {
      F64Block& B = bt.b[nb++];
      const int64_t a_off = fwd ? L.in_off[l] + (int64_t)c * Kin : L.out_off[l] + (int64_t)c * O;
      const int64_t d_off = fwd ? L.out_off[l] + (int64_t)c * O : L.in_off[l] + (int64_t)c * Kin;
      B.a = a + a_off;
      B.w = d->weight[l];
      B.r = residual ? residual + d_off : nullptr;
      B.d = out + d_off;
      B.Q = fwd ? Kin : O;
      B.J = fwd ? O : Kin;
      B.s = alpha * d->scale[l];
      if (B.J > max_j) max_j = B.J;
    }
  }
  const dim3 grid((unsigned)((n + F64_T - 1) / F64_T), (unsigned)((max_j + F64_T - 1) / F64_T), (unsigned)nb);
  if (fwd) hipLaunchKernelGGL(linear_f64_kernel<true>, grid, dim3(256), 0, s, bt);
  else hipLaunchKernelGGL(linear_f64_kernel<false>, grid, dim3(256), 0, s, bt);
  FC_LAUNCH_CHECK();
  return FC_OK;
}

// Weight-gradient plan: the ranks with a non-null grad_w, their tiles, and the number of row
// parts (the same for every rank: one launch). Returns the workspace size in doubles.
int64_t plan_wgrad_f64(const fc_linear_desc_f64* d, int64_t n, double* const* grad_w, F64WBatch& wb) {
  wb = F64WBatch{};
  const int common = d->in_l_max < d->out_l_max ? d->in_l_max : d->out_l_max;
  int tiles = 0;
  int64_t elems = 0;
  for (int l = 0; l <= common; ++l) {
    if (!grad_w[l]) continue;
    F64WRank& R = wb.r[wb.n_ranks++];
    R.O = d->out_features;
    R.Q = d->in_features * d->in_paths[l];
    R.m = 2 * l + 1;
    R.tiles_q = (R.Q + F64_T - 1) / F64_T;
    R.tile0 = tiles;
    R.s = d->scale[l];
    tiles += ((R.O + F64_T - 1) / F64_T) * R.tiles_q;
    elems += (int64_t)R.O * R.Q;
  }
  // about 1024 workgroups over the chip, each part at least 256 node rows long
  int64_t parts = (1024 + tiles - 1) / (tiles > 0 ? tiles : 1);
  if (parts > n / 256) parts = n / 256;
  if (parts > F64_MAXPARTS) parts = F64_MAXPARTS;
  if (parts < 1) parts = 1;
  wb.parts = (int32_t)parts;
  return parts > 1 ? parts * elems : 0;
}

}  // namespace
}  // namespace fc

using namespace fc;

extern "C" int fc_linear_fwd_f64(const fc_linear_desc_f64* d, int64_t n, const double* x, double alpha,
                                 const double* residual, double* out, void* stream) {
  int st = check_f64(d);
  if (st != FC_OK) return st;
  if (n < 0) return FC_ERR_SHAPE;
  if (n == 0) return FC_OK;
  if (!x || !out) return FC_ERR_NULL;
  hipStream_t s = (hipStream_t)stream;
  const F64Layout L = layout_f64(d);
  st = launch_blocks(d, L, n, x, alpha, residual, out, true, s);
  if (st != FC_OK) return st;
  if (L.common < d->out_l_max)
    return fill_f64(n, L.out_dim, L.out_off[L.common + 1], L.out_dim - L.out_off[L.common + 1], residual, out, s);
  return FC_OK;
}

extern "C" int fc_linear_dgrad_f64(const fc_linear_desc_f64* d, int64_t n, const double* go, double alpha,
                                   const double* residual, double* gx, void* stream) {
  int st = check_f64(d);
  if (st != FC_OK) return st;
  if (n < 0) return FC_ERR_SHAPE;
  if (n == 0) return FC_OK;
  if (!go || !gx) return FC_ERR_NULL;
  hipStream_t s = (hipStream_t)stream;
  const F64Layout L = layout_f64(d);
  st = launch_blocks(d, L, n, go, alpha, residual, gx, false, s);
  if (st != FC_OK) return st;
  if (L.common < d->in_l_max)
    return fill_f64(n, L.in_dim, L.in_off[L.common + 1], L.in_dim - L.in_off[L.common + 1], residual, gx, s);
  return FC_OK;
}

extern "C" int64_t fc_linear_wgrad_f64_workspace(const fc_linear_desc_f64* d, int64_t n, double* const* grad_w) {
  const int st = check_f64(d);
  if (st != FC_OK) return -st;
  if (n < 0) return -FC_ERR_SHAPE;
  // only which entries are non-NULL matters here (NULL array: every rank)
  double* all[FC_MAX_RANKS];
  for (int l = 0; l < FC_MAX_RANKS; ++l) all[l] = reinterpret_cast<double*>(16);
  F64WBatch wb;
  return plan_wgrad_f64(d, n, grad_w ? grad_w : all, wb);
}

extern "C" int fc_linear_wgrad_f64(const fc_linear_desc_f64* d, int64_t n, const double* go, const double* x,
                                   double alpha, double* const* grad_w, double* workspace, int64_t workspace_doubles,
                                   void* stream) {
  int st = check_f64(d);
  if (st != FC_OK) return st;
  if (n < 0) return FC_ERR_SHAPE;
  if (!grad_w) return FC_ERR_NULL;
  hipStream_t s = (hipStream_t)stream;
  const int common = d->in_l_max < d->out_l_max ? d->in_l_max : d->out_l_max;
  if (n == 0) {  // no rows: zero gradients (a fill kernel, so the call can be graph-captured)
    for (int l = 0; l <= common; ++l)
      if (grad_w[l]) {
        const int64_t sz = (int64_t)d->out_features * d->in_features * d->in_paths[l];
        st = fill_f64(1, sz, 0, sz, nullptr, grad_w[l], s);
        if (st != FC_OK) return st;
      }
    return FC_OK;
  }
  if (!go || !x) return FC_ERR_NULL;
  F64WBatch wb;
  const int64_t need = plan_wgrad_f64(d, n, grad_w, wb);
  if (wb.n_ranks == 0) return FC_OK;
  if (need > 0 && (!workspace || workspace_doubles < need)) return FC_ERR_WORKSPACE;
  const F64Layout L = layout_f64(d);
  wb.n = n;
  wb.g_ld = L.out_dim;
  wb.x_ld = L.in_dim;
  int tiles = 0, k = 0;
  int64_t ws_off = 0;
  for (int l = 0; l <= common; ++l) {
    if (!grad_w[l]) continue;
    F64WRank& R = wb.r[k++];
    R.g = go + L.out_off[l];
    R.x = x + L.in_off[l];
    R.dw = grad_w[l];
    R.ws = need > 0 ? workspace + ws_off : nullptr;
    R.s = alpha * d->scale[l];
    ws_off += (int64_t)wb.parts * R.O * R.Q;
    tiles = R.tile0 + ((R.O + F64_T - 1) / F64_T) * R.tiles_q;
  }
  hipLaunchKernelGGL(linear_wgrad_f64_kernel, dim3((unsigned)tiles, (unsigned)wb.parts), dim3(256), 0, s, wb);
  FC_LAUNCH_CHECK();
  if (wb.parts == 1) return FC_OK;
  for (int i = 0; i < wb.n_ranks; ++i) {
    const F64WRank& R = wb.r[i];
    const int64_t size = (int64_t)R.O * R.Q;
    hipLaunchKernelGGL(wgrad_f64_reduce_kernel, dim3((unsigned)((size + 255) / 256)), dim3(256), 0, s, R.ws, wb.parts,
                       size, R.s, R.dw);
    FC_LAUNCH_CHECK();
  }
  return FC_OK;
}
