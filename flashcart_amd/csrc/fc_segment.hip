// Segmented reductions over sorted index ranges (no atomics, deterministic order).
#include "fc_common.h"

namespace fc {

// rowptr[n] = lower_bound(idx_sorted, n): each edge fills the entries of the node
// range (idx[e-1], idx[e]]; the last edge also fills (idx[E-1], n_nodes].
__global__ void csr_from_sorted_kernel(int64_t n_edges, const int32_t* __restrict__ idx, int64_t n_nodes,
                                       int32_t* __restrict__ rowptr) {
  const int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (e > n_edges) return;
  const int64_t lo = e == 0 ? 0 : (int64_t)idx[e - 1] + 1;
  const int64_t hi = e == n_edges ? n_nodes : (int64_t)idx[e];
  for (int64_t n = lo; n <= hi && n <= n_nodes; ++n) rowptr[n] = (int32_t)e;
}

// dst[s, c] = sum over the segment, one thread per (segment, column).
__global__ void segment_sum_kernel(int64_t n_seg, int64_t width, const float* __restrict__ src,
                                   const int32_t* __restrict__ perm, const int32_t* __restrict__ ptr,
                                   float* __restrict__ dst) {
  const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (t >= n_seg * width) return;
  const int64_t s = t / width, c = t % width;
  float acc = 0.f;
  for (int32_t k = ptr[s]; k < ptr[s + 1]; ++k) {
    const int64_t r = perm ? (int64_t)perm[k] : (int64_t)k;
    acc += src[r * width + c];
  }
  dst[t] = acc;
}

// grad_pos[n] = sum_{sender segment} g[perm[k]] - sum_{receiver segment} g[k]
__global__ void edge_grad_to_nodes_kernel(int64_t n_nodes, int64_t n_recv, int64_t n_send, const float* __restrict__ g,
                                          const int32_t* __restrict__ rowptr, const int32_t* __restrict__ sperm,
                                          const int32_t* __restrict__ sptr, float* __restrict__ gpos) {
  const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (t >= n_nodes * 3) return;
  const int64_t n = t / 3, c = t % 3;
  float acc = 0.f;
  if (n < n_send)
    for (int32_t k = sptr[n]; k < sptr[n + 1]; ++k) acc += g[(int64_t)sperm[k] * 3 + c];
  if (n < n_recv)
    for (int32_t k = rowptr[n]; k < rowptr[n + 1]; ++k) acc -= g[(int64_t)k * 3 + c];
  gpos[t] = acc;
}

// Column sums dst[c] = sum_r src[r, c] in a fixed order (one block per column tile).
__global__ void colsum_kernel(int64_t rows, int64_t cols, const float* __restrict__ src, float* __restrict__ dst) {
  const int64_t c = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (c >= cols) return;
  float acc = 0.f;
  for (int64_t r = 0; r < rows; ++r) acc += src[r * cols + c];
  dst[c] = acc;
}

__global__ void fill_kernel(int64_t n, float v, float* __restrict__ dst) {
  const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (t < n) dst[t] = v;
}

int segment_sum(int64_t n_seg, int64_t width, const float* src, const int32_t* perm, const int32_t* ptr, float* dst,
                hipStream_t s) {
  const int64_t total = n_seg * width;
  if (total == 0) return FC_OK;
  const int bs = 256;
  hipLaunchKernelGGL(segment_sum_kernel, dim3((unsigned)((total + bs - 1) / bs)), dim3(bs), 0, s, n_seg, width, src,
                     perm, ptr, dst);
  FC_LAUNCH_CHECK();
  return FC_OK;
}

int colsum(int64_t rows, int64_t cols, const float* src, float* dst, hipStream_t s) {
  if (cols == 0) return FC_OK;
  const int bs = 256;
  hipLaunchKernelGGL(colsum_kernel, dim3((unsigned)((cols + bs - 1) / bs)), dim3(bs), 0, s, rows, cols, src, dst);
  FC_LAUNCH_CHECK();
  return FC_OK;
}

int fill(int64_t n, float v, float* dst, hipStream_t s) {
  if (n == 0) return FC_OK;
  const int bs = 256;
  hipLaunchKernelGGL(fill_kernel, dim3((unsigned)((n + bs - 1) / bs)), dim3(bs), 0, s, n, v, dst);
  FC_LAUNCH_CHECK();
  return FC_OK;
}

}  // namespace fc

using namespace fc;

extern "C" int fc_csr_from_sorted(int64_t n_edges, const int32_t* idx, int64_t n_nodes, int32_t* rowptr,
                                  void* stream) {
  if (n_edges < 0 || n_nodes < 0) return FC_ERR_SHAPE;
  if (!rowptr || (n_edges > 0 && !idx)) return FC_ERR_NULL;
  const int bs = 256;
  hipLaunchKernelGGL(csr_from_sorted_kernel, dim3((unsigned)((n_edges + 1 + bs - 1) / bs)), dim3(bs), 0,
                     (hipStream_t)stream, n_edges, idx, n_nodes, rowptr);
  FC_LAUNCH_CHECK();
  return FC_OK;
}

extern "C" int fc_edge_grad_to_nodes(const fc_csr* gr, const float* g, float* gpos, void* stream) {
  if (!gr || !gpos) return FC_ERR_NULL;
  if (!gr->rowptr || !gr->sender_perm || !gr->sender_ptr) return FC_ERR_NULL;
  if (gr->n_edges > 0 && !g) return FC_ERR_NULL;
  const int64_t rows = gr->n_sender_rows > gr->n_nodes ? gr->n_sender_rows : gr->n_nodes;
  if (rows == 0) return FC_OK;
  const int bs = 256;
  hipLaunchKernelGGL(edge_grad_to_nodes_kernel, dim3((unsigned)((rows * 3 + bs - 1) / bs)), dim3(bs), 0,
                     (hipStream_t)stream, rows, gr->n_nodes, gr->n_sender_rows, g, gr->rowptr, gr->sender_perm, gr->sender_ptr,
                     gpos);
  FC_LAUNCH_CHECK();
  return FC_OK;
}

extern "C" int fc_segment_sum(int64_t n_seg, int64_t width, const float* src, const int32_t* perm,
                              const int32_t* ptr, float* dst, void* stream) {
  if (n_seg < 0 || width < 0) return FC_ERR_SHAPE;
  if (n_seg * width > 0 && (!ptr || !dst)) return FC_ERR_NULL;
  return segment_sum(n_seg, width, src, perm, ptr, dst, (hipStream_t)stream);
}
