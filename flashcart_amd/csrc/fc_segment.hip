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

// Wide rows (width >= 64): one workgroup per segment (blockIdx.y splits rows wider than
// 512 columns), threads over columns (float4 when the rows are 16-byte aligned). The rows of
// a segment are summed in order; four are loaded before they are added, so each wave keeps
// four row reads in flight.
template <typename V>
__device__ __forceinline__ void add_to(V& a, const V& b);
template <>
__device__ __forceinline__ void add_to<float4>(float4& a, const float4& b) {
  a.x += b.x; a.y += b.y; a.z += b.z; a.w += b.w;
}
template <>
__device__ __forceinline__ void add_to<float>(float& a, const float& b) { a += b; }

template <typename V>
__device__ __forceinline__ void segment_cols(int64_t w, const V* __restrict__ src, const int32_t* __restrict__ perm,
                                             int32_t k0, int32_t k1, V* __restrict__ dst) {
  for (int64_t c = threadIdx.x + (int64_t)blockIdx.y * blockDim.x; c < w; c += (int64_t)gridDim.y * blockDim.x) {
    V acc{};
    auto row = [&](int32_t k) { return perm ? (int64_t)perm[k] : (int64_t)k; };
    int32_t k = k0;
    for (; k + 4 <= k1; k += 4) {
      const V v0 = src[row(k) * w + c], v1 = src[row(k + 1) * w + c];
      const V v2 = src[row(k + 2) * w + c], v3 = src[row(k + 3) * w + c];
      add_to(acc, v0); add_to(acc, v1); add_to(acc, v2); add_to(acc, v3);
    }
    for (; k < k1; ++k) add_to(acc, src[row(k) * w + c]);
    dst[c] = acc;
  }
}

__global__ void __launch_bounds__(512) segment_rows_kernel(int64_t width, const float* __restrict__ src,
                                                           const int32_t* __restrict__ perm,
                                                           const int32_t* __restrict__ ptr, float* __restrict__ dst,
                                                           int vec4, int64_t n_seg) {
  const int64_t s = xcd_row(n_seg);
  if (s >= n_seg) return;
  const int32_t k0 = ptr[s], k1 = ptr[s + 1];
  if (vec4) {
    segment_cols<float4>(width >> 2, reinterpret_cast<const float4*>(src), perm, k0, k1,
                         reinterpret_cast<float4*>(dst + s * width));
  } else {
    segment_cols<float>(width, src, perm, k0, k1, dst + s * width);
  }
}

// Narrow rows (width < 64, e.g. per-graph energies): one workgroup per segment, threads
// over rows, then a fixed-shape tree reduction (wave64 butterfly + LDS), per column.
__global__ void __launch_bounds__(256) segment_narrow_kernel(int64_t width, const float* __restrict__ src,
                                                             const int32_t* __restrict__ perm,
                                                             const int32_t* __restrict__ ptr,
                                                             float* __restrict__ dst) {
  __shared__ float part[4];
  const int64_t s = blockIdx.x;
  const int32_t k0 = ptr[s], k1 = ptr[s + 1];
  const int t = threadIdx.x;
  for (int64_t c = 0; c < width; ++c) {
    float acc = 0.f;
    for (int32_t k = k0 + t; k < k1; k += blockDim.x) {
      const int64_t r = perm ? (int64_t)perm[k] : (int64_t)k;
      acc += src[r * width + c];
    }
    acc = wave_sum(acc);
    if ((t & 63) == 0) part[t >> 6] = acc;
    __syncthreads();
    if (t == 0) dst[s * width + c] = (part[0] + part[1]) + (part[2] + part[3]);
    __syncthreads();
  }
}

// grad_pos[n] = sum_{sender segment} g[perm[k]] - sum_{receiver segment} g[k], one wave per node:
// lane l takes the segments' edges l, l + 64, ... (its sender edges, then minus its receiver
// edges) and the wave adds the 64 partial sums by a fixed butterfly, so the result does not
// depend on scheduling. (A thread per node component walking its ~50 edges one after another
// left a small graph with a few dozen waves of dependent gathers.)
__global__ void __launch_bounds__(256) edge_grad_to_nodes_kernel(int64_t n_nodes, int64_t n_recv, int64_t n_send,
                                                               const float* __restrict__ g,
                                                               const int32_t* __restrict__ rowptr,
                                                               const int32_t* __restrict__ sperm,
                                                               const int32_t* __restrict__ sptr,
                                                               float* __restrict__ gpos) {
  const int64_t n = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (n >= n_nodes) return;  // uniform over the wave
  float a0 = 0.f, a1 = 0.f, a2 = 0.f;
  if (n < n_send)
    for (int32_t k = sptr[n] + lane; k < sptr[n + 1]; k += 64) {
      const float* r = g + (int64_t)sperm[k] * 3;
      a0 += r[0]; a1 += r[1]; a2 += r[2];
    }
  if (n < n_recv)
    for (int32_t k = rowptr[n] + lane; k < rowptr[n + 1]; k += 64) {
      const float* r = g + (int64_t)k * 3;
      a0 -= r[0]; a1 -= r[1]; a2 -= r[2];
    }
  a0 = wave_sum(a0);
  a1 = wave_sum(a1);
  a2 = wave_sum(a2);
  if (lane < 3) gpos[n * 3 + lane] = lane == 0 ? a0 : (lane == 1 ? a1 : a2);
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
  if (n_seg * width == 0) return FC_OK;
  if (n_seg > 0x7fffffff) return FC_ERR_SHAPE;
  if (width < 64) {
    hipLaunchKernelGGL(segment_narrow_kernel, dim3((unsigned)n_seg), dim3(256), 0, s, width, src, perm, ptr, dst);
  } else {
    const int vec4 = (width % 4 == 0) && (((uintptr_t)src & 15) == 0) && (((uintptr_t)dst & 15) == 0);
    const int64_t cols = vec4 ? width / 4 : width;
    // whole waves covering the columns, at most 512 threads (one workgroup per segment for
    // rows of up to 512 columns: 288 float4 at 9 x 128 take 320 threads)
    const int64_t threads = cols >= 512 ? 512 : (cols + 63) / 64 * 64;
    const unsigned gy = (unsigned)((cols + threads - 1) / threads);
    hipLaunchKernelGGL(segment_rows_kernel, dim3((unsigned)xcd_grid(n_seg), gy), dim3((unsigned)threads), 0, s, width,
                       src, perm, ptr, dst, vec4, n_seg);
  }
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
  hipLaunchKernelGGL(edge_grad_to_nodes_kernel, dim3((unsigned)((rows + 3) / 4)), dim3(256), 0,
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
