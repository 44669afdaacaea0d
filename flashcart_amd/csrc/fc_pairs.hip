// Edge pairs of a full neighbour list: edge (i <- j, S) and its reverse (j <- i, -S).
//
// The interaction layers' radial MLP reads only the edge length, and the length of
// v = (pos[j] - pos[i]) + s is bitwise the same for the reverse edge whenever its shift
// vector is the exact negation of s (IEEE rounding is symmetric under negation, and
// x^2 + y^2 + z^2 does not see the sign). Both edges of a pair therefore get identical
// per-edge weights, which are formed once per pair. This file finds the pairs (receiver rows
// sorted by strictly increasing (sender, shift), as this library's neighbour lists are):
//   pair_slot[e] = 2p (the edge with the lower index) or 2p + 1 (its reverse), pairs
//   numbered in the order of their lower edge, pair_edge[p] = that lower edge and
//   pair_upper[p] = its reverse;
//   counts[0] = edges without a (unique, mutual) reverse, counts[1] = pairs.
// The caller uses the pairing only when counts[0] == 0. Index work only: the result is
// exact and independent of the launch shape.
#include "fc_common.h"

namespace fc {

constexpr int kPairBlock = 256;
constexpr int kPairPerThread = 4;
constexpr int kPairTile = kPairBlock * kPairPerThread;

// Reverse of edge e: the edge of receiver j whose sender is i and whose shift is -S. Rows must
// be sorted by strictly increasing (sender, shift), as the neighbour lists of this library emit
// them; the reverse is then found by bisection. An edge whose key does not exceed its
// predecessor's in the row (unsorted row or duplicate edge) gets -2, so the pairing is refused.
// Senders outside the receiver rows (ghost atoms) have no reverse (-1).
__device__ __forceinline__ int edge_key_cmp(const int32_t* idx_j, const int32_t* shifts, int32_t k, int32_t i,
                                            int32_t t0, int32_t t1, int32_t t2) {
  const int32_t a = idx_j[k];
  if (a != i) return a < i ? -1 : 1;
  if (!shifts) return 0;
  const int32_t b0 = shifts[3 * (int64_t)k], b1 = shifts[3 * (int64_t)k + 1], b2 = shifts[3 * (int64_t)k + 2];
  if (b0 != t0) return b0 < t0 ? -1 : 1;
  if (b1 != t1) return b1 < t1 ? -1 : 1;
  if (b2 != t2) return b2 < t2 ? -1 : 1;
  return 0;
}

__global__ void pair_find_kernel(int64_t n_edges, int64_t n_nodes, const int32_t* __restrict__ idx_i,
                                 const int32_t* __restrict__ idx_j, const int32_t* __restrict__ rowptr,
                                 const int32_t* __restrict__ shifts, int32_t* __restrict__ rev) {
  const int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (e >= n_edges) return;
  const int32_t i = idx_i[e], j = idx_j[e];
  const int32_t s0 = shifts ? shifts[3 * e] : 0, s1 = shifts ? shifts[3 * e + 1] : 0, s2 = shifts ? shifts[3 * e + 2] : 0;
  if (e > 0 && idx_i[e - 1] == i && edge_key_cmp(idx_j, shifts, (int32_t)(e - 1), j, s0, s1, s2) >= 0) {
    rev[e] = -2;  // not strictly after its predecessor in the row
    return;
  }
  int32_t r = -1;
  if (i >= 0 && i < n_nodes && j >= 0 && j < n_nodes) {
    const int32_t k1 = rowptr[j + 1];
    int32_t lo = rowptr[j], hi = k1;  // first entry >= (i, -S)
    while (lo < hi) {
      const int32_t mid = lo + ((hi - lo) >> 1);
      if (edge_key_cmp(idx_j, shifts, mid, i, -s0, -s1, -s2) < 0) lo = mid + 1;
      else hi = mid;
    }
    if (lo < k1 && (int64_t)lo != e && edge_key_cmp(idx_j, shifts, lo, i, -s0, -s1, -s2) == 0) r = lo;
  }
  rev[e] = r;
}

__device__ __forceinline__ bool pair_mutual(const int32_t* rev, int64_t e, int64_t n_edges) {
  const int32_t r = rev[e];
  return r >= 0 && r < n_edges && rev[r] == (int32_t)e;
}

// Sum over the workgroup (kPairBlock threads), valid in thread 0.
__device__ __forceinline__ int block_sum_int(int v, int* lds) {
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  const int t = threadIdx.x;
  if ((t & 63) == 0) lds[t >> 6] = v;
  __syncthreads();
  int s = 0;
  if (t == 0)
    for (int w = 0; w < kPairBlock / 64; ++w) s += lds[w];
  __syncthreads();
  return s;
}

// Per tile of kPairTile edges: number of lower edges of mutual pairs, and of unpaired edges.
__global__ void __launch_bounds__(kPairBlock) pair_count_kernel(int64_t n_edges, const int32_t* __restrict__ rev,
                                                                int32_t* __restrict__ tile_pairs,
                                                                int32_t* __restrict__ tile_bad) {
  __shared__ int lds[kPairBlock / 64];
  const int64_t base = (int64_t)blockIdx.x * kPairTile;
  int np = 0, nb = 0;
  for (int q = 0; q < kPairPerThread; ++q) {
    const int64_t e = base + q * kPairBlock + threadIdx.x;
    if (e >= n_edges) break;
    if (pair_mutual(rev, e, n_edges)) np += (int64_t)rev[e] > e ? 1 : 0;
    else ++nb;
  }
  np = block_sum_int(np, lds);
  nb = block_sum_int(nb, lds);
  if (threadIdx.x == 0) {
    tile_pairs[blockIdx.x] = np;
    tile_bad[blockIdx.x] = nb;
  }
}

// One workgroup: exclusive scan of the tile pair counts (in place), totals into counts.
__global__ void __launch_bounds__(kPairBlock) pair_scan_kernel(int64_t n_tiles, int32_t* __restrict__ tile_pairs,
                                                               const int32_t* __restrict__ tile_bad,
                                                               int32_t* __restrict__ counts) {
  __shared__ int lds[kPairBlock];
  const int t = threadIdx.x;
  int carry = 0, bad = 0;
  for (int64_t c0 = 0; c0 < n_tiles; c0 += kPairBlock) {
    const int64_t k = c0 + t;
    const int v = k < n_tiles ? tile_pairs[k] : 0;
    bad += k < n_tiles ? tile_bad[k] : 0;
    lds[t] = v;
    __syncthreads();
    for (int o = 1; o < kPairBlock; o <<= 1) {  // Hillis-Steele inclusive scan
      const int add = t >= o ? lds[t - o] : 0;
      __syncthreads();
      lds[t] += add;
      __syncthreads();
    }
    if (k < n_tiles) tile_pairs[k] = carry + lds[t] - v;
    carry += lds[kPairBlock - 1];
    __syncthreads();
  }
  __shared__ int bad_lds[kPairBlock / 64];
  bad = block_sum_int(bad, bad_lds);
  if (t == 0) {
    counts[0] = bad;
    counts[1] = carry;
  }
}

// Pair ids in edge order: the lower edge of pair p writes pair_edge[p] and both slots.
__global__ void __launch_bounds__(kPairBlock) pair_assign_kernel(int64_t n_edges, const int32_t* __restrict__ rev,
                                                                 const int32_t* __restrict__ tile_off,
                                                                 int64_t max_pairs, int32_t* __restrict__ pair_slot,
                                                                 int32_t* __restrict__ pair_edge,
                                                                 int32_t* __restrict__ pair_upper) {
  __shared__ int lds[kPairBlock];
  const int t = threadIdx.x;
  const int64_t base = (int64_t)blockIdx.x * kPairTile + (int64_t)t * kPairPerThread;  // contiguous per thread
  int flag[kPairPerThread];
  int mine = 0;
  for (int q = 0; q < kPairPerThread; ++q) {
    const int64_t e = base + q;
    flag[q] = 0;
    if (e < n_edges) {
      if (pair_mutual(rev, e, n_edges)) flag[q] = (int64_t)rev[e] > e ? 1 : 0;
      else pair_slot[e] = -1;
    }
    mine += flag[q];
  }
  lds[t] = mine;
  __syncthreads();
  for (int o = 1; o < kPairBlock; o <<= 1) {
    const int add = t >= o ? lds[t - o] : 0;
    __syncthreads();
    lds[t] += add;
    __syncthreads();
  }
  int64_t p = (int64_t)tile_off[blockIdx.x] + lds[t] - mine;
  for (int q = 0; q < kPairPerThread; ++q) {
    if (!flag[q]) continue;
    const int64_t e = base + q;
    if (p < max_pairs) {
      pair_edge[p] = (int32_t)e;
      if (pair_upper) pair_upper[p] = rev[e];
      pair_slot[e] = (int32_t)(2 * p);
      pair_slot[rev[e]] = (int32_t)(2 * p + 1);
    }
    ++p;
  }
}

// Radial-MLP inputs of the pairs: x[p, k] = feats[e_p, k] * env[e_p] with e_p = pair_edge[p].
__global__ void pair_inputs_fwd_kernel(int64_t n_pairs, int width, const int32_t* __restrict__ pair_edge,
                                       const float* __restrict__ feats, const float* __restrict__ env,
                                       float* __restrict__ x) {
  const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (t >= n_pairs * width) return;
  const int64_t p = t / width;
  const int k = (int)(t - p * width);
  const int64_t e = pair_edge[p];
  x[t] = feats[e * width + k] * env[e];
}

// Its backward for every edge: the lower edge of pair p takes the pair's gradient, the other
// edge of the pair none (each edge row written once, no fill needed). G lanes per edge (G a
// power of two >= width, at most 64), lane k handling column k; the envelope gradient is the
// sum over the group's lanes.
template <int G>
__global__ void pair_inputs_bwd_kernel(int64_t n_edges, int width, const int32_t* __restrict__ pair_slot,
                                       const float* __restrict__ feats, const float* __restrict__ env,
                                       const float* __restrict__ gx, float* __restrict__ g_feats,
                                       float* __restrict__ g_env) {
  const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t e = t / G;
  const int k = (int)(t % G);
  const bool on = e < n_edges && k < width;
  float g = 0.f, f = 0.f, en = 0.f;
  if (on) {
    const int32_t s = pair_slot[e];
    en = env[e];
    f = feats[e * width + k];
    g = (s & 1) == 0 ? gx[(int64_t)(s >> 1) * width + k] : 0.f;
    if (g_feats) g_feats[e * width + k] = g * en;
  }
  float acc = g * f;
#pragma unroll
  for (int o = G / 2; o > 0; o >>= 1) acc += __shfl_xor(acc, o, 64);
  if (g_env && e < n_edges && k == 0) g_env[e] = acc;
}

}  // namespace fc

using namespace fc;

extern "C" int fc_pair_inputs_fwd(int64_t n_pairs, int32_t width, const int32_t* pair_edge, const float* feats,
                                  const float* env, float* x, void* stream) {
  if (n_pairs < 0 || width < 1) return FC_ERR_SHAPE;
  if (n_pairs == 0) return FC_OK;
  if (!pair_edge || !feats || !env || !x) return FC_ERR_NULL;
  const int64_t n = n_pairs * width;
  hipLaunchKernelGGL(pair_inputs_fwd_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, (hipStream_t)stream,
                     n_pairs, width, pair_edge, feats, env, x);
  FC_LAUNCH_CHECK();
  return FC_OK;
}

extern "C" int fc_pair_inputs_bwd(int64_t n_edges, int32_t width, const int32_t* pair_slot, const float* feats,
                                  const float* env, const float* gx, float* g_feats, float* g_env, void* stream) {
  if (n_edges < 0 || width < 1) return FC_ERR_SHAPE;
  if (n_edges == 0 || (!g_feats && !g_env)) return FC_OK;
  if (!pair_slot || !feats || !env || !gx) return FC_ERR_NULL;
  if (width > 64) return FC_ERR_SHAPE;
  int g = 1;
  while (g < width) g <<= 1;
  const int64_t threads = n_edges * g;
  const dim3 grid((unsigned)((threads + 255) / 256)), block(256);
  hipStream_t s = (hipStream_t)stream;
  switch (g) {
    case 1: hipLaunchKernelGGL(pair_inputs_bwd_kernel<1>, grid, block, 0, s, n_edges, width, pair_slot, feats, env, gx, g_feats, g_env); break;
    case 2: hipLaunchKernelGGL(pair_inputs_bwd_kernel<2>, grid, block, 0, s, n_edges, width, pair_slot, feats, env, gx, g_feats, g_env); break;
    case 4: hipLaunchKernelGGL(pair_inputs_bwd_kernel<4>, grid, block, 0, s, n_edges, width, pair_slot, feats, env, gx, g_feats, g_env); break;
    case 8: hipLaunchKernelGGL(pair_inputs_bwd_kernel<8>, grid, block, 0, s, n_edges, width, pair_slot, feats, env, gx, g_feats, g_env); break;
    case 16: hipLaunchKernelGGL(pair_inputs_bwd_kernel<16>, grid, block, 0, s, n_edges, width, pair_slot, feats, env, gx, g_feats, g_env); break;
    case 32: hipLaunchKernelGGL(pair_inputs_bwd_kernel<32>, grid, block, 0, s, n_edges, width, pair_slot, feats, env, gx, g_feats, g_env); break;
    default: hipLaunchKernelGGL(pair_inputs_bwd_kernel<64>, grid, block, 0, s, n_edges, width, pair_slot, feats, env, gx, g_feats, g_env); break;
  }
  FC_LAUNCH_CHECK();
  return FC_OK;
}

extern "C" int64_t fc_edge_pairs_workspace(int64_t n_edges) {
  if (n_edges < 0) return -FC_ERR_SHAPE;
  const int64_t tiles = (n_edges + kPairTile - 1) / kPairTile;
  return n_edges + 2 * tiles;
}

extern "C" int fc_edge_pairs(const fc_csr* gr, const int32_t* idx_i, const int32_t* shifts, int32_t* pair_slot,
                             int32_t* pair_edge, int32_t* pair_upper, int32_t* reverse, int64_t max_pairs,
                             int32_t* counts, int32_t* workspace, int64_t workspace_ints, void* stream) {
  if (!gr || !counts) return FC_ERR_NULL;
  const int64_t E = gr->n_edges;
  if (E < 0 || gr->n_nodes < 0 || max_pairs < 0) return FC_ERR_SHAPE;
  if (E > 0x7ffffffe) return FC_ERR_SHAPE;
  if (workspace_ints < fc_edge_pairs_workspace(E) || (E > 0 && !workspace)) return FC_ERR_WORKSPACE;
  if (E > 0 && (!idx_i || !gr->idx_j || !gr->rowptr || !pair_slot || (max_pairs > 0 && !pair_edge)))
    return FC_ERR_NULL;
  hipStream_t s = (hipStream_t)stream;
  const int64_t tiles = (E + kPairTile - 1) / kPairTile;
  int32_t* rev = reverse ? reverse : workspace;
  int32_t* tile_pairs = workspace + E;
  int32_t* tile_bad = tile_pairs + tiles;
  if (E > 0) {
    hipLaunchKernelGGL(pair_find_kernel, dim3((unsigned)((E + 255) / 256)), dim3(256), 0, s, E, gr->n_nodes, idx_i,
                       gr->idx_j, gr->rowptr, shifts, rev);
    FC_LAUNCH_CHECK();
    hipLaunchKernelGGL(pair_count_kernel, dim3((unsigned)tiles), dim3(kPairBlock), 0, s, E, rev, tile_pairs, tile_bad);
    FC_LAUNCH_CHECK();
  }
  // also run for E == 0: it writes the zero counts
  hipLaunchKernelGGL(pair_scan_kernel, dim3(1), dim3(kPairBlock), 0, s, tiles, tile_pairs, tile_bad, counts);
  FC_LAUNCH_CHECK();
  if (E > 0) {
    hipLaunchKernelGGL(pair_assign_kernel, dim3((unsigned)tiles), dim3(kPairBlock), 0, s, E, rev, tile_pairs,
                       max_pairs, pair_slot, pair_edge, pair_upper);
    FC_LAUNCH_CHECK();
  }
  return FC_OK;
}
