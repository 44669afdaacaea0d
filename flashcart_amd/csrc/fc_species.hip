// First interaction layer as a species density (energy + forces inference).
//
// In the first interaction layer the sender features are rank 0 and depend on the species
// alone (x_j = linear_first(embedding)[Z_j]), the weights are the radial MLP's output layer
// over its last hidden activation h_e (64 values, no bias), and the paths (0, l, l) have
// coefficient 1 (reference nn/layers.py:351-369, src/flashcart/o3/_codegen_tensor_product.py
// :399-414). With per-edge weights w_e[l, c] = s2 sum_k W2[l C + c, k] h_e[k]:
//   out[i, (l, m), c] = alpha sum_{e -> i} w_e[l, c] x_{Z_j}[c] y_e[(l, m)]
//                     = alpha s2 sum_{Z, k} x_Z[c] W2[l C + c, k] A_i[(l, m), Z, k],
//   A_i[(l, m), Z, k] = sum_{e -> i, Z_j = Z} h_e[k] y_e[(l, m)].
// So the layer is a per-receiver density A (this file, a segmented sum over the receiver's
// edges, no atomics) followed by one equivariant linear map per rank over K = n_species x 64
// (fc_linear_fwd with in_features 64, in_paths n_species): the E x paths x C weight tensor of
// the edge-wise path is never formed. The backward mirrors it: dA from the linear map's input
// gradient (fc_linear_dgrad), then per edge
//   dL/dh_e[k] = sum_{(l, m)} dA_i[(l, m), Z_j, k] y_e[(l, m)],
//   dL/dy_e[(l, m)] = sum_k dA_i[(l, m), Z_j, k] h_e[k].
// h is stored per edge pair (edge e reads row pair_slot[e] / 2); dL/dh is written per edge at
// row pair_slot[e] (pair-major), so a pair's two rows sum to the gradient of its h row.
#include "fc_common.h"

namespace fc {

constexpr int kSpeciesMax = 8;  // species of the density (register/LDS budget)
constexpr int kHid = 64;        // hidden width of the radial MLP

// One workgroup (256 threads) per receiver: wave w accumulates the senders of species w and
// w + 4 (lane k: hidden index k, all components in registers), so each edge costs FMAs in one
// wave only; every output element is written once. Edges are taken U at a time, the batch's
// species, pair slots, h values and edge attributes loaded before any is used.
template <int D>
__global__ void __launch_bounds__(256) species_density_fwd_kernel(int64_t n_rows, int n_species, int y_stride,
                                                                  const int32_t* __restrict__ rowptr,
                                                                  const int32_t* __restrict__ pair_slot,
                                                                  const int32_t* __restrict__ zj,
                                                                  const float* __restrict__ h,
                                                                  const float* __restrict__ y, float* __restrict__ dens) {
  constexpr int U = 16, ZW = kSpeciesMax / 4;  // species per wave
  const int64_t row = xcd_row(n_rows);
  if (row >= n_rows) return;
  const int k = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  float acc[ZW][D];
#pragma unroll
  for (int q = 0; q < ZW; ++q)
#pragma unroll
    for (int c = 0; c < D; ++c) acc[q][c] = 0.f;
  const int32_t e0 = rowptr[row], e1 = rowptr[row + 1];
  for (int32_t b = e0; b < e1; b += U) {
    int z[U], sl[U];
    float hk[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int32_t e = b + u < e1 ? b + u : e1 - 1;  // clamped; the duplicate is skipped below
      z[u] = b + u < e1 ? zj[e] : -1;
      sl[u] = pair_slot[e];
    }
    // h only where this wave takes the edge (uniform branches; the loads are all issued before
    // the first FMA waits for them)
#pragma unroll
    for (int u = 0; u < U; ++u) {
      hk[u] = 0.f;
      if ((z[u] & 3) == wave && z[u] < 4 * ZW && sl[u] >= 0) hk[u] = h[(int64_t)(sl[u] >> 1) * kHid + k];
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
#pragma unroll
      for (int q = 0; q < ZW; ++q) {
        if (z[u] != wave + 4 * q) continue;  // uniform branch
        const float* yr = y + (int64_t)(b + u) * y_stride;
#pragma unroll
        for (int c = 0; c < D; ++c) acc[q][c] = fmaf(hk[u], yr[c], acc[q][c]);
      }
    }
  }
  float* o = dens + row * (int64_t)D * n_species * kHid;
#pragma unroll
  for (int q = 0; q < ZW; ++q) {
    const int z = wave + 4 * q;
    if (z >= n_species) continue;
#pragma unroll
    for (int c = 0; c < D; ++c) o[((int64_t)c * n_species + z) * kHid + k] = acc[q][c];
  }
}

// Sum of N values over the 64 lanes of a wave (N a power of two): afterwards lane group
// lane >> (6 - log2 N) == v holds the total of value v.
template <int N>
__device__ __forceinline__ float wave_reduce_n(float (&v)[N], int lane) {
  constexpr int LOGN = N == 1 ? 0 : N == 2 ? 1 : N == 4 ? 2 : N == 8 ? 3 : 4;
  static_assert((1 << LOGN) == N, "power of two up to 16");
#pragma unroll
  for (int s = 0; s < LOGN; ++s) {
    const int half = N >> (s + 1);
    const int o = 32 >> s;
    const bool lower = (lane & o) == 0;
#pragma unroll
    for (int j = 0; j < half; ++j) {
      // the empty asm makes a and b plain values: the optimizer would otherwise turn the two
      // selects of array elements into one element load at a lane-dependent index, which is
      // lowered to a compare-and-select chain over the whole array
      float a = v[j], b = v[j + half];
      asm volatile("" : "+v"(a), "+v"(b));
      const float mine = lower ? a : b;
      const float send = lower ? b : a;
      v[j] = mine + __shfl_xor(send, o, 64);
    }
  }
  float r = v[0];
#pragma unroll
  for (int o = 32 >> LOGN; o > 0; o >>= 1) r += __shfl_xor(r, o, 64);
  return r;
}

// Backward: one workgroup per receiver; dA_i staged in LDS (dynamic, D x n_species x 64 floats);
// wave w takes edges e0 + w + 4 u, U of them at a time with their operands loaded first; lane
// k forms dL/dh_e[k] and the wave reduces dL/dy_e over k (components of y above the layer's
// ranks get zero).
template <int D>
__global__ void __launch_bounds__(256) species_density_bwd_kernel(int64_t n_rows, int n_species, int y_stride,
                                                                  const int32_t* __restrict__ rowptr,
                                                                  const int32_t* __restrict__ pair_slot,
                                                                  const int32_t* __restrict__ zj,
                                                                  const float* __restrict__ h,
                                                                  const float* __restrict__ y,
                                                                  const float* __restrict__ g_dens,
                                                                  float* __restrict__ g_h, float* __restrict__ g_y) {
  constexpr int R = D <= 1 ? 1 : D <= 2 ? 2 : D <= 4 ? 4 : D <= 8 ? 8 : 16;
  constexpr int SH = R == 1 ? 6 : R == 2 ? 5 : R == 4 ? 4 : R == 8 ? 3 : 2;
  constexpr int U = 4;
  extern __shared__ float ga[];
  const int64_t row = xcd_row(n_rows);
  if (row >= n_rows) return;
  const int t = threadIdx.x, lane = t & 63;
  const int wave = __builtin_amdgcn_readfirstlane(t >> 6);  // uniform: the edge operands are scalar loads
  const int32_t e0 = rowptr[row], e1 = rowptr[row + 1];
  if (e0 >= e1) return;  // uniform over the workgroup: no barrier is skipped by a part of it
  const int per = D * n_species * kHid;
  const float4* gd = reinterpret_cast<const float4*>(g_dens + row * (int64_t)per);
  for (int i = t; i < per / 4; i += 256) reinterpret_cast<float4*>(ga)[i] = gd[i];
  __syncthreads();
  for (int32_t b = e0 + wave; b < e1; b += 4 * U) {
    int z[U], sl[U];
    float hk[U], yv[U][D];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int32_t e = b + 4 * u < e1 ? b + 4 * u : b;  // clamped; skipped below
      z[u] = zj[e];
      sl[u] = pair_slot[e];
#pragma unroll
      for (int c = 0; c < D; ++c) yv[u][c] = y[(int64_t)e * y_stride + c];
    }
#pragma unroll
    for (int u = 0; u < U; ++u) hk[u] = sl[u] >= 0 ? h[(int64_t)(sl[u] >> 1) * kHid + lane] : 0.f;
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int32_t e = b + 4 * u;
      if (e >= e1) continue;  // uniform (no break: the loop must unroll, its arrays stay in registers)
      float gh = 0.f;
      float gyv[R];
#pragma unroll
      for (int c = 0; c < R; ++c) gyv[c] = 0.f;
      if (z[u] >= 0 && z[u] < n_species) {
#pragma unroll
        for (int c = 0; c < D; ++c) {
          const float a = ga[(c * n_species + z[u]) * kHid + lane];
          gh = fmaf(a, yv[u][c], gh);
          gyv[c] = a * hk[u];
        }
      }
      if (sl[u] >= 0) g_h[(int64_t)sl[u] * kHid + lane] = gh;  // an unpaired edge has no h row
      const float r = wave_reduce_n<R>(gyv, lane);
      const int v = lane >> SH;
      if ((lane & ((1 << SH) - 1)) == 0 && v < D) g_y[(int64_t)e * y_stride + v] = r;
      for (int c = D + lane; c < y_stride; c += 64) g_y[(int64_t)e * y_stride + c] = 0.f;
    }
  }
}

template <int D>
static int launch_species(bool bwd, int64_t n_rows, int n_species, int y_stride, const int32_t* rowptr,
                          const int32_t* slot, const int32_t* zj, const float* h, const float* y,
                          const float* dens_or_grad, float* g_h, float* out, hipStream_t s) {
  const dim3 grid((unsigned)xcd_grid(n_rows)), block(256);
  if (!bwd)
    hipLaunchKernelGGL(species_density_fwd_kernel<D>, grid, block, 0, s, n_rows, n_species, y_stride, rowptr, slot, zj,
                       h, y, out);
  else
    hipLaunchKernelGGL(species_density_bwd_kernel<D>, grid, block, (size_t)D * n_species * kHid * sizeof(float), s,
                       n_rows, n_species, y_stride, rowptr, slot, zj, h, y, dens_or_grad, g_h, out);
  FC_LAUNCH_CHECK();
  return FC_OK;
}

static int dispatch_species(int l_max, bool bwd, int64_t n_rows, int n_species, int y_stride, const int32_t* rowptr,
                            const int32_t* slot, const int32_t* zj, const float* h, const float* y, const float* g,
                            float* g_h, float* out, hipStream_t s) {
  switch (l_max) {
    case 0: return launch_species<1>(bwd, n_rows, n_species, y_stride, rowptr, slot, zj, h, y, g, g_h, out, s);
    case 1: return launch_species<4>(bwd, n_rows, n_species, y_stride, rowptr, slot, zj, h, y, g, g_h, out, s);
    case 2: return launch_species<9>(bwd, n_rows, n_species, y_stride, rowptr, slot, zj, h, y, g, g_h, out, s);
    case 3: return launch_species<16>(bwd, n_rows, n_species, y_stride, rowptr, slot, zj, h, y, g, g_h, out, s);
  }
  return FC_ERR_UNSUPPORTED_L;
}

}  // namespace fc

using namespace fc;

static int check_species(const fc_csr* gr, int32_t l_max, int32_t y_l_max, int32_t n_species) {
  if (!gr) return FC_ERR_NULL;
  if (l_max > 3 || y_l_max > 3) return FC_ERR_UNSUPPORTED_L;
  if (l_max < 0 || l_max > y_l_max) return FC_ERR_BAD_DESC;
  if (n_species < 1 || n_species > kSpeciesMax) return FC_ERR_SHAPE;
  if (gr->n_nodes < 0 || gr->n_edges < 0) return FC_ERR_SHAPE;
  if (gr->n_nodes > 0 && !gr->rowptr) return FC_ERR_NULL;
  if (gr->n_edges > 0 && !gr->pair_slot) return FC_ERR_NULL;
  return FC_OK;
}

extern "C" int fc_species_density_fwd(const fc_csr* gr, int32_t l_max, int32_t y_l_max, int32_t n_species,
                                      const int32_t* edge_species, const float* h, const float* y, float* dens,
                                      void* stream) {
  int st = check_species(gr, l_max, y_l_max, n_species);
  if (st != FC_OK) return st;
  if (gr->n_nodes == 0) return FC_OK;
  if (!dens || (gr->n_edges > 0 && (!edge_species || !h || !y))) return FC_ERR_NULL;
  return dispatch_species(l_max, false, gr->n_nodes, n_species, (y_l_max + 1) * (y_l_max + 1), gr->rowptr,
                          gr->pair_slot, edge_species, h, y, nullptr, nullptr, dens, (hipStream_t)stream);
}

extern "C" int fc_species_density_bwd(const fc_csr* gr, int32_t l_max, int32_t y_l_max, int32_t n_species,
                                      const int32_t* edge_species, const float* h, const float* y,
                                      const float* g_dens, float* g_h, float* g_y, void* stream) {
  int st = check_species(gr, l_max, y_l_max, n_species);
  if (st != FC_OK) return st;
  if (gr->n_nodes == 0 || gr->n_edges == 0) return FC_OK;
  if (!edge_species || !h || !y || !g_dens || !g_h || !g_y) return FC_ERR_NULL;
  if (((uintptr_t)g_dens & 15) != 0) return FC_ERR_SHAPE;  // staged as float4
  return dispatch_species(l_max, true, gr->n_nodes, n_species, (y_l_max + 1) * (y_l_max + 1), gr->rowptr,
                          gr->pair_slot, edge_species, h, y, g_dens, g_h, g_y, (hipStream_t)stream);
}
