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
// wave only; every output element is written once. The receiver's edges are taken 64 at a
// time: their species, pair slots and edge attributes go to LDS with one vector load per
// thread (no chain of per-edge scalar loads), then each wave loads the h rows of its edges U
// at a time, all before the first FMA waits for them.
template <int D>
__global__ void __launch_bounds__(256) species_density_fwd_kernel(int64_t n_rows, int n_species, int y_stride,
                                                                  const int32_t* __restrict__ rowptr,
                                                                  const int32_t* __restrict__ pair_slot,
                                                                  const int32_t* __restrict__ zj,
                                                                  const float* __restrict__ h,
                                                                  const float* __restrict__ y, float* __restrict__ dens) {
  constexpr int U = 16, ZW = kSpeciesMax / 4;  // species per wave
  constexpr int B = 64;                        // edges staged per block
  __shared__ int zs[B], ss[B];
  __shared__ float ys[B * D];
  const int64_t row = xcd_row(n_rows);
  if (row >= n_rows) return;
  const int t = threadIdx.x, k = t & 63;
  const int wave = __builtin_amdgcn_readfirstlane(t >> 6);
  float acc[ZW][D];
#pragma unroll
  for (int q = 0; q < ZW; ++q)
#pragma unroll
    for (int c = 0; c < D; ++c) acc[q][c] = 0.f;
  const int32_t e0 = rowptr[row], e1 = rowptr[row + 1];
  for (int32_t b0 = e0; b0 < e1; b0 += B) {
    const int n = e1 - b0 < B ? e1 - b0 : B;
    if (b0 > e0) __syncthreads();  // the previous block's LDS reads are done
    if (t < B) {
      zs[t] = t < n ? zj[b0 + t] : -1;
      ss[t] = t < n ? pair_slot[b0 + t] : -1;
    }
    for (int i = t; i < n * D; i += 256) {
      const int u = i / D, c = i - u * D;
      ys[i] = y[(int64_t)(b0 + u) * y_stride + c];
    }
    __syncthreads();
    for (int u0 = 0; u0 < n; u0 += U) {
      int z[U];
      float hk[U];
      // h only where this wave takes the edge (uniform branches; the loads are all issued before
      // the first FMA waits for them)
#pragma unroll
      for (int u = 0; u < U; ++u) {
        z[u] = u0 + u < n ? __builtin_amdgcn_readfirstlane(zs[u0 + u]) : -1;
        const int sl = u0 + u < n ? __builtin_amdgcn_readfirstlane(ss[u0 + u]) : -1;
        hk[u] = 0.f;
        if ((z[u] & 3) == wave && z[u] >= 0 && z[u] < 4 * ZW && sl >= 0) hk[u] = h[(int64_t)(sl >> 1) * kHid + k];
      }
#pragma unroll
      for (int u = 0; u < U; ++u) {
#pragma unroll
        for (int q = 0; q < ZW; ++q) {
          if (z[u] != wave + 4 * q) continue;  // uniform branch
          const float* yr = ys + (u0 + u) * D;
#pragma unroll
          for (int c = 0; c < D; ++c) acc[q][c] = fmaf(hk[u], yr[c], acc[q][c]);
        }
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
  constexpr int LOGN = N == 1 ? 0 : N == 2 ? 1 : N == 4 ? 2 : N == 8 ? 3 : N == 16 ? 4 : 5;
  static_assert((1 << LOGN) == N, "power of two up to 32");
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
  constexpr int R = D <= 1 ? 1 : D <= 2 ? 2 : D <= 4 ? 4 : D <= 8 ? 8 : D <= 16 ? 16 : 32;  // >= D
  constexpr int SH = R == 1 ? 6 : R == 2 ? 5 : R == 4 ? 4 : R == 8 ? 3 : R == 16 ? 2 : 1;
  static_assert(R >= D, "one reduction slot per component");
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
    case 4: return launch_species<25>(bwd, n_rows, n_species, y_stride, rowptr, slot, zj, h, y, g, g_h, out, s);
  }
  return FC_ERR_UNSUPPORTED_L;
}

// The matrices of the species density's layer map, all ranks in one launch (they are formed
// from the parameters at every evaluation, so a replayed graph sees weights written in place):
//   x[Z, c] = s_first / *alpha_div * sum_j table[Z, j] w_first[c, j]
//   maps[l][o, Z * nh + k] = sum_c w_second[l][o, c] x[Z, c] w_radial[(l * c_mid + c) * nh + k]
// Workgroup (o block of 16, Z, l). x[Z, :] goes to LDS (four threads per row of w_first, each a
// quarter of the row); per chunk of 128 c, the chunk's w_radial rows and the block's w_second
// columns are staged in LDS by all threads at once (the first chunk together with the table row),
// and each thread forms four outputs (o = o0 + t / 16, k = t % 16 + 16 j) from LDS. A few global
// round trips in all: the kernel is latency-bound (tens of workgroups).
struct SpeciesMapsArgs {
  const float* table;
  const float* w_first;
  const float* alpha_div;
  const float* w_second[FC_MAX_RANKS];
  const float* w_radial;
  float* maps[FC_MAX_RANKS];
  float s_first;
  int c_in, c_mid, c_out, nh, n_species;
  bool x_vec;   // c_in a multiple of 16 and w_first 16-byte aligned: rows read as float4
  bool st_vec;  // c_mid and nh multiples of 4, w_radial and w_second 16-byte aligned: staged as float4
};

constexpr int kMapsMaxMid = 1024, kMapsMaxIn = 1024, kMapsChunk = 128;

__global__ void __launch_bounds__(256) species_maps_kernel(SpeciesMapsArgs a) {
  __shared__ float xs[kMapsMaxMid];
  __shared__ __attribute__((aligned(16))) float tb[kMapsMaxIn];
  __shared__ __attribute__((aligned(16))) float w2s[kMapsChunk * 64];
  __shared__ __attribute__((aligned(16))) float wss[16 * kMapsChunk];
  const int t = threadIdx.x, Z = blockIdx.y, l = blockIdx.z;
  const int ol = t >> 4, o = blockIdx.x * 16 + ol;
  const float* w2 = a.w_radial + (int64_t)l * a.c_mid * a.nh;
  const float* ws = a.w_second[l];
  // chunk c0 of w_radial's rows and of the block's w_second columns into LDS
  auto stage = [&](int c0, int cn) {
    if (a.st_vec) {  // float4 loads, eight in flight per thread
      const float4* src = reinterpret_cast<const float4*>(w2 + (int64_t)c0 * a.nh);
      float4* dst = reinterpret_cast<float4*>(w2s);
      const int n4 = cn * a.nh / 4;
#pragma unroll 8
      for (int i = t; i < n4; i += 256) dst[i] = src[i];
      const int q4 = cn / 4;
      for (int i = t; i < 16 * q4; i += 256) {
        const int r = i / q4, cc = 4 * (i - r * q4), oo = blockIdx.x * 16 + r;
        *reinterpret_cast<float4*>(wss + r * kMapsChunk + cc) =
            oo < a.c_out ? *reinterpret_cast<const float4*>(ws + (int64_t)oo * a.c_mid + c0 + cc)
                         : make_float4(0.f, 0.f, 0.f, 0.f);
      }
      return;
    }
    for (int i = t; i < cn * a.nh; i += 256) w2s[i] = w2[(int64_t)c0 * a.nh + i];
    for (int i = t; i < 16 * cn; i += 256) {
      const int r = i / cn, cc = i - r * cn, oo = blockIdx.x * 16 + r;
      wss[r * kMapsChunk + cc] = oo < a.c_out ? ws[(int64_t)oo * a.c_mid + c0 + cc] : 0.f;
    }
  };
  // the first chunk loads together with the table row (neither depends on x)
  for (int j = t; j < a.c_in; j += 256) tb[j] = a.table[(int64_t)Z * a.c_in + j];
  stage(0, a.c_mid < kMapsChunk ? a.c_mid : kMapsChunk);
  const float div = *a.alpha_div;
  __syncthreads();
  // x: four threads per row of w_first, thread q of a row taking the row's quarter q (as float4
  // loads issued eight at a time when the rows allow it: the loads, not the FMAs, set the time)
  const int q = t & 3, qn = (a.c_in + 3) / 4, j0 = q * qn, j1 = j0 + qn < a.c_in ? j0 + qn : a.c_in;
  for (int c0 = 0; c0 < a.c_mid; c0 += 64) {
    const int c = c0 + (t >> 2);
    float d = 0.f;
    if (c < a.c_mid) {
      const float* wr = a.w_first + (int64_t)c * a.c_in;
      if (a.x_vec) {
        const float4* w4 = reinterpret_cast<const float4*>(wr + j0);
        const float4* t4 = reinterpret_cast<const float4*>(tb + j0);
#pragma unroll 8
        for (int j = 0; j < qn / 4; ++j) {
          const float4 w = w4[j], x = t4[j];
          d = fmaf(x.x, w.x, d);
          d = fmaf(x.y, w.y, d);
          d = fmaf(x.z, w.z, d);
          d = fmaf(x.w, w.w, d);
        }
      } else {
        for (int j = j0; j < j1; ++j) d = fmaf(tb[j], wr[j], d);
      }
    }
    d += __shfl_xor(d, 1, 64);
    d += __shfl_xor(d, 2, 64);
    if (q == 0 && c < a.c_mid) xs[c] = d * a.s_first / div;
  }
  float acc[4] = {0.f, 0.f, 0.f, 0.f};
  for (int c0 = 0; c0 < a.c_mid; c0 += kMapsChunk) {
    const int cn = a.c_mid - c0 < kMapsChunk ? a.c_mid - c0 : kMapsChunk;
    if (c0 > 0) {
      __syncthreads();  // the previous chunk consumed
      stage(c0, cn);
    }
    __syncthreads();  // x and this chunk in LDS
    for (int cc = 0; cc < cn; ++cc) {
      const float wx = wss[ol * kMapsChunk + cc] * xs[c0 + cc];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int k = (t & 15) + 16 * j;
        if (k < a.nh) acc[j] = fmaf(wx, w2s[cc * a.nh + k], acc[j]);
      }
    }
  }
  if (o >= a.c_out) return;
  float* mr = a.maps[l] + (int64_t)o * a.n_species * a.nh + (int64_t)Z * a.nh;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int k = (t & 15) + 16 * j;
    if (k < a.nh) mr[k] = acc[j];
  }
}

}  // namespace fc

using namespace fc;

extern "C" int fc_species_maps(int32_t n_species, int32_t c_in, int32_t c_mid, int32_t c_out, int32_t n_hidden,
                               int32_t n_ranks, const float* table, const float* w_first, float s_first,
                               const float* alpha_div, const float* const* w_second, const float* w_radial,
                               float* const* maps, void* stream) {
  if (n_species < 1 || n_species > kSpeciesMax || c_in < 1 || c_out < 1 || n_hidden < 1) return FC_ERR_SHAPE;
  if (c_mid < 1 || c_mid > kMapsMaxMid || c_in > kMapsMaxIn || n_hidden > 64) return FC_ERR_SHAPE;
  if (n_ranks < 1 || n_ranks > FC_MAX_RANKS) return FC_ERR_UNSUPPORTED_L;
  if (!table || !w_first || !alpha_div || !w_second || !w_radial || !maps) return FC_ERR_NULL;
  SpeciesMapsArgs a{};
  for (int l = 0; l < n_ranks; ++l) {
    if (!w_second[l] || !maps[l]) return FC_ERR_NULL;
    a.w_second[l] = w_second[l];
    a.maps[l] = maps[l];
  }
  a.table = table;
  a.w_first = w_first;
  a.alpha_div = alpha_div;
  a.w_radial = w_radial;
  a.s_first = s_first;
  a.c_in = c_in;
  a.c_mid = c_mid;
  a.c_out = c_out;
  a.nh = n_hidden;
  a.n_species = n_species;
  a.x_vec = (c_in % 16) == 0 && ((uintptr_t)w_first & 15) == 0;
  a.st_vec = (c_mid % 4) == 0 && (n_hidden % 4) == 0 && ((uintptr_t)w_radial & 15) == 0;
  for (int l = 0; l < n_ranks; ++l) a.st_vec = a.st_vec && ((uintptr_t)w_second[l] & 15) == 0;
  hipLaunchKernelGGL(species_maps_kernel, dim3((unsigned)((c_out + 15) / 16), (unsigned)n_species, (unsigned)n_ranks),
                     dim3(256), 0, (hipStream_t)stream, a);
  FC_LAUNCH_CHECK();
  return FC_OK;
}

static int check_species(const fc_csr* gr, int32_t l_max, int32_t y_l_max, int32_t n_species) {
  if (!gr) return FC_ERR_NULL;
  if (l_max >= FC_MAX_RANKS || y_l_max >= FC_MAX_RANKS) return FC_ERR_UNSUPPORTED_L;
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
