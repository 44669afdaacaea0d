// Device neighbour list: the cell-list search of fc_neighbor_list (fc_neighbors.cpp) on the
// GPU, for structures whose positions already live in HBM (an MD step, a batch built on
// the device). Replaces NeighborList.build (reference src/flashcart/data/neighbors.py:56-77,
// :120-143) like the host list, and returns the same pairs in the same order:
// (i, j, S) with |pos[j] - pos[i] + S.cell| < cutoff, self pairs with S = 0 removed,
// sorted by (i, j, Sx, Sy, Sz).
//
// Same edge set as the host list, bit for bit: fractional coordinates, wrapping, image
// positions and squared distances are evaluated in float64 with the host's expressions
// and operation order, and without fused multiply-adds (this file is compiled with
// -ffp-contract=off; the host build has none), so every comparison with cutoff^2 takes
// the same branch.
//
// Steps (one stream, two small device-to-host reads):
//   wrap:  fractional coordinates, wrapped into [0, 1) along periodic axes (+ integer offsets)
//   range: min / max of the fractional coordinates along open axes (read back)
//   bin:   bins of fractional width >= reach (cutoff / plane spacing) over the unit cell
//          (periodic axes) or [min, max] (open axes); counting sort of the atoms by bin
//   count: one wave per receiver visits its (2D+1)^3 neighbouring bins, periodic bins
//          through their image shift (virtual bin v = bin + shift * bins, so every
//          (atom, image) candidate appears once), and counts the pairs (ballot)
//   scan:  receiver offsets (read back: the number of pairs)
//   fill:  one wave per receiver collects its pairs' keys (j, S) in LDS, sorts them
//          (bitonic) and writes them at its offset.
#include <cmath>
#include <mutex>

#include "fc_common.h"

namespace fc {

constexpr int kNLMaxPerAtom = 1024;  // pairs per receiver held in LDS by the fill kernel
constexpr int kNLShiftBias = 512;    // shift components packed in 10 bits each: |S| < 512

struct NLPlan {
  double cell[9], inv[9];
  double base[3], width[3];
  double c2;
  int32_t nb[3], D[3], pbc[3];
  int64_t n;
};

__device__ __forceinline__ int nl_bin_of(double f, double base, double width, int nb) {
  int v = (int)floor((f - base) / width);
  return v < 0 ? 0 : (v >= nb ? nb - 1 : v);
}

__global__ void nl_wrap_kernel(NLPlan p, const double* __restrict__ pos, double* __restrict__ w,
                               int32_t* __restrict__ off) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= p.n) return;
  for (int k = 0; k < 3; ++k) {
    const double f = pos[3 * i] * p.inv[k] + pos[3 * i + 1] * p.inv[3 + k] + pos[3 * i + 2] * p.inv[6 + k];
    if (p.pbc[k]) {
      const double fl = floor(f);
      w[3 * i + k] = f - fl;
      off[3 * i + k] = (int32_t)fl;
    } else {
      w[3 * i + k] = f;
      off[3 * i + k] = 0;
    }
  }
}

// min / max of the fractional coordinates per axis (one workgroup of 256 threads).
__global__ void __launch_bounds__(256) nl_range_kernel(int64_t n, const double* __restrict__ w,
                                                       double* __restrict__ out) {
  __shared__ double lo[3][256], hi[3][256];
  const int t = threadIdx.x;
  double l[3] = {1e300, 1e300, 1e300}, h[3] = {-1e300, -1e300, -1e300};
  for (int64_t i = t; i < n; i += 256)
    for (int k = 0; k < 3; ++k) {
      l[k] = fmin(l[k], w[3 * i + k]);
      h[k] = fmax(h[k], w[3 * i + k]);
    }
  for (int k = 0; k < 3; ++k) {
    lo[k][t] = l[k];
    hi[k][t] = h[k];
  }
  __syncthreads();
  for (int s = 128; s > 0; s >>= 1) {
    if (t < s)
      for (int k = 0; k < 3; ++k) {
        lo[k][t] = fmin(lo[k][t], lo[k][t + s]);
        hi[k][t] = fmax(hi[k][t], hi[k][t + s]);
      }
    __syncthreads();
  }
  if (t < 3) {
    out[t] = lo[t][0];
    out[3 + t] = hi[t][0];
  }
}

__global__ void nl_fill_int_kernel(int64_t n, int32_t* __restrict__ a, int32_t v) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) a[i] = v;
}

__global__ void nl_bin_kernel(NLPlan p, const double* __restrict__ w, int32_t* __restrict__ bin,
                              int32_t* __restrict__ hist) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= p.n) return;
  int b[3];
  for (int k = 0; k < 3; ++k) b[k] = nl_bin_of(w[3 * i + k], p.base[k], p.width[k], p.nb[k]);
  const int id = (b[0] * p.nb[1] + b[1]) * p.nb[2] + b[2];
  bin[i] = id;
  atomicAdd(&hist[id], 1);
}

// The order of atoms inside a bin depends on scheduling; the fill kernel sorts every
// receiver's pairs, so the output does not.
__global__ void nl_scatter_kernel(int64_t n, const int32_t* __restrict__ bin, const int64_t* __restrict__ head,
                                  int32_t* __restrict__ cursor, int32_t* __restrict__ order) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  const int id = bin[i];
  order[head[id] + atomicAdd(&cursor[id], 1)] = (int32_t)i;
}

// Exclusive prefix sum of n counts into out[0..n] (out[n] = total), one workgroup of 1024
// threads, each scanning a contiguous chunk.
__global__ void __launch_bounds__(1024) nl_scan_kernel(int64_t n, const int32_t* __restrict__ in,
                                                        int64_t* __restrict__ out) {
  __shared__ int64_t part[1024];
  const int t = threadIdx.x;
  const int64_t chunk = (n + 1023) / 1024;
  const int64_t a = t * chunk, b = a + chunk < n ? a + chunk : n;
  int64_t s = 0;
  for (int64_t i = a; i < b; ++i) s += in[i];
  part[t] = s;
  __syncthreads();
  for (int o = 1; o < 1024; o <<= 1) {
    const int64_t v = t >= o ? part[t - o] : 0;
    __syncthreads();
    part[t] += v;
    __syncthreads();
  }
  int64_t run = part[t] - s;  // exclusive prefix of this chunk
  for (int64_t i = a; i < b; ++i) {
    out[i] = run;
    run += in[i];
  }
  if (t == 1023) out[n] = part[1023];
}

// Visit every candidate (j, image) of receiver i; calls hit(j, S) for the pairs within the
// cutoff. Lanes of the wave stride over the atoms of each bin.
template <class F>
__device__ __forceinline__ void nl_visit(const NLPlan& p, int64_t i, const double* __restrict__ w,
                                         const int32_t* __restrict__ off, const int64_t* __restrict__ head,
                                         const int32_t* __restrict__ order, int lane, F&& hit) {
  const double wi[3] = {w[3 * i], w[3 * i + 1], w[3 * i + 2]};
  double xi[3];
  for (int k = 0; k < 3; ++k) xi[k] = wi[0] * p.cell[k] + wi[1] * p.cell[3 + k] + wi[2] * p.cell[6 + k];
  int b[3];
  for (int k = 0; k < 3; ++k) b[k] = nl_bin_of(wi[k], p.base[k], p.width[k], p.nb[k]);
  const int oi[3] = {off[3 * i], off[3 * i + 1], off[3 * i + 2]};
  for (int v0 = b[0] - p.D[0]; v0 <= b[0] + p.D[0]; ++v0) {
    if (!p.pbc[0] && (v0 < 0 || v0 >= p.nb[0])) continue;
    const int s0 = p.pbc[0] ? (int)floor((double)v0 / p.nb[0]) : 0;
    const int r0 = v0 - s0 * p.nb[0];
    for (int v1 = b[1] - p.D[1]; v1 <= b[1] + p.D[1]; ++v1) {
      if (!p.pbc[1] && (v1 < 0 || v1 >= p.nb[1])) continue;
      const int s1 = p.pbc[1] ? (int)floor((double)v1 / p.nb[1]) : 0;
      const int r1 = v1 - s1 * p.nb[1];
      for (int v2 = b[2] - p.D[2]; v2 <= b[2] + p.D[2]; ++v2) {
        if (!p.pbc[2] && (v2 < 0 || v2 >= p.nb[2])) continue;
        const int s2 = p.pbc[2] ? (int)floor((double)v2 / p.nb[2]) : 0;
        const int r2 = v2 - s2 * p.nb[2];
        const int bb = (r0 * p.nb[1] + r1) * p.nb[2] + r2;
        const int64_t q0 = head[bb], q1 = head[bb + 1];
        for (int64_t q = q0; q < q1; q += 64) {  // wave-uniform trip count
          bool ok = false;
          int64_t j = 0;
          int S[3] = {0, 0, 0};
          if (q + lane < q1) {
            j = order[q + lane];
            const double f[3] = {w[3 * j] + s0, w[3 * j + 1] + s1, w[3 * j + 2] + s2};
            double d2 = 0.0;
            for (int k = 0; k < 3; ++k) {
              const double xk = f[0] * p.cell[k] + f[1] * p.cell[3 + k] + f[2] * p.cell[6 + k];
              d2 += (xk - xi[k]) * (xk - xi[k]);
            }
            S[0] = s0 - off[3 * j] + oi[0];
            S[1] = s1 - off[3 * j + 1] + oi[1];
            S[2] = s2 - off[3 * j + 2] + oi[2];
            ok = d2 < p.c2 && !(j == i && S[0] == 0 && S[1] == 0 && S[2] == 0);
          }
          hit(ok, j, S);
        }
      }
    }
  }
}

// One wave per receiver: counts[i] = pairs of i; *status = 1 if any receiver exceeds the
// per-receiver capacity of the fill kernel or a shift does not fit the packed key.
__global__ void __launch_bounds__(256) nl_count_kernel(NLPlan p, const double* __restrict__ w,
                                                       const int32_t* __restrict__ off,
                                                       const int64_t* __restrict__ head,
                                                       const int32_t* __restrict__ order, int32_t* __restrict__ counts,
                                                       int32_t* __restrict__ status) {
  const int lane = threadIdx.x & 63;
  const int64_t i = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (i >= p.n) return;
  int cnt = 0;
  bool bad = false;
  nl_visit(p, i, w, off, head, order, lane, [&](bool ok, int64_t, const int* S) {
    cnt += __popcll(__ballot(ok));
    if (ok)
      for (int k = 0; k < 3; ++k) bad |= S[k] <= -kNLShiftBias || S[k] >= kNLShiftBias;
  });
  bad = __any(bad) || cnt > kNLMaxPerAtom;
  if (lane == 0) {
    counts[i] = cnt;
    if (bad) atomicOr(status, 1);
  }
}

// One 64-thread workgroup per receiver: collect the (j, S) keys in LDS, sort, write.
__global__ void __launch_bounds__(64) nl_fill_kernel(NLPlan p, const double* __restrict__ w,
                                                     const int32_t* __restrict__ off, const int64_t* __restrict__ head,
                                                     const int32_t* __restrict__ order,
                                                     const int64_t* __restrict__ rowptr, int64_t* __restrict__ out_i,
                                                     int64_t* __restrict__ out_j, int32_t* __restrict__ out_shift) {
  __shared__ uint64_t keys[kNLMaxPerAtom];
  const int lane = threadIdx.x;
  const int64_t i = blockIdx.x;
  const int64_t start = rowptr[i];
  const int cnt = (int)(rowptr[i + 1] - start);
  int fillc = 0;
  nl_visit(p, i, w, off, head, order, lane, [&](bool ok, int64_t j, const int* S) {
    const uint64_t m = __ballot(ok);
    if (ok) {
      const int slot = fillc + __popcll(m & ((1ull << lane) - 1ull));
      keys[slot] = ((uint64_t)j << 32) | ((uint64_t)(S[0] + kNLShiftBias) << 20) |
                   ((uint64_t)(S[1] + kNLShiftBias) << 10) | (uint64_t)(S[2] + kNLShiftBias);
    }
    fillc += __popcll(m);
  });
  int P = 1;
  while (P < cnt) P <<= 1;
  for (int t = cnt + lane; t < P; t += 64) keys[t] = ~0ull;
  __syncthreads();
  for (int k = 2; k <= P; k <<= 1)
    for (int jj = k >> 1; jj > 0; jj >>= 1) {
      for (int t = lane; t < P; t += 64) {
        const int u = t ^ jj;
        if (u > t) {
          const uint64_t a = keys[t], b = keys[u];
          const bool up = (t & k) == 0;
          if ((a > b) == up) {
            keys[t] = b;
            keys[u] = a;
          }
        }
      }
      __syncthreads();
    }
  for (int t = lane; t < cnt; t += 64) {
    const uint64_t key = keys[t];
    out_i[start + t] = i;
    out_j[start + t] = (int64_t)(key >> 32);
    out_shift[3 * (start + t)] = (int32_t)((key >> 20) & 1023u) - kNLShiftBias;
    out_shift[3 * (start + t) + 1] = (int32_t)((key >> 10) & 1023u) - kNLShiftBias;
    out_shift[3 * (start + t) + 2] = (int32_t)(key & 1023u) - kNLShiftBias;
  }
}

static void nl_cross(const double* a, const double* b, double* c) {
  c[0] = a[1] * b[2] - a[2] * b[1];
  c[1] = a[2] * b[0] - a[0] * b[2];
  c[2] = a[0] * b[1] - a[1] * b[0];
}

// Workspace layout (bytes, 256-aligned pieces); the bin count is capped at 4n + 64.
struct NLWorkspace {
  double* w;
  double* range;
  int32_t* off;
  int32_t* bin;
  int32_t* order;
  int32_t* hist;
  int32_t* counts;
  int32_t* status;
  int64_t* head;
  int64_t* rowptr;
};

static int64_t nl_max_bins(int64_t n) { return 4 * n + 64; }

static int64_t nl_layout(int64_t n, char* base, NLWorkspace* ws) {
  int64_t o = 0;
  auto take = [&](int64_t bytes) {
    const int64_t at = o;
    o += (bytes + 255) / 256 * 256;
    return base ? base + at : nullptr;
  };
  const int64_t nb = nl_max_bins(n);
  NLWorkspace t{};
  t.w = reinterpret_cast<double*>(take(3 * n * sizeof(double)));
  t.range = reinterpret_cast<double*>(take(6 * sizeof(double)));
  t.off = reinterpret_cast<int32_t*>(take(3 * n * sizeof(int32_t)));
  t.bin = reinterpret_cast<int32_t*>(take(n * sizeof(int32_t)));
  t.order = reinterpret_cast<int32_t*>(take(n * sizeof(int32_t)));
  t.hist = reinterpret_cast<int32_t*>(take((nb + 1) * sizeof(int32_t)));
  t.counts = reinterpret_cast<int32_t*>(take((n + 1) * sizeof(int32_t)));
  t.status = reinterpret_cast<int32_t*>(take(sizeof(int32_t)));
  t.head = reinterpret_cast<int64_t*>(take((nb + 1) * sizeof(int64_t)));
  t.rowptr = reinterpret_cast<int64_t*>(take((n + 1) * sizeof(int64_t)));
  if (ws) *ws = t;
  return o;
}

}  // namespace fc

using namespace fc;

extern "C" int64_t fc_neighbor_list_device_workspace(int64_t n) {
  if (n < 0) return -FC_ERR_SHAPE;
  return nl_layout(n, nullptr, nullptr);
}

namespace fc {

// The list from positions in HBM, with its working arrays laid out from `workspace` (at least
// nl_layout(n) bytes, already checked by the caller). Returns the pair count or -fc_status.
static int64_t nl_build(int64_t n, const double* pos, const double* cell, const int32_t* pbc, double cutoff,
                        int64_t capacity, int64_t* out_i, int64_t* out_j, int32_t* out_shift, void* workspace,
                        hipStream_t s) {
  NLWorkspace ws;
  nl_layout(n, reinterpret_cast<char*>(workspace), &ws);

  NLPlan p{};
  p.n = n;
  for (int k = 0; k < 9; ++k) p.cell[k] = cell[k];
  for (int k = 0; k < 3; ++k) p.pbc[k] = pbc[k] ? 1 : 0;
  const double* m = cell;
  const double det = m[0] * (m[4] * m[8] - m[5] * m[7]) - m[1] * (m[3] * m[8] - m[5] * m[6]) +
                     m[2] * (m[3] * m[7] - m[4] * m[6]);
  if (std::fabs(det) < 1e-300) return -FC_ERR_BAD_DESC;
  {  // the host list's inverse, operation for operation
    const double id = 1.0 / det;
    p.inv[0] = (m[4] * m[8] - m[5] * m[7]) * id;
    p.inv[1] = (m[2] * m[7] - m[1] * m[8]) * id;
    p.inv[2] = (m[1] * m[5] - m[2] * m[4]) * id;
    p.inv[3] = (m[5] * m[6] - m[3] * m[8]) * id;
    p.inv[4] = (m[0] * m[8] - m[2] * m[6]) * id;
    p.inv[5] = (m[2] * m[3] - m[0] * m[5]) * id;
    p.inv[6] = (m[3] * m[7] - m[4] * m[6]) * id;
    p.inv[7] = (m[1] * m[6] - m[0] * m[7]) * id;
    p.inv[8] = (m[0] * m[4] - m[1] * m[3]) * id;
  }
  double reach[3];
  {
    double vv[3];
    nl_cross(cell + 3, cell + 6, vv);
    const double vol = std::fabs(cell[0] * vv[0] + cell[1] * vv[1] + cell[2] * vv[2]);
    for (int k = 0; k < 3; ++k) {
      double c[3];
      nl_cross(cell + 3 * ((k + 1) % 3), cell + 3 * ((k + 2) % 3), c);
      reach[k] = cutoff / (vol / std::sqrt(c[0] * c[0] + c[1] * c[1] + c[2] * c[2]));
    }
  }
  p.c2 = cutoff * cutoff;
  const int bs = 256;
  const unsigned g_atoms = (unsigned)((n + bs - 1) / bs);
  hipLaunchKernelGGL(nl_wrap_kernel, dim3(g_atoms), dim3(bs), 0, s, p, pos, ws.w, ws.off);
  if (hipGetLastError() != hipSuccess) return -FC_ERR_LAUNCH;
  double lo[3] = {0, 0, 0}, hi[3] = {1, 1, 1};
  if (!(p.pbc[0] && p.pbc[1] && p.pbc[2])) {
    double r[6];
    hipLaunchKernelGGL(nl_range_kernel, dim3(1), dim3(256), 0, s, n, ws.w, ws.range);
    if (hipGetLastError() != hipSuccess) return -FC_ERR_LAUNCH;
    if (hipMemcpyAsync(r, ws.range, sizeof(r), hipMemcpyDeviceToHost, s) != hipSuccess ||
        hipStreamSynchronize(s) != hipSuccess)
      return -FC_ERR_LAUNCH;
    for (int k = 0; k < 3; ++k)
      if (!p.pbc[k]) { lo[k] = r[k]; hi[k] = r[3 + k]; }
  }
  // Bins of fractional width >= reach (1e-6 margin: rounding of the coordinates never puts
  // two atoms closer than the cutoff two bins apart). Periodic axes: D = ceil(reach / width)
  // neighbouring bins each way (several images when the cell is thinner than the cutoff).
  for (int k = 0; k < 3; ++k) {
    const double span = hi[k] - lo[k];
    int nbk = (int)std::floor(span / (reach[k] * (1.0 + 1e-6)));
    nbk = nbk < 1 ? 1 : (nbk > 512 ? 512 : nbk);
    p.nb[k] = nbk;
    p.base[k] = lo[k];
    p.width[k] = span > 0 ? span / nbk : 1.0;
    p.D[k] = p.pbc[k] ? (int)std::ceil(reach[k] / p.width[k]) : 1;
  }
  while ((int64_t)p.nb[0] * p.nb[1] * p.nb[2] > nl_max_bins(n)) {  // coarser bins for sparse systems
    int k = 0;
    for (int q = 1; q < 3; ++q)
      if (p.nb[q] > p.nb[k]) k = q;
    p.nb[k] = (p.nb[k] + 1) / 2;
    p.width[k] = (hi[k] - lo[k]) > 0 ? (hi[k] - lo[k]) / p.nb[k] : 1.0;
    p.D[k] = p.pbc[k] ? (int)std::ceil(reach[k] / p.width[k]) : 1;
  }
  const int64_t nbins = (int64_t)p.nb[0] * p.nb[1] * p.nb[2];
  hipLaunchKernelGGL(nl_fill_int_kernel, dim3((unsigned)((nbins + 1 + bs - 1) / bs)), dim3(bs), 0, s, nbins + 1,
                     ws.hist, 0);
  hipLaunchKernelGGL(nl_fill_int_kernel, dim3(1), dim3(bs), 0, s, (int64_t)1, ws.status, 0);
  hipLaunchKernelGGL(nl_bin_kernel, dim3(g_atoms), dim3(bs), 0, s, p, ws.w, ws.bin, ws.hist);
  hipLaunchKernelGGL(nl_scan_kernel, dim3(1), dim3(1024), 0, s, nbins, ws.hist, ws.head);
  hipLaunchKernelGGL(nl_fill_int_kernel, dim3((unsigned)((nbins + bs - 1) / bs)), dim3(bs), 0, s, nbins, ws.hist, 0);
  hipLaunchKernelGGL(nl_scatter_kernel, dim3(g_atoms), dim3(bs), 0, s, n, ws.bin, ws.head, ws.hist, ws.order);
  hipLaunchKernelGGL(nl_count_kernel, dim3((unsigned)((n + 3) / 4)), dim3(256), 0, s, p, ws.w, ws.off, ws.head,
                     ws.order, ws.counts, ws.status);
  hipLaunchKernelGGL(nl_scan_kernel, dim3(1), dim3(1024), 0, s, n, ws.counts, ws.rowptr);
  if (hipGetLastError() != hipSuccess) return -FC_ERR_LAUNCH;
  int64_t total = 0;
  int32_t status = 0;
  if (hipMemcpyAsync(&total, ws.rowptr + n, sizeof(total), hipMemcpyDeviceToHost, s) != hipSuccess ||
      hipMemcpyAsync(&status, ws.status, sizeof(status), hipMemcpyDeviceToHost, s) != hipSuccess ||
      hipStreamSynchronize(s) != hipSuccess)
    return -FC_ERR_LAUNCH;
  if (status) return -FC_ERR_SHAPE;  // > 1024 pairs for one atom, or |S| >= 512
  if (total > capacity || total == 0) return total;
  if (!out_i || !out_j || !out_shift) return -FC_ERR_NULL;
  hipLaunchKernelGGL(nl_fill_kernel, dim3((unsigned)n), dim3(64), 0, s, p, ws.w, ws.off, ws.head, ws.order,
                     ws.rowptr, out_i, out_j, out_shift);
  if (hipGetLastError() != hipSuccess) return -FC_ERR_LAUNCH;
  return total;
}

static int64_t nl_check_args(int64_t n, const double* pos, const double* cell, const int32_t* pbc, double cutoff) {
  if (n < 0 || !(cutoff > 0.0) || !cell || !pbc) return -FC_ERR_BAD_DESC;
  if (n > 0x7fffffff || (n > 0 && !pos)) return -FC_ERR_SHAPE;
  return 0;
}

// Working memory of the allocation-free entry point: one copy of this array per device (a module
// global), held until the process ends. Host code never passes `scratch` itself to a kernel or a
// copy (in host code the name is only a stand-in for the symbol): it uses the device address that
// hipGetSymbolAddress returns for the current device, kept in g_scratch_ptr.
constexpr int64_t kNLScratchBytes = int64_t(64) << 20;
static __device__ __align__(256) char scratch[kNLScratchBytes];

constexpr int kMaxDevices = 64;
static std::mutex g_scratch_mu;
static void* g_scratch_ptr[kMaxDevices];

// The current device's address of `scratch` (looked up once per device, with that device current).
static int nl_scratch_address(void** out) {
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return FC_ERR_LAUNCH;
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void* p = nullptr;
    if (hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)) != hipSuccess || !p) return FC_ERR_LAUNCH;
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return FC_OK;
}

}  // namespace fc

extern "C" int64_t fc_neighbor_list_device(int64_t n, const double* pos, const double* cell, const int32_t* pbc,
                                           double cutoff, int64_t capacity, int64_t* out_i, int64_t* out_j,
                                           int32_t* out_shift, void* workspace, int64_t workspace_bytes,
                                           void* stream) {
  const int64_t bad = nl_check_args(n, pos, cell, pbc, cutoff);
  if (bad) return bad;
  if (n == 0) return 0;
  if (!workspace || workspace_bytes < nl_layout(n, nullptr, nullptr)) return -FC_ERR_WORKSPACE;
  return nl_build(n, pos, cell, pbc, cutoff, capacity, out_i, out_j, out_shift, workspace, (hipStream_t)stream);
}

extern "C" int64_t fc_neighbor_list_device_noalloc_max_atoms(void) {
  int64_t lo = 0, hi = int64_t(1) << 31;  // largest n whose working arrays fit the scratch array
  while (lo < hi) {
    const int64_t mid = (lo + hi + 1) / 2;
    if (nl_layout(mid, nullptr, nullptr) <= kNLScratchBytes) lo = mid; else hi = mid - 1;
  }
  return lo;
}

extern "C" int64_t fc_neighbor_list_device_noalloc(int64_t n, const double* pos, const double* cell,
                                                   const int32_t* pbc, double cutoff, int64_t capacity,
                                                   int64_t* out_i, int64_t* out_j, int32_t* out_shift,
                                                   void* stream) {
  const int64_t bad = nl_check_args(n, pos, cell, pbc, cutoff);
  if (bad) return bad;
  if (n == 0) return 0;
  if (nl_layout(n, nullptr, nullptr) > kNLScratchBytes) return -FC_ERR_SCRATCH_LIMIT;
  void* base = nullptr;
  const int st = nl_scratch_address(&base);
  if (st != FC_OK) return -st;
  return nl_build(n, pos, cell, pbc, cutoff, capacity, out_i, out_j, out_shift, base, (hipStream_t)stream);
}
