// Irreducible Cartesian tensor product kernels (forward and vector-Jacobian product).
//
// One template covers the two modes of TensorProduct.forward:
//   CONV = true  : out[i] = sum_{e in in(i)} sum_p w[e,p,:] (x) contract_p(in1[idx_j[e]], in2[e])
//                  over a receiver-sorted CSR (rowptr), as in the reference's
//                  tp_fwd_csr_kernel (src/flashcart/o3/_codegen_tensor_product.py:3245-3311);
//   CONV = false : independent rows (reference tp_fwd_kernel, :2062-2140).
// Work decomposition (gfx950, wave64): one workgroup per output row (node), one lane
// per feature channel; per-path accumulators live in VGPRs and every output element
// is stored exactly once, so the aggregation needs no atomics. The edge loop is
// uniform across the workgroup: with a single in2 channel (BC2, the interaction
// layers) the edge attributes are wave-uniform scalar loads, and the per-edge
// coupling matrices A_p[a][b] = sum_c B_p[a,b,c] y_c are formed once per edge. The
// operands of the next edge are prefetched into registers while the current edge
// is contracted, so the HBM latency of the gathered rows is hidden at 2-3 waves/SIMD.
#pragma once
#include "fc_common.h"
#include "fc_tp_paths.h"  // generated for the build's rank limit

namespace fc {

struct TPArgs {
  const float* in1;
  const float* in2;
  const float* w;
  const int32_t* idx_j;    // conv: sender per edge
  const int32_t* rowptr;   // conv: receiver CSR, n_rows + 1 entries
  const int32_t* wslot;    // conv, optional: edge e reads weight row wslot[e] / 2 (the two edges of a
                           // pair share a row); its weight gradient stays at row e
  const float* grad_out;   // bwd only
  float* out;              // fwd output
  float* grad_in1;         // bwd: rows mode -> grad wrt in1 rows; conv mode -> per-edge messages
  float* grad_in2;
  float* grad_w;           // per-item weight gradient (item = edge or row)
  int64_t n_rows;
  int64_t n_edges;         // conv: edges of the graph (launch shape only)
  int32_t F1, F2, C;       // in1 / in2 / output features (1 broadcasts)
  int32_t shared_w, reduced;
  float alpha;             // output scale (fwd) / its transpose (bwd)
  const float* alpha_div;  // optional device scalar s: the scale is alpha / s
  // rows backward only: gradients added to grad_in1 / grad_in2 (leading res*_comps
  // components of each row, row width res*_comps * C; may alias the gradient)
  const float* res1;
  const float* res2;
  int32_t res1_comps, res2_comps;
  // convolution backward in sender order (tp_bwd_send_kernel): receiver of each edge and the
  // sender CSR; n_rows counts senders; grad_in1 receives the input gradient rows directly
  const int32_t* idx_i;
  const int32_t* sperm;
  const int32_t* sptr;
  int32_t sender_major;
};

// s_waitcnt immediate (gfx9 encoding) that waits until at most vm vector-memory operations of the
// wave are outstanding (no LDS/scalar or export wait). The empty asm before it keeps the compiler
// from moving memory accesses across the wait, so the operations counted are the ones in program
// order before it.
#define FC_VMCNT_IMM(vm) (((vm) & 0xF) | ((((vm) >> 4) & 3) << 14) | (0x7 << 4) | (0xF << 8))
__device__ __forceinline__ void vm_wait_barrier() { asm volatile("" ::: "memory"); }

// Zeros read in place of the weight row of an edge that a pairing left without a partner (slot
// -1): the backward kernels then issue the same loads on every path and need no select on the
// loaded values (which the compiler would place where it waits for them). Device globals start
// zeroed and nothing writes this one.
constexpr int kZeroRowFloats = 96 * 256;
__device__ float zero_weight_row[kZeroRowFloats];

template <int L1, int L2, int LO, bool SYM>
struct TPConfig {
  using PL = PathList<L1, L2, LO, SYM>;
  static constexpr int NP = PL::NP;
  static constexpr int D1 = ncomp(L1);
  static constexpr int D2 = ncomp(L2);
  static constexpr int NOUT = PL::NOUT;
  static constexpr int NOUT_RED = PL::NOUT_RED;
};

// Output scale: alpha, divided by the device scalar *alpha_div when one is given (read once per
// workgroup; the divisor's storage is the caller's, e.g. a module buffer).
__device__ __forceinline__ float scale_of(const TPArgs& g) {
  return g.alpha_div ? g.alpha / *g.alpha_div : g.alpha;
}

// Weight row of edge e (the pair's row when edges share weights); negative for an edge that a
// pairing left without a partner (slot -1), whose weights then count as zero.
__device__ __forceinline__ int64_t weight_row(const TPArgs& g, int64_t e) {
  return g.wslot ? (int64_t)(g.wslot[e] >> 1) : e;
}

// Operands of one edge (or row) for one lane.
template <int D1, int D2, int NP>
struct EdgeOps {
  float x[D1], y[D2], w[NP];
};

// GIVEN: the caller passes the edge's sender j_given and weight row wrow_given (no index loads here).
template <int D1, int D2, int NP, bool CONV, bool BC2, bool LOADY = true, bool GIVEN = false>
__device__ __forceinline__ void load_edge(const TPArgs& g, int64_t e, int f1, int f2, int fw, bool active,
                                          EdgeOps<D1, D2, NP>& o, int64_t j_given = 0, int64_t wrow_given = 0) {
  const int64_t j = GIVEN ? j_given : CONV ? (int64_t)g.idx_j[e] : e;
  const int64_t s1 = (int64_t)D1 * g.F1;
#pragma unroll
  for (int u = 0; u < D1; ++u) o.x[u] = active ? g.in1[j * s1 + u * g.F1 + f1] : 0.f;
  if constexpr (!LOADY) {
  } else if constexpr (BC2) {
#pragma unroll
    for (int u = 0; u < D2; ++u) o.y[u] = g.in2[e * D2 + u];
  } else {
    const int64_t s2 = (int64_t)D2 * g.F2;
#pragma unroll
    for (int u = 0; u < D2; ++u) o.y[u] = active ? g.in2[e * s2 + u * g.F2 + f2] : 0.f;
  }
  const int64_t wrow = g.shared_w ? 0 : GIVEN ? wrow_given : weight_row(g, e);
  if (wrow < 0) {  // uniform over the workgroup
#pragma unroll
    for (int i = 0; i < NP; ++i) o.w[i] = 0.f;
    return;
  }
  const float* wr = g.w + wrow * (int64_t)NP * g.C;
#pragma unroll
  for (int i = 0; i < NP; ++i) o.w[i] = active ? wr[i * g.C + fw] : 0.f;
}

// Per-edge coupling matrices in LDS. With a single in2 channel (BC2) the matrices
// A_p(y_e) are the same for every channel of an edge, so forming them in each lane
// repeats the work 64 times per wave. Instead, lanes 0..n-1 of each wave form them for
// a chunk of n edges (each wave a contiguous share of the paths) into LDS, and the
// edge loop reads them back as broadcast LDS loads. Each path's block is padded to a
// multiple of 4 floats (16-byte aligned).
template <int L1, int L2, int LO, bool SYM>
struct AmatLayout {
  using PL = PathList<L1, L2, LO, SYM>;
  template <int I>
  static constexpr int size() {
    constexpr PathDesc P = PL::at(I);
    return (TPPath<P.r1, P.r2, P.lo>::NA + 3) & ~3;
  }
  template <int I>
  static constexpr int off() {
    if constexpr (I == 0) return 0;
    else return off<I - 1>() + size<I - 1>();
  }
  static constexpr int total = off<PL::NP>();
  // edges per chunk: two chunk buffers within 32 KiB
  static constexpr int chunk = total * 16 * 2 * 4 <= 32768 ? 16 : (32768 / (total * 2 * 4) > 0 ? 32768 / (total * 2 * 4) : 1);
};

// Lanes 0..n-1 of each wave form the coupling matrices of edge c0 + lane for this
// wave's share of the paths.
template <int L1, int L2, int LO, bool SYM>
__device__ __forceinline__ void fill_amat(const float* __restrict__ in2, int64_t c0, int n, float* a, int lane,
                                          int wave, int nw) {
  using PL = PathList<L1, L2, LO, SYM>;
  using AL = AmatLayout<L1, L2, LO, SYM>;
  constexpr int D2 = ncomp(L2);
  if (lane >= n) return;
  float y[D2];
#pragma unroll
  for (int u = 0; u < D2; ++u) y[u] = in2[(c0 + lane) * D2 + u];
  float* ae = a + lane * AL::total;
  const int p0 = wave * PL::NP / nw, p1 = (wave + 1) * PL::NP / nw;
  static_for<PL::NP>([&](auto ic) {
    constexpr int i = decltype(ic)::value;
    if (i >= p0 && i < p1) {
      constexpr PathDesc P = PL::at(i);
      TPPath<P.r1, P.r2, P.lo>::amat(y + P.r2 * P.r2, ae + AL::template off<i>());
    }
  });
}

// EG > 1 (convolution with C = 32 or 64 only): EG groups of C lanes share a receiver (block C * EG
// threads), group g taking the edges e0 + g, e0 + g + EG, ...; the groups' partial sums are added in
// LDS in group order (so results are reproducible run to run) and stored by group 0. This gives a
// graph with few receivers and few channels enough waves to hide the gather latency.
template <int L1, int L2, int LO, bool SYM, bool CONV, bool BC2, int EG = 1>
__global__ void __launch_bounds__(256) tp_fwd_kernel(TPArgs g) {
  // The forward keeps the per-lane coupling matrices: it is bound by the gathered
  // operand stream, and staging the matrices in LDS (as the backward does) measured
  // slower here (chunk barriers and broadcast LDS reads on the critical path).
  using CF = TPConfig<L1, L2, LO, SYM>;
  using PL = typename CF::PL;
  constexpr int D1 = CF::D1, D2 = CF::D2, NOUT = CF::NOUT, NP = CF::NP;
  static_assert(EG == 1 || CONV, "edge groups split a receiver's edges");
  extern __shared__ float part_lds[];  // EG > 1: (EG - 1) x NOUT x C partial sums
  const int64_t row = CONV ? xcd_row(g.n_rows) : (int64_t)blockIdx.x;
  const int C = g.C;
  const int grp = EG == 1 ? 0 : (int)threadIdx.x / C;
  const int f = EG == 1 ? (int)threadIdx.x : (int)threadIdx.x % C;
  if (row >= g.n_rows) return;  // uniform over the workgroup
  if (EG == 1 && f >= C) return;
  const int f1 = g.F1 == 1 ? 0 : f;
  const int f2 = g.F2 == 1 ? 0 : f;

  float acc[NOUT];
#pragma unroll
  for (int k = 0; k < NOUT; ++k) acc[k] = 0.f;

  int64_t e0 = row, e1 = row + 1;
  if constexpr (CONV) { e0 = g.rowptr[row] + grp; e1 = g.rowptr[row + 1]; }
  EdgeOps<D1, D2, NP> cur, nxt;
  // With edge groups an edge's index differs between groups, so idx_j[e] and its pair slot are
  // vector loads that the row loads would wait for one edge at a time. Instead the group's lanes
  // stage the senders and weight rows of its next C edges in LDS (one load each, C edges per wait)
  // and the loop reads them from there.
  __shared__ int32_t ix_lds[CONV && EG > 1 ? 2 * EG * 64 : 1];
  auto stage_idx = [&](int64_t k0) {  // the group's edges k0 .. k0 + C - 1
    if constexpr (CONV && EG > 1) {
      const int64_t e = e0 + (k0 + f) * EG;
      if (e < e1) {
        ix_lds[grp * 128 + f] = g.idx_j[e];
        ix_lds[grp * 128 + 64 + f] = g.shared_w ? 0 : (int32_t)weight_row(g, e);
      }
    }
  };
  auto load_k = [&](int64_t k, EdgeOps<D1, D2, NP>& o) {  // the group's edge k
    const int64_t e = e0 + k * EG;
    if constexpr (CONV && EG > 1) {
      const int s = (int)(k & (C - 1));  // C is 32 or 64 with edge groups
      load_edge<D1, D2, NP, CONV, BC2, true, true>(g, e, f1, f2, f, true, o, ix_lds[grp * 128 + s],
                                                   ix_lds[grp * 128 + 64 + s]);
    } else {
      load_edge<D1, D2, NP, CONV, BC2>(g, e, f1, f2, f, true, o);
    }
  };
  stage_idx(0);
  if (e0 < e1) load_k(0, nxt);
  int64_t k = 0;
  for (int64_t e = e0; e < e1; e += EG, ++k) {
    cur = nxt;
    if (e + EG < e1) {
      if (((k + 1) & (C - 1)) == 0) stage_idx(k + 1);
      load_k(k + 1, nxt);
    }
    static_for<NP>([&](auto ic) {
      constexpr int i = decltype(ic)::value;
      constexpr PathDesc P = PL::at(i);
      using T = TPPath<P.r1, P.r2, P.lo>;
      float A[T::NA], t[T::NO];
      T::amat(cur.y + P.r2 * P.r2, A);
      T::apply(A, cur.x + P.r1 * P.r1, t);
#pragma unroll
      for (int a = 0; a < T::NO; ++a) acc[PL::out_index(i, a)] = fmaf(cur.w[i], t[a], acc[PL::out_index(i, a)]);
    });
  }
  if constexpr (EG > 1) {
    if (grp > 0) {
#pragma unroll
      for (int k = 0; k < NOUT; ++k) part_lds[((grp - 1) * NOUT + k) * C + f] = acc[k];
    }
    __syncthreads();
    if (grp > 0) return;
#pragma unroll
    for (int q = 1; q < EG; ++q)
#pragma unroll
      for (int k = 0; k < NOUT; ++k) acc[k] += part_lds[((q - 1) * NOUT + k) * C + f];
  }
  if (!g.reduced) {
    float* o = g.out + row * (int64_t)NOUT * C + f;
    const float alpha = scale_of(g);
#pragma unroll
    for (int k = 0; k < NOUT; ++k) o[(int64_t)k * C] = alpha * acc[k];
  } else {
    constexpr int NR = CF::NOUT_RED;
    float red[NR];
#pragma unroll
    for (int k = 0; k < NR; ++k) red[k] = 0.f;
    static_for<NP>([&](auto ic) {
      constexpr int i = decltype(ic)::value;
      constexpr PathDesc P = PL::at(i);
#pragma unroll
      for (int a = 0; a < 2 * P.lo + 1; ++a) red[PL::out_index_red(i, a)] += acc[PL::out_index(i, a)];
    });
    float* o = g.out + row * (int64_t)NR * C + f;
    const float alpha = scale_of(g);
#pragma unroll
    for (int k = 0; k < NR; ++k) o[(int64_t)k * C] = alpha * red[k];
  }
}

__host__ __device__ constexpr int log2_exact(int n) { return n <= 1 ? 0 : 1 + log2_exact(n >> 1); }

__host__ __device__ constexpr int pow2_at_least(int n) {
  int p = 1;
  while (p < n) p <<= 1;
  return p;
}

// Sum N per-lane values (N a power of two <= 64) over the 64 lanes of a wave with a
// halving butterfly: every exchange step keeps half of the values (N-1 + 6-log2 N
// shuffles instead of 6 N). Afterwards every lane of group lane >> (6 - log2 N) == v
// holds the total of value v.
// W = 32 reduces each half of the wave on its own: afterwards lane group (lane & 31) >> (5 - log2 N)
// == v of each half holds that half's total of value v.
template <int N, int W = 64>
__device__ __forceinline__ float wave_reduce_halving(float (&v)[N], int lane) {
  constexpr int LOGN = log2_exact(N);
  static_assert((1 << LOGN) == N, "N must be a power of two");
  static_assert((W == 32 || W == 64) && N <= W, "lane groups of 32 or 64");
  static_for<LOGN>([&](auto sc) {
    constexpr int s = decltype(sc)::value;
    constexpr int half = N >> (s + 1);
    const int o = (W / 2) >> s;
    const bool lower = (lane & o) == 0;
#pragma unroll
    for (int j = 0; j < half; ++j) {
      const float mine = lower ? v[j] : v[j + half];
      const float send = lower ? v[j + half] : v[j];
      v[j] = mine + __shfl_xor(send, o, 64);
    }
  });
  float r = v[0];
#pragma unroll
  for (int o = (W / 2) >> LOGN; o > 0; o >>= 1) r += __shfl_xor(r, o, 64);
  return r;
}

// Backward (vector-Jacobian product) of tp_fwd_kernel. With v_p = A_p^T go_p (one
// transposed product shared by the weight and in1 gradients):
//   grad_w[item, p, f]  = sum_a go[a,p,f] (A_p x)[a] = sum_b v_p[b] x[b]
//   gx[b]              += w[p,f] v_p[b]                      (conv: per-edge message)
//   gy[c]              += sum_{a,b} B_p[a,b,c] go[a,p,f] (w[p,f] x[b])
// Channel-broadcast operands (F == 1) get their gradient summed over channels: a
// halving butterfly in each wave, then a cross-wave sum through LDS in a fixed
// order, so the result is deterministic. Edges are processed in chunks of
// bwd_chunk<...>() edges (the LDS coupling-matrix chunk in BC2 convolutions).
template <int L1, int L2, int LO, bool SYM, bool CONV, bool BC2>
__host__ __device__ constexpr int bwd_chunk() {
  return (CONV && BC2) ? AmatLayout<L1, L2, LO, SYM>::chunk : 16;
}

template <int L1, int L2, int LO, bool SYM, bool CONV, bool BC2>
__global__ void __launch_bounds__(256, 2) tp_bwd_kernel(TPArgs g) {
  using CF = TPConfig<L1, L2, LO, SYM>;
  using PL = typename CF::PL;
  using AL = AmatLayout<L1, L2, LO, SYM>;
  constexpr int D1 = CF::D1, D2 = CF::D2, NOUT = CF::NOUT, NP = CF::NP;
  constexpr int R1 = pow2_at_least(D1), R2 = pow2_at_least(D2);
  constexpr int SH1 = 6 - log2_exact(R1), SH2 = 6 - log2_exact(R2);
  constexpr bool LDSA = CONV && BC2;
  constexpr int CH = bwd_chunk<L1, L2, LO, SYM, CONV, BC2>();
  extern __shared__ float red_lds[];  // [CH][waves][D1 + D2], only when reducing over channels
  __shared__ __align__(16) float a_lds[LDSA ? 2 * CH * AL::total : 1];

  const int64_t row = CONV ? xcd_row(g.n_rows) : (int64_t)blockIdx.x;
  if (row >= g.n_rows) return;
  const int f = threadIdx.x;
  const int C = g.C;
  const bool active = f < C;
  const int fa = active ? f : 0;
  const int f1 = g.F1 == 1 ? 0 : fa;
  const int f2 = g.F2 == 1 ? 0 : fa;
  const int wave = f >> 6, lane = f & 63, nw = blockDim.x >> 6;
  const int64_t s1 = (int64_t)D1 * g.F1, sw = (int64_t)NP * C;
  const bool need1 = g.grad_in1 != nullptr, need2 = g.grad_in2 != nullptr, needw = g.grad_w != nullptr;
  // BC2 implies F2 == 1, so F1 == C there: in1 is never channel-reduced (compile-time,
  // which keeps the unused butterfly registers of gx out of the kernel).
  const bool red1 = !BC2 && need1 && g.F1 == 1 && C > 1, red2 = need2 && g.F2 == 1 && C > 1;
  const float alpha = scale_of(g);

  float go[NOUT];
  if (!g.reduced) {
#pragma unroll
    for (int k = 0; k < NOUT; ++k)
      go[k] = active ? alpha * g.grad_out[row * (int64_t)NOUT * C + (int64_t)k * C + fa] : 0.f;
  } else {
    constexpr int NR = CF::NOUT_RED;
    float gr[NR];
#pragma unroll
    for (int k = 0; k < NR; ++k)
      gr[k] = active ? alpha * g.grad_out[row * (int64_t)NR * C + (int64_t)k * C + fa] : 0.f;
    static_for<NP>([&](auto ic) {
      constexpr int i = decltype(ic)::value;
      constexpr PathDesc P = PL::at(i);
#pragma unroll
      for (int a = 0; a < 2 * P.lo + 1; ++a) go[PL::out_index(i, a)] = gr[PL::out_index_red(i, a)];
    });
  }

  int64_t e0 = row, e1 = row + 1;
  if constexpr (CONV) { e0 = g.rowptr[row]; e1 = g.rowptr[row + 1]; }
  EdgeOps<D1, D2, NP> cur, nxt;
  if (e0 < e1) {
    load_edge<D1, D2, NP, CONV, BC2, !LDSA>(g, e0, f1, f2, fa, active, nxt);
    if constexpr (LDSA) {
      fill_amat<L1, L2, LO, SYM>(g.in2, e0, e1 - e0 < CH ? (int)(e1 - e0) : CH, a_lds, lane, wave, nw);
      __syncthreads();
    }
  }
  int buf = 0;
  for (int64_t c0 = e0; c0 < e1; c0 += CH) {
    const int64_t c1 = c0 + CH < e1 ? c0 + CH : e1;
    const int n_next = e1 - c1 < CH ? (int)(e1 - c1) : CH;
    const float* ab = a_lds + buf * CH * AL::total;
    for (int64_t e = c0; e < c1; ++e) {
      cur = nxt;
      if (e + 1 < e1) load_edge<D1, D2, NP, CONV, BC2, !LDSA>(g, e + 1, f1, f2, fa, active, nxt);
      const float* ae = ab + (int)(e - c0) * AL::total;
      float gx[R1], gy[R2];
#pragma unroll
      for (int u = 0; u < R1; ++u) gx[u] = 0.f;
#pragma unroll
      for (int u = 0; u < R2; ++u) gy[u] = 0.f;
      static_for<NP>([&](auto ic) {
        constexpr int i = decltype(ic)::value;
        constexpr PathDesc P = PL::at(i);
        using T = TPPath<P.r1, P.r2, P.lo>;
        const float* xp = cur.x + P.r1 * P.r1;
        float gop[T::NO];
#pragma unroll
        for (int a = 0; a < T::NO; ++a) gop[a] = go[PL::out_index(i, a)];
        if (needw || need1) {
          // v = A_p^T go_p serves both: grad_w = <go_p, A_p x> = <v, x>, gx += w_p v
          float v[T::N1];
#pragma unroll
          for (int b = 0; b < T::N1; ++b) v[b] = 0.f;
          if constexpr (LDSA) {
            T::apply_t(ae + AL::template off<i>(), gop, v);
          } else {
            float A[T::NA];
            T::amat(cur.y + P.r2 * P.r2, A);
            T::apply_t(A, gop, v);
          }
          if (needw) {
            float s = 0.f;
#pragma unroll
            for (int b = 0; b < T::N1; ++b) s = fmaf(v[b], xp[b], s);
            if (active) g.grad_w[e * sw + i * C + f] = s;
          }
          if (need1) {
#pragma unroll
            for (int b = 0; b < T::N1; ++b) gx[P.r1 * P.r1 + b] = fmaf(cur.w[i], v[b], gx[P.r1 * P.r1 + b]);
          }
        }
        if (need2) {  // gy += B_p(go_p, w_p x)
          float xw[T::N1];
#pragma unroll
          for (int b = 0; b < T::N1; ++b) xw[b] = cur.w[i] * xp[b];
          T::vjp2(gop, xw, gy + P.r2 * P.r2);
        }
      });
      const int slot = (int)(e - c0);
      if (need1) {
        if (red1) {
          const float s = wave_reduce_halving<R1>(gx, lane);
          const int v = lane >> SH1;
          if ((lane & ((1 << SH1) - 1)) == 0 && v < D1) red_lds[(slot * nw + wave) * (D1 + D2) + v] = s;
        } else if (active) {
#pragma unroll
          for (int u = 0; u < D1; ++u) g.grad_in1[e * s1 + u * g.F1 + f] = gx[u];
        }
      }
      if (need2) {
        if (red2) {
          const float s = wave_reduce_halving<R2>(gy, lane);
          const int v = lane >> SH2;
          if ((lane & ((1 << SH2) - 1)) == 0 && v < D2) red_lds[(slot * nw + wave) * (D1 + D2) + D1 + v] = s;
        } else if (active) {
          const int64_t s2 = (int64_t)D2 * g.F2;
#pragma unroll
          for (int u = 0; u < D2; ++u) g.grad_in2[e * s2 + u * g.F2 + f] = gy[u];
        }
      }
    }
    if (LDSA && n_next > 0) {
      // the other buffer was last read in the previous chunk, before this chunk's barrier;
      // the barrier below (or the reduction's first one) publishes it
      fill_amat<L1, L2, LO, SYM>(g.in2, c1, n_next, a_lds + (buf ^ 1) * CH * AL::total, lane, wave, nw);
    }
    if (red1 || red2) {
      __syncthreads();
      const int n = (int)(c1 - c0);
      for (int k = f; k < n * (D1 + D2); k += blockDim.x) {
        const int slot = k / (D1 + D2), u = k % (D1 + D2);
        float s = 0.f;
        for (int w = 0; w < nw; ++w) s += red_lds[(slot * nw + w) * (D1 + D2) + u];
        const int64_t e = c0 + slot;
        if (u < D1) {
          if (red1) g.grad_in1[e * D1 + u] = s;
        } else if (red2) {
          g.grad_in2[e * D2 + (u - D1)] = s;
        }
      }
      __syncthreads();
    } else if (LDSA && n_next > 0) {
      __syncthreads();
    }
    buf ^= 1;
  }
}

// Backward of the interaction-layer convolution (one in2 channel, unreduced outputs),
// specialised at compile time: C channels (every lane active, operand offsets are
// immediates), the weight and edge-attribute gradients always formed, the per-edge in1
// messages when NEED1. Same arithmetic, in the same order, as tp_bwd_kernel<..., CONV, BC2>;
// without the run-time flags the path contractions are one basic block, so loads, stores and
// LDS reads of neighbouring paths interleave with their FMAs. The edge loop is unrolled by
// two with two operand sets (no register copies between iterations): the operands of the
// next edge load while the current one is contracted.
// EG edge groups of C lanes share a receiver (block C * EG threads): group g takes the edges
// e0 + g, e0 + g + EG, ..., so a receiver with few channels (C = 32: two groups per wave; C = 64:
// one wave per group) still gives the GPU enough waves when the graph has few receivers. Every
// per-edge output is written by one group, so the groups need no combining step.
template <int L1, int L2, int LO, bool SYM>
__host__ __device__ constexpr int bwd_conv_chunk() {
  return AmatLayout<L1, L2, LO, SYM>::chunk >= 2 ? (AmatLayout<L1, L2, LO, SYM>::chunk & ~1) : 2;
}

template <int L1, int L2, int LO, bool SYM, int C, int EG, bool NEED1>
__global__ void __launch_bounds__(C * EG, 2) tp_bwd_conv_kernel(TPArgs g) {
  using CF = TPConfig<L1, L2, LO, SYM>;
  using PL = typename CF::PL;
  using AL = AmatLayout<L1, L2, LO, SYM>;
  constexpr int D1 = CF::D1, D2 = CF::D2, NOUT = CF::NOUT, NP = CF::NP;
  constexpr int T = C * EG;                          // threads
  constexpr int NW = T / 64;                         // waves
  constexpr int GW = C >= 64 ? 64 : C;               // lanes of a group within one wave
  constexpr int NWG = C >= 64 ? C / 64 : 1;          // waves per group
  constexpr int R2 = pow2_at_least(D2), SH2 = log2_exact(GW) - log2_exact(R2);
  constexpr int CH = bwd_conv_chunk<L1, L2, LO, SYM>();
  static_assert((C == 32 || C % 64 == 0) && C <= 256 && T % 64 == 0 && T <= 256, "whole waves of whole groups");
  static_assert(CH % (2 * EG) == 0, "every full chunk gives each group an even number of edges");
  static_assert(2 * CH * AL::total * 4 <= 65536, "coupling-matrix chunks exceed the LDS budget");
  constexpr int64_t SW = (int64_t)NP * C, S1 = (int64_t)D1 * C;
  __shared__ __align__(16) float a_lds[2 * CH * AL::total];
  __shared__ float red_lds[CH * NWG * D2];
  __shared__ int32_t ix_lds[3 * 2 * CH];  // sender and weight row of the edges of three chunks

  const int64_t row = xcd_row(g.n_rows);
  if (row >= g.n_rows) return;
  const int t = threadIdx.x, wave = t >> 6, lane = t & 63;
  const int grp = EG == 1 ? 0 : t / C, f = EG == 1 ? t : t % C;
  const int wig = C >= 64 ? f >> 6 : 0;  // wave within the group
  const int64_t e0 = g.rowptr[row], e1 = g.rowptr[row + 1];
  if (e0 >= e1) return;  // uniform over the workgroup: no barrier is skipped by a part of it

  // The edge loop reads each edge's sender and weight row from LDS, where they are staged two
  // chunks ahead (chunk q in slot q % 3), filled at a chunk boundary with the coupling matrices.
  // Read from global memory in the loop, they are vector loads whose waits (vector-memory
  // operations of a wave complete in issue order) also wait for the prefetched operands and the
  // stores issued before them.
  auto fill_idx = [&](int64_t q0, int q) {
    const int64_t n = e1 - q0 < CH ? e1 - q0 : CH;
    if (t < n) {
      const int64_t e = q0 + t;
      ix_lds[(q % 3) * 2 * CH + t] = g.idx_j[e];
      ix_lds[(q % 3) * 2 * CH + CH + t] = g.wslot ? (g.wslot[e] >> 1) : 0;
    }
  };

  const float alpha = scale_of(g);
  float go[NOUT];
#pragma unroll
  for (int k = 0; k < NOUT; ++k) go[k] = alpha * g.grad_out[row * (int64_t)NOUT * C + (int64_t)k * C + f];

  // Operands of an edge given its sender j and weight row: exactly LD vector loads on every path
  // (an unpaired edge's weights, row -1, are read from the zero row).
  static_assert(SW <= kZeroRowFloats, "zero row");
  auto load_rows = [&](int64_t j, int64_t wrow, EdgeOps<D1, D2, NP>& o) {
    const float* xr = g.in1 + j * S1 + f;
#pragma unroll
    for (int u = 0; u < D1; ++u) o.x[u] = xr[u * C];
    const float* wr = (wrow < 0 ? zero_weight_row : g.w + wrow * SW) + f;
#pragma unroll
    for (int i = 0; i < NP; ++i) o.w[i] = wr[i * C];
  };
  // operands of edge e = (chunk q's first edge) + s, s < CH, from the staged indices
  auto load = [&](int64_t e, int q, int s, EdgeOps<D1, D2, NP>& o) {
    const int* ix = ix_lds + (q % 3) * 2 * CH;
    load_rows(ix[s], g.wslot ? (int64_t)ix[CH + s] : e, o);
  };
  // Before a step the wave waits until at most LD + ST vector-memory operations are outstanding:
  // those issued after the step's own operand loads are the other operand set's loads (LD, every
  // one issued, clamped to the last edge) and the previous step's stores (ST). Operations of a
  // wave complete in issue order, so the step's operands have then arrived, while the next
  // edge's loads and the last stores stay in flight. (The compiler's own waits, placed where a
  // loaded register is first used, count conservatively across the loop's paths and waited for
  // the loads just issued.) A chunk boundary waits for everything: the coupling-matrix fill
  // waits for its own loads, issued after all others.
  constexpr int LD = D1 + NP, ST = NP + (NEED1 ? D1 : 0);
  constexpr int VM_STEP = LD + ST < 63 ? LD + ST : 63;  // at most 63 can be outstanding
  auto wait_operands = [&]() {
    vm_wait_barrier();
    __builtin_amdgcn_s_waitcnt(FC_VMCNT_IMM(VM_STEP));
  };

  auto step = [&](int64_t e, const EdgeOps<D1, D2, NP>& cur, const float* ae, int slot) {
    float gx[D1], gy[R2];
#pragma unroll
    for (int u = 0; u < D1; ++u) gx[u] = 0.f;
#pragma unroll
    for (int u = 0; u < R2; ++u) gy[u] = 0.f;
    float* gwr = g.grad_w + e * SW + f;
    static_for<NP>([&](auto ic) {
      constexpr int i = decltype(ic)::value;
      constexpr PathDesc P = PL::at(i);
      using TP = TPPath<P.r1, P.r2, P.lo>;
      const float* xp = cur.x + P.r1 * P.r1;
      float gop[TP::NO];
#pragma unroll
      for (int a = 0; a < TP::NO; ++a) gop[a] = go[PL::out_index(i, a)];
      float v[TP::N1];
#pragma unroll
      for (int b = 0; b < TP::N1; ++b) v[b] = 0.f;
      TP::apply_t(ae + AL::template off<i>(), gop, v);
      float s = 0.f;
#pragma unroll
      for (int b = 0; b < TP::N1; ++b) s = fmaf(v[b], xp[b], s);
      gwr[i * C] = s;
      if constexpr (NEED1) {
#pragma unroll
        for (int b = 0; b < TP::N1; ++b) gx[P.r1 * P.r1 + b] = fmaf(cur.w[i], v[b], gx[P.r1 * P.r1 + b]);
      }
      float xw[TP::N1];
#pragma unroll
      for (int b = 0; b < TP::N1; ++b) xw[b] = cur.w[i] * xp[b];
      TP::vjp2(gop, xw, gy + P.r2 * P.r2);
    });
    const float s = wave_reduce_halving<R2, GW>(gy, lane);
    const int v = (lane & (GW - 1)) >> SH2;
    if ((lane & ((1 << SH2) - 1)) == 0 && v < D2) red_lds[(slot * NWG + wig) * D2 + v] = s;
    if constexpr (NEED1) {
      float* mr = g.grad_in1 + e * S1 + f;
#pragma unroll
      for (int u = 0; u < D1; ++u) mr[u * C] = gx[u];
    }
  };

  EdgeOps<D1, D2, NP> opa, opb;
  {  // the first edge's operands, from the global indices (the fill below waits for them)
    const int64_t ef = e0 + grp < e1 ? e0 + grp : e1 - 1;
    load_rows(g.idx_j[ef], weight_row(g, ef), opa);
  }
  vm_wait_barrier();
  fill_idx(e0, 0);
  if (e0 + CH < e1) fill_idx(e0 + CH, 1);
  fill_amat<L1, L2, LO, SYM>(g.in2, e0, e1 - e0 < CH ? (int)(e1 - e0) : CH, a_lds, lane, wave, NW);
  __syncthreads();
  vm_wait_barrier();
  __builtin_amdgcn_s_waitcnt(FC_VMCNT_IMM(0));  // the first operands (fewer than LD + ST operations follow them)
  int buf = 0, q = 0;
  // Every chunk but the last holds CH edges, an even number per group, so each chunk starts on
  // operand set a; group grp takes the chunk's slots grp, grp + EG, ...
  // (a load looks at most 2 EG <= CH edges ahead: into this chunk or the next)
  auto load_at = [&](int64_t e, int64_t c0, EdgeOps<D1, D2, NP>& o) {
    const int s = (int)(e - c0);
    if (s < CH) load(e, q, s, o);
    else load(e, q + 1, s - CH, o);
  };
  for (int64_t c0 = e0; c0 < e1; c0 += CH, ++q) {
    const int64_t c1 = c0 + CH < e1 ? c0 + CH : e1;
    const int n = (int)(c1 - c0);
    const int n_next = e1 - c1 < CH ? (int)(e1 - c1) : CH;
    const float* ab = a_lds + buf * CH * AL::total;
    // pairs of edges, then (last chunk only) an odd edge: the loop body has no branch around its
    // loads, stores or waits
    int64_t e = c0 + grp;
    for (; e + EG < c1; e += 2 * EG) {
      const int slot = (int)(e - c0);
      load_at(e + EG, c0, opb);
      wait_operands();
      step(e, opa, ab + slot * AL::total, slot);
      load_at(e + 2 * EG < e1 ? e + 2 * EG : e1 - 1, c0, opa);
      wait_operands();
      step(e + EG, opb, ab + (slot + EG) * AL::total, slot + EG);
    }
    if (e < c1) {
      // opa was loaded before the last step's ST stores (or before a full wait)
      vm_wait_barrier();
      __builtin_amdgcn_s_waitcnt(FC_VMCNT_IMM(ST < 63 ? ST : 63));
      step(e, opa, ab + (int)(e - c0) * AL::total, (int)(e - c0));
    }
    vm_wait_barrier();
    // the other buffer was last read in the previous chunk, before that chunk's barriers; index
    // slot (q + 2) % 3 held chunk q - 1, whose last reads were in that chunk's loop
    if (n_next > 0) fill_amat<L1, L2, LO, SYM>(g.in2, c1, n_next, a_lds + (buf ^ 1) * CH * AL::total, lane, wave, NW);
    if (c1 + CH < e1) fill_idx(c1 + CH, q + 2);
    __syncthreads();
    for (int k = t; k < n * D2; k += T) {
      const int slot = k / D2, u = k % D2;
      float s = 0.f;
#pragma unroll
      for (int w = 0; w < NWG; ++w) s += red_lds[(slot * NWG + w) * D2 + u];
      g.grad_in2[(c0 + slot) * D2 + u] = s;
    }
    __syncthreads();
    buf ^= 1;
  }
}

// The convolution backward in sender order, for C = 64 channels and at most
// kSendMaxOut unreduced output rows (the interaction layers of the 64-channel models): one
// workgroup per sender j walks j's out-edges (sender_perm), gathers each receiver's output
// gradient row and keeps j's in1 row resident, so the in1 gradient of j is summed in registers
// and written once, with no per-edge messages and no separate segmented sum. Per edge it forms
// the weight gradient and the edge-attribute gradient as the receiver-order kernel does (same
// products; the in1 gradient sums in sender order). EG edge groups share a sender as there;
// their in1-gradient partial sums are added in LDS in group order (reproducible).
constexpr int kSendMaxOut = 40;

// Coupling matrices of a chunk of edges given by position in sender_perm.
template <int L1, int L2, int LO, bool SYM>
__device__ __forceinline__ void fill_amat_perm(const float* __restrict__ in2, const int32_t* __restrict__ sperm,
                                               int64_t c0, int n, float* a, int lane, int wave, int nw) {
  using PL = PathList<L1, L2, LO, SYM>;
  using AL = AmatLayout<L1, L2, LO, SYM>;
  constexpr int D2 = ncomp(L2);
  if (lane >= n) return;
  const int64_t e = sperm[c0 + lane];
  float y[D2];
#pragma unroll
  for (int u = 0; u < D2; ++u) y[u] = in2[e * D2 + u];
  float* ae = a + lane * AL::total;
  const int p0 = wave * PL::NP / nw, p1 = (wave + 1) * PL::NP / nw;
  static_for<PL::NP>([&](auto ic) {
    constexpr int i = decltype(ic)::value;
    if (i >= p0 && i < p1) {
      constexpr PathDesc P = PL::at(i);
      TPPath<P.r1, P.r2, P.lo>::amat(y + P.r2 * P.r2, ae + AL::template off<i>());
    }
  });
}

template <int NOUT, int NP>
struct SendOps {
  float go[NOUT], w[NP];
};

template <int L1, int L2, int LO, bool SYM, int C, int EG>
__global__ void __launch_bounds__(C * EG, 2) tp_bwd_send_kernel(TPArgs g) {
  using CF = TPConfig<L1, L2, LO, SYM>;
  using PL = typename CF::PL;
  using AL = AmatLayout<L1, L2, LO, SYM>;
  constexpr int D1 = CF::D1, D2 = CF::D2, NOUT = CF::NOUT, NP = CF::NP;
  constexpr int T = C * EG, NW = T / 64;
  constexpr int GW = C >= 64 ? 64 : C, NWG = C >= 64 ? C / 64 : 1;
  constexpr int R2 = pow2_at_least(D2), SH2 = log2_exact(GW) - log2_exact(R2);
  constexpr int CH = bwd_conv_chunk<L1, L2, LO, SYM>();
  static_assert(C == 64 && T % 64 == 0 && T <= 256, "whole waves of whole groups");
  static_assert(NOUT <= kSendMaxOut, "the gathered output-gradient rows stay in registers");
  static_assert(CH % (2 * EG) == 0, "every full chunk gives each group an even number of edges");
  constexpr int64_t SW = (int64_t)NP * C, S1 = (int64_t)D1 * C, SO = (int64_t)NOUT * C;
  __shared__ __align__(16) float a_lds[2 * CH * AL::total];
  __shared__ float red_lds[CH * NWG * D2];
  __shared__ float gx_lds[(EG > 1 ? EG - 1 : 1) * D1 * C];
  __shared__ int32_t ix_lds[3 * 3 * CH];  // edge, receiver and weight row of the edges of three chunks

  const int64_t row = xcd_row(g.n_rows);  // the sender
  if (row >= g.n_rows) return;
  const int t = threadIdx.x, wave = t >> 6, lane = t & 63;
  const int grp = EG == 1 ? 0 : t / C, f = EG == 1 ? t : t % C;
  const int wig = C >= 64 ? f >> 6 : 0;
  const int64_t k0 = g.sptr[row], k1 = g.sptr[row + 1];
  const float alpha = scale_of(g);
  float x[D1], gx[D1];
#pragma unroll
  for (int u = 0; u < D1; ++u) {
    x[u] = g.in1[row * S1 + (int64_t)u * C + f];
    gx[u] = 0.f;
  }

  // Each out-edge's edge id, receiver and weight row are staged in LDS two chunks ahead (chunk
  // q in slot q % 3), as in tp_bwd_conv_kernel: read from global memory in the loop they are
  // vector loads whose waits also wait for the prefetched rows. The output-gradient rows are
  // scaled where they are used, not as they are loaded, for the same reason.
  auto fill_idx = [&](int64_t q0, int q) {
    const int64_t n = k1 - q0 < CH ? k1 - q0 : CH;
    if (t < n) {
      const int32_t e = g.sperm[q0 + t];
      int32_t* ix = ix_lds + (q % 3) * 3 * CH;
      ix[t] = e;
      ix[CH + t] = g.idx_i[e];
      ix[2 * CH + t] = g.wslot ? (g.wslot[e] >> 1) : e;
    }
  };

  // exactly LD vector loads on every path (row -1: the zero row)
  static_assert(SW <= kZeroRowFloats, "zero row");
  auto load_rows = [&](int64_t i, int64_t wrow, SendOps<NOUT, NP>& o) {
    const float* gr = g.grad_out + i * SO + f;
#pragma unroll
    for (int a = 0; a < NOUT; ++a) o.go[a] = gr[(int64_t)a * C];
    const float* wr = (wrow < 0 ? zero_weight_row : g.w + wrow * SW) + f;
#pragma unroll
    for (int p = 0; p < NP; ++p) o.w[p] = wr[p * C];
  };
  auto load = [&](int q, int s, SendOps<NOUT, NP>& o) {
    const int* ix = ix_lds + (q % 3) * 3 * CH;
    load_rows(ix[CH + s], ix[2 * CH + s], o);
  };
  // explicit waits before each step, as in tp_bwd_conv_kernel: LD loads per edge, ST stores per step
  constexpr int LD = NOUT + NP, ST = NP;
  constexpr int VM_STEP = LD + ST < 63 ? LD + ST : 63;
  auto wait_operands = [&]() {
    vm_wait_barrier();
    __builtin_amdgcn_s_waitcnt(FC_VMCNT_IMM(VM_STEP));
  };

  auto step = [&](int64_t e, const SendOps<NOUT, NP>& cur, const float* ae, int slot) {
    float gy[R2];
#pragma unroll
    for (int u = 0; u < R2; ++u) gy[u] = 0.f;
    float* gwr = g.grad_w + e * SW + f;
    static_for<NP>([&](auto ic) {
      constexpr int i = decltype(ic)::value;
      constexpr PathDesc P = PL::at(i);
      using TP = TPPath<P.r1, P.r2, P.lo>;
      const float* xp = x + P.r1 * P.r1;
      float gop[TP::NO];
#pragma unroll
      for (int a = 0; a < TP::NO; ++a) gop[a] = alpha * cur.go[PL::out_index(i, a)];
      float v[TP::N1];
#pragma unroll
      for (int b = 0; b < TP::N1; ++b) v[b] = 0.f;
      TP::apply_t(ae + AL::template off<i>(), gop, v);
      float sw = 0.f;
#pragma unroll
      for (int b = 0; b < TP::N1; ++b) sw = fmaf(v[b], xp[b], sw);
      gwr[i * C] = sw;
#pragma unroll
      for (int b = 0; b < TP::N1; ++b) gx[P.r1 * P.r1 + b] = fmaf(cur.w[i], v[b], gx[P.r1 * P.r1 + b]);
      float xw[TP::N1];
#pragma unroll
      for (int b = 0; b < TP::N1; ++b) xw[b] = cur.w[i] * xp[b];
      TP::vjp2(gop, xw, gy + P.r2 * P.r2);
    });
    const float s = wave_reduce_halving<R2, GW>(gy, lane);
    const int v = (lane & (GW - 1)) >> SH2;
    if ((lane & ((1 << SH2) - 1)) == 0 && v < D2) red_lds[(slot * NWG + wig) * D2 + v] = s;
  };

  if (k0 < k1) {  // uniform over the workgroup
    SendOps<NOUT, NP> opa, opb;
    fill_idx(k0, 0);
    if (k0 + CH < k1) fill_idx(k0 + CH, 1);
    fill_amat_perm<L1, L2, LO, SYM>(g.in2, g.sperm, k0, k1 - k0 < CH ? (int)(k1 - k0) : CH, a_lds, lane, wave, NW);
    __syncthreads();
    load(0, k0 + grp < k1 ? grp : (int)(k1 - 1 - k0), opa);
    vm_wait_barrier();
    __builtin_amdgcn_s_waitcnt(FC_VMCNT_IMM(0));  // the first operands
    int buf = 0, q = 0;
    // a load looks at most 2 EG <= CH edges ahead: into this chunk or the next
    auto load_at = [&](int64_t k, int64_t c0, SendOps<NOUT, NP>& o) {
      const int s = (int)(k - c0);
      if (s < CH) load(q, s, o);
      else load(q + 1, s - CH, o);
    };
    for (int64_t c0 = k0; c0 < k1; c0 += CH, ++q) {
      const int64_t c1 = c0 + CH < k1 ? c0 + CH : k1;
      const int n = (int)(c1 - c0);
      const int n_next = k1 - c1 < CH ? (int)(k1 - c1) : CH;
      const float* ab = a_lds + buf * CH * AL::total;
      const int* ixe = ix_lds + (q % 3) * 3 * CH;  // this chunk's edge ids
      // pairs of edges, then (last chunk only) an odd edge, as in tp_bwd_conv_kernel
      int64_t k = c0 + grp;
      for (; k + EG < c1; k += 2 * EG) {
        const int slot = (int)(k - c0);
        load_at(k + EG, c0, opb);
        wait_operands();
        step(ixe[slot], opa, ab + slot * AL::total, slot);
        load_at(k + 2 * EG < k1 ? k + 2 * EG : k1 - 1, c0, opa);
        wait_operands();
        step(ixe[slot + EG], opb, ab + (slot + EG) * AL::total, slot + EG);
      }
      if (k < c1) {
        vm_wait_barrier();
        __builtin_amdgcn_s_waitcnt(FC_VMCNT_IMM(ST < 63 ? ST : 63));
        step(ixe[k - c0], opa, ab + (int)(k - c0) * AL::total, (int)(k - c0));
      }
      vm_wait_barrier();
      if (n_next > 0)
        fill_amat_perm<L1, L2, LO, SYM>(g.in2, g.sperm, c1, n_next, a_lds + (buf ^ 1) * CH * AL::total, lane, wave, NW);
      // slot (q + 2) % 3 held chunk q - 1, whose last reads were in that chunk's loop
      if (c1 + CH < k1) fill_idx(c1 + CH, q + 2);
      __syncthreads();
      for (int r = t; r < n * D2; r += T) {
        const int slot = r / D2, u = r % D2;
        float sum = 0.f;
#pragma unroll
        for (int w = 0; w < NWG; ++w) sum += red_lds[(slot * NWG + w) * D2 + u];
        g.grad_in2[(int64_t)ixe[slot] * D2 + u] = sum;
      }
      __syncthreads();
      buf ^= 1;
    }
  }
  // the groups' in1 gradients, added in group order
  if constexpr (EG > 1) {
    if (grp > 0) {
#pragma unroll
      for (int u = 0; u < D1; ++u) gx_lds[((grp - 1) * D1 + u) * C + f] = gx[u];
    }
    __syncthreads();
    if (grp > 0) return;
#pragma unroll
    for (int q = 1; q < EG; ++q)
#pragma unroll
      for (int u = 0; u < D1; ++u) gx[u] += gx_lds[((q - 1) * D1 + u) * C + f];
  }
#pragma unroll
  for (int u = 0; u < D1; ++u) g.grad_in1[row * S1 + (int64_t)u * C + f] = gx[u];
}

// Backward of the node-wise (rows) product with full-width inputs (F1 == F2 == C) and
// per-path outputs: no channel reduction, so no LDS or barriers. The output gradient
// of a path is read when the path is processed (the node-wise kernels have no edge
// loop to amortise a full go row over, and keeping it all in registers halves the
// occupancy that hides the loads).
template <int L1, int L2, int LO, bool SYM>
__global__ void __launch_bounds__(256) tp_bwd_rows_kernel(TPArgs g) {
  using CF = TPConfig<L1, L2, LO, SYM>;
  using PL = typename CF::PL;
  constexpr int D1 = CF::D1, D2 = CF::D2, NOUT = CF::NOUT, NP = CF::NP;
  const int64_t row = blockIdx.x;
  const int f = threadIdx.x;
  const int C = g.C;
  if (f >= C || row >= g.n_rows) return;
  const bool need1 = g.grad_in1 != nullptr, need2 = g.grad_in2 != nullptr, needw = g.grad_w != nullptr;
  const float alpha = scale_of(g);
  const float* gor = g.grad_out + row * (int64_t)NOUT * C + f;
  const float* wr = (g.shared_w ? g.w : g.w + row * (int64_t)NP * C) + f;
  float x[D1], y[D2], gx[D1], gy[D2];
#pragma unroll
  for (int u = 0; u < D1; ++u) { x[u] = g.in1[(row * D1 + u) * (int64_t)C + f]; gx[u] = 0.f; }
#pragma unroll
  for (int u = 0; u < D2; ++u) { y[u] = g.in2[(row * D2 + u) * (int64_t)C + f]; gy[u] = 0.f; }
  static_for<NP>([&](auto ic) {
    constexpr int i = decltype(ic)::value;
    constexpr PathDesc P = PL::at(i);
    using T = TPPath<P.r1, P.r2, P.lo>;
    const float* xp = x + P.r1 * P.r1;
    float go[T::NO];
#pragma unroll
    for (int a = 0; a < T::NO; ++a) go[a] = alpha * gor[(int64_t)PL::out_index(i, a) * C];
    const float w = wr[i * C];
    if (needw || need1) {  // v = A_p^T go_p: grad_w = <v, x>, gx += w v
      float A[T::NA], v[T::N1];
      T::amat(y + P.r2 * P.r2, A);
#pragma unroll
      for (int b = 0; b < T::N1; ++b) v[b] = 0.f;
      T::apply_t(A, go, v);
      if (needw) {
        float s = 0.f;
#pragma unroll
        for (int b = 0; b < T::N1; ++b) s = fmaf(v[b], xp[b], s);
        g.grad_w[row * (int64_t)NP * C + i * C + f] = s;
      }
      if (need1) {
#pragma unroll
        for (int b = 0; b < T::N1; ++b) gx[P.r1 * P.r1 + b] = fmaf(w, v[b], gx[P.r1 * P.r1 + b]);
      }
    }
    if (need2) {  // gy += B_p(go_p, w x)
      float xw[T::N1];
#pragma unroll
      for (int b = 0; b < T::N1; ++b) xw[b] = w * xp[b];
      T::vjp2(go, xw, gy + P.r2 * P.r2);
    }
  });
  // residual gradients: each element is read and then written by this thread only
  if (need1) {
    if (g.res1) {
#pragma unroll
      for (int u = 0; u < D1; ++u)
        if (u < g.res1_comps) gx[u] += g.res1[(row * g.res1_comps + u) * (int64_t)C + f];
    }
#pragma unroll
    for (int u = 0; u < D1; ++u) g.grad_in1[(row * D1 + u) * (int64_t)C + f] = gx[u];
  }
  if (need2) {
    if (g.res2) {
#pragma unroll
      for (int u = 0; u < D2; ++u)
        if (u < g.res2_comps) gy[u] += g.res2[(row * g.res2_comps + u) * (int64_t)C + f];
    }
#pragma unroll
    for (int u = 0; u < D2; ++u) g.grad_in2[(row * D2 + u) * (int64_t)C + f] = gy[u];
  }
}

// Edge groups per receiver of the convolution kernels with C <= 64 channels: enough waves to
// occupy the GPU (about four per SIMD, 4,096) when the graph has few receivers, at most 256
// threads per workgroup and at most half the mean in-degree per group.
inline int conv_edge_groups(int64_t n_rows, int64_t n_edges, int C) {
  // 512 receivers x 8 edges with 32 channels: 29.0 us per forward + backward with four groups,
  // 32.4 us with eight (measured on the standalone product of the benchmark's first configuration)
  const int max_eg = C == 32 || C == 64 ? 4 : 1;
  int eg = C == 32 ? 2 : 1;
  const double deg = n_rows > 0 ? (double)n_edges / (double)n_rows : 0.0;
  while (eg < max_eg && (double)n_rows * eg * C / 64.0 < 4096.0 && 2.0 * eg <= deg) eg *= 2;
  return eg;
}

// The specialised convolution backward with C channels and EG edge groups; false (nothing
// launched) when a full coupling-matrix chunk would not split evenly over the groups.
template <int L1, int L2, int LO, bool SYM, int C, int EG>
bool launch_bwd_conv(const TPArgs& g, dim3 grid, hipStream_t stream) {
  if constexpr (bwd_conv_chunk<L1, L2, LO, SYM>() % (2 * EG) != 0) {
    return false;
  } else {
    if (g.grad_in1) hipLaunchKernelGGL((tp_bwd_conv_kernel<L1, L2, LO, SYM, C, EG, true>), grid, dim3(C * EG), 0, stream, g);
    else hipLaunchKernelGGL((tp_bwd_conv_kernel<L1, L2, LO, SYM, C, EG, false>), grid, dim3(C * EG), 0, stream, g);
    return true;
  }
}

// Sender-order backward with C channels and EG edge groups; false when a full chunk would not
// split evenly over the groups.
template <int L1, int L2, int LO, bool SYM, int C, int EG>
bool launch_bwd_send(const TPArgs& g, dim3 grid, hipStream_t stream) {
  if constexpr (bwd_conv_chunk<L1, L2, LO, SYM>() % (2 * EG) != 0) {
    return false;
  } else {
    hipLaunchKernelGGL((tp_bwd_send_kernel<L1, L2, LO, SYM, C, EG>), grid, dim3(C * EG), 0, stream, g);
    return true;
  }
}

// launch_tp's answer when a sender-order backward was asked for a configuration it does not cover
constexpr int kSendNotApplicable = -100;

template <int L1, int L2, int LO, bool SYM, int EG>
void launch_fwd_groups(const TPArgs& g, dim3 grid, hipStream_t stream) {
  using CF = TPConfig<L1, L2, LO, SYM>;
  const size_t lds = sizeof(float) * (size_t)(EG - 1) * CF::NOUT * g.C;
  hipLaunchKernelGGL((tp_fwd_kernel<L1, L2, LO, SYM, true, true, EG>), grid, dim3(g.C * EG), lds, stream, g);
}

// Host-side launcher for one configuration.
template <int L1, int L2, int LO, bool SYM>
int launch_tp(const TPArgs& g, bool conv, bool bwd, hipStream_t stream) {
  if (g.n_rows == 0) return FC_OK;
  const int threads = ((g.C + 63) / 64) * 64;
  if (threads > 256) return FC_ERR_SHAPE;
  dim3 grid((unsigned)(conv ? xcd_grid(g.n_rows) : g.n_rows)), block(threads);
  const bool bc2 = conv && g.F2 == 1;
  // edge groups for few-channel convolutions (one in2 channel, full-width in1)
  const int eg0 = (bc2 && g.F1 == g.C && (g.C == 32 || g.C == 64)) ? conv_edge_groups(g.n_rows, g.n_edges, g.C) : 1;
  if (bwd) {
    const bool reduce = (g.grad_in1 && g.F1 == 1 && g.C > 1) || (g.grad_in2 && g.F2 == 1 && g.C > 1);
    const size_t per_edge = reduce ? sizeof(float) * (threads / 64) * (ncomp(L1) + ncomp(L2)) : 0;
    if (g.sender_major) {  // only launched here; the caller falls back to messages otherwise
      if constexpr (!SYM && L2 >= 1 && TPConfig<L1, L2, LO, SYM>::NOUT <= kSendMaxOut) {
        // 64 channels only: with 32 (the standalone 2x2->2 product, 512 senders) the sender order
        // measured 7% slower per call than messages plus their gather
        if (conv && bc2 && !g.reduced && !g.shared_w && g.grad_w && g.grad_in2 && g.grad_in1 && g.F1 == g.C &&
            g.C == 64) {
          const int eg = conv_edge_groups(g.n_rows, g.n_edges, g.C);
          const dim3 sgrid((unsigned)xcd_grid(g.n_rows));
          const bool done = (eg >= 4 && launch_bwd_send<L1, L2, LO, SYM, 64, 4>(g, sgrid, stream)) ||
                            (eg >= 2 && launch_bwd_send<L1, L2, LO, SYM, 64, 2>(g, sgrid, stream)) ||
                            launch_bwd_send<L1, L2, LO, SYM, 64, 1>(g, sgrid, stream);
          if (done) {
            FC_LAUNCH_CHECK();
            return FC_OK;
          }
        }
      }
      return kSendNotApplicable;
    }
    if constexpr (!SYM && L2 >= 1) {
      // interaction-layer shape: the compile-time specialisation
      if (conv && bc2 && !g.reduced && !g.shared_w && g.grad_w && g.grad_in2 && g.F1 == g.C &&
          (g.C == 32 || g.C == 64 || g.C == 128)) {  // per-edge weights: the kernel reads w[e] rows
        bool done = false;
        if (g.C == 128) {
          done = launch_bwd_conv<L1, L2, LO, SYM, 128, 1>(g, grid, stream);
        } else if (g.C == 64) {
          done = (eg0 >= 4 && launch_bwd_conv<L1, L2, LO, SYM, 64, 4>(g, grid, stream)) ||
                 (eg0 >= 2 && launch_bwd_conv<L1, L2, LO, SYM, 64, 2>(g, grid, stream)) ||
                 launch_bwd_conv<L1, L2, LO, SYM, 64, 1>(g, grid, stream);
        } else {
          done = (eg0 >= 4 && launch_bwd_conv<L1, L2, LO, SYM, 32, 4>(g, grid, stream)) ||
                 launch_bwd_conv<L1, L2, LO, SYM, 32, 2>(g, grid, stream);
        }
        if (done) {
          FC_LAUNCH_CHECK();
          return FC_OK;
        }
      }
    }
    if (conv) {
      if (bc2)
        hipLaunchKernelGGL((tp_bwd_kernel<L1, L2, LO, SYM, true, true>), grid, block,
                           (per_edge * bwd_chunk<L1, L2, LO, SYM, true, true>()), stream, g);
      else
        hipLaunchKernelGGL((tp_bwd_kernel<L1, L2, LO, SYM, true, false>), grid, block,
                           (per_edge * bwd_chunk<L1, L2, LO, SYM, true, false>()), stream, g);
    } else if (g.F1 == g.C && g.F2 == g.C && !g.reduced) {
      hipLaunchKernelGGL((tp_bwd_rows_kernel<L1, L2, LO, SYM>), grid, block, 0, stream, g);
    } else {
      hipLaunchKernelGGL((tp_bwd_kernel<L1, L2, LO, SYM, false, false>), grid, block,
                         (per_edge * bwd_chunk<L1, L2, LO, SYM, false, false>()), stream, g);
    }
  } else {
    // the forward's groups add their partial sums at the end: half as many groups measured as fast
    // with 64 channels (water box, 1,536 receivers: 52 us with one group per receiver, 48 with two,
    // 51 with four), as many as the backward with 32
    const int eg = g.C == 64 ? (eg0 + 1) / 2 : eg0;
    if (conv) {
      if (bc2 && eg >= 4) launch_fwd_groups<L1, L2, LO, SYM, 4>(g, grid, stream);
      else if (bc2 && eg >= 2) launch_fwd_groups<L1, L2, LO, SYM, 2>(g, grid, stream);
      else if (bc2) hipLaunchKernelGGL((tp_fwd_kernel<L1, L2, LO, SYM, true, true>), grid, block, 0, stream, g);
      else hipLaunchKernelGGL((tp_fwd_kernel<L1, L2, LO, SYM, true, false>), grid, block, 0, stream, g);
    } else {
      hipLaunchKernelGGL((tp_fwd_kernel<L1, L2, LO, SYM, false, false>), grid, block, 0, stream, g);
    }
  }
  FC_LAUNCH_CHECK();
  return FC_OK;
}

// Per-L1 dispatchers, defined in fc_tp_l<L1>.hip (split for parallel compilation).
int dispatch_tp_l0(int l2, int lo, bool sym, const TPArgs& g, bool conv, bool bwd, hipStream_t s);
int dispatch_tp_l1(int l2, int lo, bool sym, const TPArgs& g, bool conv, bool bwd, hipStream_t s);
int dispatch_tp_l2(int l2, int lo, bool sym, const TPArgs& g, bool conv, bool bwd, hipStream_t s);
int dispatch_tp_l3(int l2, int lo, bool sym, const TPArgs& g, bool conv, bool bwd, hipStream_t s);
#if FC_KERNEL_L_MAX >= 4
int dispatch_tp_l4(int l2, int lo, bool sym, const TPArgs& g, bool conv, bool bwd, hipStream_t s);
#endif

template <int L1>
int dispatch_tp_for(int l2, int lo, bool sym, const TPArgs& g, bool conv, bool bwd, hipStream_t s) {
#define FC_TP_CASE(A, B)                                                        \
  if (l2 == A && lo == B) {                                                     \
    if (sym) {                                                                  \
      if constexpr (L1 == A) return launch_tp<L1, A, B, true>(g, conv, bwd, s); \
      else return FC_ERR_BAD_DESC;                                              \
    }                                                                           \
    return launch_tp<L1, A, B, false>(g, conv, bwd, s);                         \
  }
  FC_TP_CASE(0, 0) FC_TP_CASE(0, 1) FC_TP_CASE(0, 2) FC_TP_CASE(0, 3)
  FC_TP_CASE(1, 0) FC_TP_CASE(1, 1) FC_TP_CASE(1, 2) FC_TP_CASE(1, 3)
  FC_TP_CASE(2, 0) FC_TP_CASE(2, 1) FC_TP_CASE(2, 2) FC_TP_CASE(2, 3)
  FC_TP_CASE(3, 0) FC_TP_CASE(3, 1) FC_TP_CASE(3, 2) FC_TP_CASE(3, 3)
#if FC_KERNEL_L_MAX >= 4
  FC_TP_CASE(0, 4) FC_TP_CASE(1, 4) FC_TP_CASE(2, 4) FC_TP_CASE(3, 4)
  FC_TP_CASE(4, 0) FC_TP_CASE(4, 1) FC_TP_CASE(4, 2) FC_TP_CASE(4, 3) FC_TP_CASE(4, 4)
#endif
#undef FC_TP_CASE
  return FC_ERR_UNSUPPORTED_L;
}

}  // namespace fc
