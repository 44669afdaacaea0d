// Shared device/host helpers for the flashcart HIP library (gfx950 / CDNA4).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>
#include <utility>

#include "../../include/flashcart_hip.h"

namespace fc {

// ---------------------------------------------------------------------------
// Compile-time path list of one tensor-product configuration.
//
// Order (the weight / output layout contract): for each output rank lo, first the
// canonical pairs (l1 >= l2, l1 read from in1), l1 ascending then l2 ascending;
// then, unless symmetric, the exchanged unequal pairs (l1 > l2, l1 read from in2).
// Reference: src/flashcart/o3/utils.py:157-203,
// src/flashcart/o3/_codegen_tensor_product.py:596-622,964-983.
// ---------------------------------------------------------------------------
struct PathDesc {
  int r1, r2, lo;  // rank read from in1, rank read from in2, output rank
  int q;           // position of the path inside its output-rank block
};

__host__ __device__ constexpr bool allowed(int l1, int l2, int lo) {
  return l1 >= 0 && l2 >= 0 && lo >= 0 && lo >= (l1 > l2 ? l1 - l2 : l2 - l1) && lo <= l1 + l2 &&
         ((l1 + l2 + lo) % 2 == 0);
}

template <int L1, int L2, int LO, bool SYM>
struct PathList {
  static constexpr int LP = L1 > L2 ? L1 : L2;

  // Visit paths in order; returns the count, fills `out` when non-null.
  __host__ __device__ static constexpr int enumerate(PathDesc* out) {
    int n = 0;
    for (int lo = 0; lo <= LO; ++lo) {
      int q = 0;
      for (int l1 = 0; l1 <= LP; ++l1)
        for (int l2 = 0; l2 <= l1; ++l2)
          if (allowed(l1, l2, lo) && l1 <= L1 && l2 <= L2) {
            if (out) out[n] = PathDesc{l1, l2, lo, q};
            ++n; ++q;
          }
      if (!SYM)
        for (int l1 = 0; l1 <= LP; ++l1)
          for (int l2 = 0; l2 < l1; ++l2)
            if (allowed(l1, l2, lo) && l1 <= L2 && l2 <= L1) {
              if (out) out[n] = PathDesc{l2, l1, lo, q};
              ++n; ++q;
            }
    }
    return n;
  }
  static constexpr int NP = enumerate(nullptr);

  // All derived quantities are tabulated once per configuration (constant
  // evaluation in clang is slow, and the kernels query them per path/component).
  struct Table {
    PathDesc p[64];
    int per_lo[8];
    int off[9];      // non-reduced block offsets (components)
    int off_red[9];  // reduced block offsets
  };
  __host__ __device__ static constexpr Table make_table() {
    Table t{};
    enumerate(t.p);
    for (int i = 0; i < NP; ++i) t.per_lo[t.p[i].lo] += 1;
    for (int l = 0; l <= LO; ++l) {
      t.off[l + 1] = t.off[l] + (2 * l + 1) * t.per_lo[l];
      t.off_red[l + 1] = t.off_red[l] + (2 * l + 1) * (t.per_lo[l] > 0 ? 1 : 0);
    }
    return t;
  }
  static constexpr Table T = make_table();

  __host__ __device__ static constexpr PathDesc at(int i) { return T.p[i]; }
  __host__ __device__ static constexpr int paths_of(int lo) { return T.per_lo[lo]; }
  // Offset (in components, i.e. units of the feature count) of output block lo.
  __host__ __device__ static constexpr int out_off(int lo, bool reduced) {
    return reduced ? T.off_red[lo] : T.off[lo];
  }
  static constexpr int NOUT = T.off[LO + 1];          // non-reduced output components
  static constexpr int NOUT_RED = T.off_red[LO + 1];  // reduced output components
  // Component index of (path i, output component a) in the non-reduced layout
  // (2lo+1, paths_lo, C) and in the reduced layout (2lo+1, C).
  __host__ __device__ static constexpr int out_index(int i, int a) {
    return T.off[T.p[i].lo] + a * T.per_lo[T.p[i].lo] + T.p[i].q;
  }
  __host__ __device__ static constexpr int out_index_red(int i, int a) { return T.off_red[T.p[i].lo] + a; }
};

template <class F, int... I>
__device__ __forceinline__ void static_for_impl(F&& f, std::integer_sequence<int, I...>) {
  (f(std::integral_constant<int, I>{}), ...);
}
template <int N, class F>
__device__ __forceinline__ void static_for(F&& f) {
  static_for_impl(f, std::make_integer_sequence<int, N>{});
}

__host__ __device__ constexpr int ncomp(int l_max) { return (l_max + 1) * (l_max + 1); }

// XCD-aware row order: the hardware deals workgroup b to XCD b % 8, so consecutive rows
// would land in 8 different L2s. Giving each XCD a contiguous row range keeps rows that
// share gathered operands (neighbouring receivers share senders) in one L2. The grid
// must be xcd_grid(n) blocks; rows >= n are padding and exit.
__host__ __device__ inline int64_t xcd_grid(int64_t n) { return n >= 64 ? (n + 7) / 8 * 8 : n; }
__device__ __forceinline__ int64_t xcd_row(int64_t n) {
  const int64_t b = blockIdx.x;
  if (n < 64) return b;
  const int64_t per = (n + 7) / 8;
  return (b % 8) * per + b / 8;
}

// Wave64 sum reduction (result valid in every lane).
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}

// A global pointer that is the same in every lane, moved to scalar registers and typed as
// global memory: accesses through it plus a 32-bit lane byte offset can compile to global
// loads and stores with a scalar base (no per-lane 64-bit address arithmetic), not flat ones.
typedef __attribute__((address_space(1))) float gfloat;
typedef __attribute__((address_space(1))) char gchar;
__device__ __forceinline__ gfloat* uniform_gptr(const float* p) {
  const uint64_t v = (uint64_t)(uintptr_t)p;
  const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)v);
  const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)(v >> 32));
  return (gfloat*)(uintptr_t)(((uint64_t)hi << 32) | lo);
}
}  // namespace fc

#define FC_LAUNCH_CHECK()                                    \
  do {                                                       \
    hipError_t _e = hipGetLastError();                       \
    if (_e != hipSuccess) return FC_ERR_LAUNCH;              \
  } while (0)
