// Fused invariant RMS normalisation of Cartesian features and its input gradient
// (reference src/flashcart/nn/layers.py:494-528, RMSLayerNorm.forward without centering):
//   inv_l[c]  = TP_sym(x_l, x_l) -> rank 0      (the (l, l, 0) coupling, unit weight)
//   m         = (1/C) sum_c sum_l inv_l[c] / ((2l+1)(L+1))
//   s         = (m + eps)^-1/2
//   out_l[a,c] = x_l[a,c] * s * g_l[c]
// The reference runs a tensor-product kernel plus five elementwise/reduction passes;
// here one pass reads x once and writes out once (and s, for the backward).
// One workgroup per node, one lane per channel; the channel sum is a wave butterfly
// plus a fixed-order sum over the waves, so results are deterministic.
#include "fc_common.h"
#include "generated/fc_tp_paths.h"

namespace fc {

template <int L>
__device__ __forceinline__ float rank_weight(int l) {
  return 1.0f / (float)((2 * l + 1) * (L + 1));
}

// Sum over the block's channels (blockDim.x = 64 * waves, <= 256); every thread gets the total.
__device__ __forceinline__ float block_channel_sum(float v, float* part) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, nw = blockDim.x >> 6;
  v = wave_sum(v);
  if (lane == 0) part[wave] = v;
  __syncthreads();
  float s = 0.f;
  for (int w = 0; w < nw; ++w) s += part[w];
  __syncthreads();
  return s;
}

template <int L>
__global__ void __launch_bounds__(256) rms_norm_fwd_kernel(int64_t n, int C, const float* __restrict__ x,
                                                           const float* __restrict__ g, float eps,
                                                           float* __restrict__ out, float* __restrict__ scale) {
  constexpr int D = ncomp(L);
  __shared__ float part[4];
  const int64_t node = blockIdx.x;
  const int f = threadIdx.x;
  const bool active = f < C;
  const int fa = active ? f : 0;
  const float* xr = x + node * (int64_t)D * C;
  float v[D];
#pragma unroll
  for (int k = 0; k < D; ++k) v[k] = active ? xr[(int64_t)k * C + fa] : 0.f;
  float t = 0.f;
  static_for<L + 1>([&](auto lc) {
    constexpr int l = decltype(lc)::value;
    float o[1];
    TPPath<l, l, 0>::fwd(v + l * l, v + l * l, o);
    t = fmaf(rank_weight<L>(l), o[0], t);
  });
  const float m = block_channel_sum(active ? t : 0.f, part) / (float)C;
  const float s = 1.0f / sqrtf(m + eps);
  if (!active) return;
  float* orow = out + node * (int64_t)D * C;
  static_for<L + 1>([&](auto lc) {
    constexpr int l = decltype(lc)::value;
    const float gs = s * g[l * C + f];
#pragma unroll
    for (int a = 0; a < 2 * l + 1; ++a) orow[(int64_t)(l * l + a) * C + f] = v[l * l + a] * gs;
  });
  if (f == 0 && scale) scale[node] = s;
}

// gx = go*g*s - (s^3 / (2C)) * R * w_l * d inv_l / dx,  R = sum_{l,a,c} go*g*x
template <int L>
__global__ void __launch_bounds__(256) rms_norm_bwd_kernel(int64_t n, int C, const float* __restrict__ go,
                                                           const float* __restrict__ x, const float* __restrict__ g,
                                                           const float* __restrict__ scale,
                                                           float* __restrict__ gx) {
  constexpr int D = ncomp(L);
  __shared__ float part[4];
  const int64_t node = blockIdx.x;
  const int f = threadIdx.x;
  const bool active = f < C;
  const int fa = active ? f : 0;
  const int64_t base = node * (int64_t)D * C;
  float v[D], gg[D];
  float r = 0.f;
  static_for<L + 1>([&](auto lc) {
    constexpr int l = decltype(lc)::value;
    const float gl = active ? g[l * C + fa] : 0.f;
#pragma unroll
    for (int a = 0; a < 2 * l + 1; ++a) {
      const int k = l * l + a;
      v[k] = active ? x[base + (int64_t)k * C + fa] : 0.f;
      gg[k] = active ? go[base + (int64_t)k * C + fa] * gl : 0.f;
      r = fmaf(gg[k], v[k], r);
    }
  });
  const float R = block_channel_sum(r, part);
  if (!active) return;
  const float s = scale[node];
  const float coef = -0.5f * s * s * s * R / (float)C;
  float* grow = gx + base;
  static_for<L + 1>([&](auto lc) {
    constexpr int l = decltype(lc)::value;
    constexpr int N = 2 * l + 1;
    float d[N];
#pragma unroll
    for (int a = 0; a < N; ++a) d[a] = 0.f;
    const float u[1] = {1.0f};
    TPPath<l, l, 0>::vjp1(u, v + l * l, d);
    TPPath<l, l, 0>::vjp2(u, v + l * l, d);
    const float cw = coef * rank_weight<L>(l);
#pragma unroll
    for (int a = 0; a < N; ++a) grow[(int64_t)(l * l + a) * C + f] = fmaf(cw, d[a], gg[l * l + a] * s);
  });
}

template <int L>
int launch_rms(bool bwd, int64_t n, int C, const float* go, const float* x, const float* g, float eps, float* out,
               float* scale, hipStream_t s) {
  const int threads = ((C + 63) / 64) * 64;
  if (bwd)
    hipLaunchKernelGGL(rms_norm_bwd_kernel<L>, dim3((unsigned)n), dim3(threads), 0, s, n, C, go, x, g, scale, out);
  else
    hipLaunchKernelGGL(rms_norm_fwd_kernel<L>, dim3((unsigned)n), dim3(threads), 0, s, n, C, x, g, eps, out, scale);
  FC_LAUNCH_CHECK();
  return FC_OK;
}

static int rms_dispatch(bool bwd, int64_t n, int l_max, int C, const float* go, const float* x, const float* g,
                        float eps, float* out, float* scale, hipStream_t s) {
  if (n < 0 || C < 1) return FC_ERR_SHAPE;
  if (l_max < 0) return FC_ERR_BAD_DESC;
  if (l_max > FC_KERNEL_L_MAX) return FC_ERR_UNSUPPORTED_L;
  if (C > 256 || n > 0x7fffffff) return FC_ERR_SHAPE;
  if (n == 0) return FC_OK;
  switch (l_max) {
    case 0: return launch_rms<0>(bwd, n, C, go, x, g, eps, out, scale, s);
    case 1: return launch_rms<1>(bwd, n, C, go, x, g, eps, out, scale, s);
    case 2: return launch_rms<2>(bwd, n, C, go, x, g, eps, out, scale, s);
    case 3: return launch_rms<3>(bwd, n, C, go, x, g, eps, out, scale, s);
  }
  return FC_ERR_UNSUPPORTED_L;
}

}  // namespace fc

using namespace fc;

extern "C" int fc_rms_norm_fwd(int64_t n, int32_t l_max, int32_t C, const float* x, const float* weight, float eps,
                               float* out, float* scale, void* stream) {
  if (n > 0 && (!x || !weight || !out)) return FC_ERR_NULL;
  return rms_dispatch(false, n, l_max, C, nullptr, x, weight, eps, out, scale, (hipStream_t)stream);
}

extern "C" int fc_rms_norm_bwd(int64_t n, int32_t l_max, int32_t C, const float* grad_out, const float* x,
                               const float* weight, const float* scale, float* grad_x, void* stream) {
  if (n > 0 && (!grad_out || !x || !weight || !scale || !grad_x)) return FC_ERR_NULL;
  return rms_dispatch(true, n, l_max, C, grad_out, x, weight, 0.f, grad_x, const_cast<float*>(scale),
                      (hipStream_t)stream);
}
