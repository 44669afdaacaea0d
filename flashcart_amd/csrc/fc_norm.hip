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
#include "fc_tp_paths.h"

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

// Second derivative (force-loss training): the backward of rms_norm_bwd. With
// G = g_l[c] broadcast over components, u = d m / dx = (1/C) w_l (vjp1 + vjp2)(x_l) and
// gx = s go G - s^3/2 t u, t = sum go G x, the cotangent cc of gx gives, per node,
//   p = sum cc go G,  q = sum cc u,  v = (1/C) w_l (vjp1 + vjp2)(cc_l)  (M_l symmetric):
//   d go = s cc G - s^3/2 q G x
//   d x  = u (-s^3/2 p + 3/4 s^5 t q) - s^3/2 q go G - s^3/2 t v
//   d g_l[c] (this node's share) = sum_a (s cc go - s^3/2 q go x)
template <int L>
__global__ void __launch_bounds__(256) rms_norm_dbwd_kernel(int64_t n, int C, const float* __restrict__ go,
                                                            const float* __restrict__ x,
                                                            const float* __restrict__ g,
                                                            const float* __restrict__ scale,
                                                            const float* __restrict__ cc, float* __restrict__ d_go,
                                                            float* __restrict__ d_x, float* __restrict__ d_g_part) {
  constexpr int D = ncomp(L);
  __shared__ float part[4];
  const int64_t node = blockIdx.x;
  const int f = threadIdx.x;
  const bool active = f < C;
  const int fa = active ? f : 0;
  const int64_t base = node * (int64_t)D * C;
  float xv[D], gv[D], cv[D], ux[D], vc[D], G[L + 1];
  float t = 0.f, p = 0.f, q = 0.f;
  static_for<L + 1>([&](auto lc) {
    constexpr int l = decltype(lc)::value;
    constexpr int N = 2 * l + 1;
    G[l] = active ? g[l * C + fa] : 0.f;
#pragma unroll
    for (int a = 0; a < N; ++a) {
      const int k = l * l + a;
      xv[k] = active ? x[base + (int64_t)k * C + fa] : 0.f;
      gv[k] = active ? go[base + (int64_t)k * C + fa] : 0.f;
      cv[k] = active ? cc[base + (int64_t)k * C + fa] : 0.f;
    }
    float dx[N], dc[N];
#pragma unroll
    for (int a = 0; a < N; ++a) dx[a] = dc[a] = 0.f;
    const float one[1] = {1.0f};
    TPPath<l, l, 0>::vjp1(one, xv + l * l, dx);
    TPPath<l, l, 0>::vjp2(one, xv + l * l, dx);
    TPPath<l, l, 0>::vjp1(one, cv + l * l, dc);
    TPPath<l, l, 0>::vjp2(one, cv + l * l, dc);
    const float wl = rank_weight<L>(l) / (float)C;
#pragma unroll
    for (int a = 0; a < N; ++a) {
      const int k = l * l + a;
      ux[k] = wl * dx[a];
      vc[k] = wl * dc[a];
      t = fmaf(gv[k] * G[l], xv[k], t);
      p = fmaf(cv[k] * gv[k], G[l], p);
      q = fmaf(cv[k], ux[k], q);
    }
  });
  t = block_channel_sum(active ? t : 0.f, part);
  p = block_channel_sum(active ? p : 0.f, part);
  q = block_channel_sum(active ? q : 0.f, part);
  if (!active) return;
  const float s = scale[node];
  const float h3 = 0.5f * s * s * s;  // s^3 / 2
  const float cu = -h3 * p + 1.5f * h3 * s * s * t * q;  // -s^3/2 p + 3/4 s^5 t q
  static_for<L + 1>([&](auto lc) {
    constexpr int l = decltype(lc)::value;
    float dg = 0.f;
#pragma unroll
    for (int a = 0; a < 2 * l + 1; ++a) {
      const int k = l * l + a;
      const int64_t o = base + (int64_t)k * C + f;
      if (d_go) d_go[o] = G[l] * (s * cv[k] - h3 * q * xv[k]);
      if (d_x) d_x[o] = cu * ux[k] - h3 * q * gv[k] * G[l] - h3 * t * vc[k];
      dg += gv[k] * (s * cv[k] - h3 * q * xv[k]);
    }
    if (d_g_part) d_g_part[(node * (L + 1) + l) * C + f] = dg;
  });
}

template <int L>
int launch_rms_dbwd(int64_t n, int C, const float* go, const float* x, const float* g, const float* scale,
                    const float* cc, float* d_go, float* d_x, float* d_g_part, hipStream_t s) {
  const int threads = ((C + 63) / 64) * 64;
  hipLaunchKernelGGL(rms_norm_dbwd_kernel<L>, dim3((unsigned)n), dim3(threads), 0, s, n, C, go, x, g, scale, cc,
                     d_go, d_x, d_g_part);
  FC_LAUNCH_CHECK();
  return FC_OK;
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
#if FC_KERNEL_L_MAX >= 4
    case 4: return launch_rms<4>(bwd, n, C, go, x, g, eps, out, scale, s);
#endif
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

extern "C" int fc_rms_norm_dbwd(int64_t n, int32_t l_max, int32_t C, const float* grad_out, const float* x,
                                const float* weight, const float* scale, const float* cot, float* d_grad_out,
                                float* d_x, float* d_weight_part, void* stream) {
  if (n < 0 || C < 1) return FC_ERR_SHAPE;
  if (l_max < 0) return FC_ERR_BAD_DESC;
  if (l_max > FC_KERNEL_L_MAX) return FC_ERR_UNSUPPORTED_L;
  if (C > 256 || n > 0x7fffffff) return FC_ERR_SHAPE;
  if (n == 0) return FC_OK;
  if (!grad_out || !x || !weight || !scale || !cot) return FC_ERR_NULL;
  hipStream_t s = (hipStream_t)stream;
  switch (l_max) {
    case 0: return launch_rms_dbwd<0>(n, C, grad_out, x, weight, scale, cot, d_grad_out, d_x, d_weight_part, s);
    case 1: return launch_rms_dbwd<1>(n, C, grad_out, x, weight, scale, cot, d_grad_out, d_x, d_weight_part, s);
    case 2: return launch_rms_dbwd<2>(n, C, grad_out, x, weight, scale, cot, d_grad_out, d_x, d_weight_part, s);
    case 3: return launch_rms_dbwd<3>(n, C, grad_out, x, weight, scale, cot, d_grad_out, d_x, d_weight_part, s);
#if FC_KERNEL_L_MAX >= 4
    case 4: return launch_rms_dbwd<4>(n, C, grad_out, x, weight, scale, cot, d_grad_out, d_x, d_weight_part, s);
#endif
  }
  return FC_ERR_UNSUPPORTED_L;
}
