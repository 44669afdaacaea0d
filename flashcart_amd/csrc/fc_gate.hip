// Rank-wise gating of equivariant features (reference src/flashcart/nn/layers.py:609-635,
// EquivariantGatedLayer.forward between value_linear and output_linear):
//   gate[n, l, c]        = act(pre[n, l, c])      act: identity, or 1.8462285453386054 * sigmoid
//   out[n, (l, a), c]    = values[n, (l, a), c] * gate[n, l, c]
// One pass instead of activation + index_select + multiply, and one pass for both
// gradients in the backward:
//   grad_values[n,(l,a),c] = grad_out * gate[n, l, c]
//   grad_pre[n, l, c]      = act'(pre) * sum_a grad_out[n,(l,a),c] * values[n,(l,a),c]
// Thread per (node, channel); ranks and components in registers.
#include "fc_common.h"
#include "fc_tp_paths.h"  // FC_KERNEL_L_MAX

namespace fc {

constexpr float kSigmoidScale = 1.8462285453386054f;  // RescaledSigmoidLayer, src/flashcart/nn/layers.py:59

__device__ __forceinline__ float gate_act(float p, int act, float* deriv) {
  if (act == 0) {
    *deriv = 1.f;
    return p;
  }
  const float s = 1.0f / (1.0f + __expf(-p));
  *deriv = kSigmoidScale * s * (1.0f - s);
  return kSigmoidScale * s;
}

__global__ void __launch_bounds__(256) gate_fwd_kernel(int64_t n, int l_max, int C, const float* __restrict__ values,
                                                       const float* __restrict__ pre, int act,
                                                       float* __restrict__ out) {
  const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (t >= n * C) return;
  const int64_t node = t / C;
  const int c = (int)(t - node * C);
  const int D = (l_max + 1) * (l_max + 1);
  const float* v = values + node * (int64_t)D * C + c;
  float* o = out + node * (int64_t)D * C + c;
  const float* p = pre + node * (int64_t)(l_max + 1) * C + c;
  for (int l = 0; l <= l_max; ++l) {
    float d;
    const float gl = gate_act(p[(int64_t)l * C], act, &d);
    for (int a = l * l; a < (l + 1) * (l + 1); ++a) o[(int64_t)a * C] = v[(int64_t)a * C] * gl;
  }
}

__global__ void __launch_bounds__(256) gate_bwd_kernel(int64_t n, int l_max, int C, const float* __restrict__ go,
                                                       const float* __restrict__ values,
                                                       const float* __restrict__ pre, int act,
                                                       float* __restrict__ g_values, float* __restrict__ g_pre) {
  const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (t >= n * C) return;
  const int64_t node = t / C;
  const int c = (int)(t - node * C);
  const int D = (l_max + 1) * (l_max + 1);
  const int64_t base = node * (int64_t)D * C + c;
  const float* p = pre + node * (int64_t)(l_max + 1) * C + c;
  for (int l = 0; l <= l_max; ++l) {
    float d;
    const float gl = gate_act(p[(int64_t)l * C], act, &d);
    float s = 0.f;
    for (int a = l * l; a < (l + 1) * (l + 1); ++a) {
      const float gv = go[base + (int64_t)a * C];
      s = fmaf(gv, values[base + (int64_t)a * C], s);
      if (g_values) g_values[base + (int64_t)a * C] = gv * gl;
    }
    if (g_pre) g_pre[node * (int64_t)(l_max + 1) * C + (int64_t)l * C + c] = s * d;
  }
}

// Second derivative (force-loss training): the backward of gate_bwd. With A = act(pre),
// cotangents cv (of grad_values) and cp (of grad_pre; either may be absent):
//   d grad_out = cv A + cp A' values,  d values = cp A' grad_out,
//   d pre = A' sum_a cv grad_out + cp A'' sum_a grad_out values.
__global__ void __launch_bounds__(256) gate_dbwd_kernel(int64_t n, int l_max, int C, const float* __restrict__ go,
                                                        const float* __restrict__ values,
                                                        const float* __restrict__ pre, int act,
                                                        const float* __restrict__ cv, const float* __restrict__ cp,
                                                        float* __restrict__ d_go, float* __restrict__ d_values,
                                                        float* __restrict__ d_pre) {
  const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (t >= n * C) return;
  const int64_t node = t / C;
  const int c = (int)(t - node * C);
  const int D = (l_max + 1) * (l_max + 1);
  const int64_t base = node * (int64_t)D * C + c;
  const int64_t pbase = node * (int64_t)(l_max + 1) * C + c;
  for (int l = 0; l <= l_max; ++l) {
    float d1;
    const float A = gate_act(pre[pbase + (int64_t)l * C], act, &d1);
    // A'' = k s (1 - s)(1 - 2 s) = A' (1 - 2 s) with s = A / k for the rescaled sigmoid
    const float d2 = act == 0 ? 0.f : d1 * (1.0f - 2.0f * A / kSigmoidScale);
    const float cpl = cp ? cp[pbase + (int64_t)l * C] : 0.f;
    float s_cg = 0.f, s_gv = 0.f;
    for (int a = l * l; a < (l + 1) * (l + 1); ++a) {
      const int64_t k = base + (int64_t)a * C;
      const float g = go[k], v = values[k];
      const float cva = cv ? cv[k] : 0.f;
      s_cg = fmaf(cva, g, s_cg);
      s_gv = fmaf(g, v, s_gv);
      if (d_go) d_go[k] = fmaf(cva, A, cpl * d1 * v);
      if (d_values) d_values[k] = cpl * d1 * g;
    }
    if (d_pre) d_pre[pbase + (int64_t)l * C] = fmaf(d1, s_cg, cpl * d2 * s_gv);
  }
}

}  // namespace fc

using namespace fc;

extern "C" int fc_gate_fwd(int64_t n, int32_t l_max, int32_t C, const float* values, const float* pre, int32_t act,
                           float* out, void* stream) {
  if (n < 0 || C < 1 || act < 0 || act > 1) return FC_ERR_BAD_DESC;
  if (l_max < 0 || l_max > FC_KERNEL_L_MAX) return FC_ERR_UNSUPPORTED_L;
  if (n == 0) return FC_OK;
  if (!values || !pre || !out) return FC_ERR_NULL;
  const int64_t total = n * C;
  hipLaunchKernelGGL(gate_fwd_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, (hipStream_t)stream, n,
                     l_max, C, values, pre, act, out);
  FC_LAUNCH_CHECK();
  return FC_OK;
}

extern "C" int fc_gate_bwd(int64_t n, int32_t l_max, int32_t C, const float* grad_out, const float* values,
                           const float* pre, int32_t act, float* grad_values, float* grad_pre, void* stream) {
  if (n < 0 || C < 1 || act < 0 || act > 1) return FC_ERR_BAD_DESC;
  if (l_max < 0 || l_max > FC_KERNEL_L_MAX) return FC_ERR_UNSUPPORTED_L;
  if (n == 0) return FC_OK;
  if (!grad_out || !values || !pre) return FC_ERR_NULL;
  const int64_t total = n * C;
  hipLaunchKernelGGL(gate_bwd_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, (hipStream_t)stream, n,
                     l_max, C, grad_out, values, pre, act, grad_values, grad_pre);
  FC_LAUNCH_CHECK();
  return FC_OK;
}

extern "C" int fc_gate_dbwd(int64_t n, int32_t l_max, int32_t C, const float* grad_out, const float* values,
                            const float* pre, int32_t act, const float* cot_values, const float* cot_pre,
                            float* d_grad_out, float* d_values, float* d_pre, void* stream) {
  if (n < 0 || C < 1 || act < 0 || act > 1) return FC_ERR_BAD_DESC;
  if (l_max < 0 || l_max > FC_KERNEL_L_MAX) return FC_ERR_UNSUPPORTED_L;
  if (n == 0) return FC_OK;
  if (!grad_out || !values || !pre) return FC_ERR_NULL;
  const int64_t total = n * C;
  hipLaunchKernelGGL(gate_dbwd_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, (hipStream_t)stream, n,
                     l_max, C, grad_out, values, pre, act, cot_values, cot_pre, d_grad_out, d_values, d_pre);
  FC_LAUNCH_CHECK();
  return FC_OK;
}
