// Eq. (1) expansion, radial bases, cutoff envelope and the fused edge-geometry pass.
//
// Edge-parallel, one thread per edge: each edge reads 12-36 B and writes
// (L+1)^2 + n_radial + 1 floats, so these kernels are HBM/launch bound; the fusion
// removes the separate gather / norm / normalise / expand / basis / cutoff passes
// (and their intermediates) of the reference forward (src/flashcart/model/
// flashcart.py:268-284) and the matching autograd chain in the backward.
#include "fc_common.h"
#include "fc_expand_poly.h"  // Expand<0..FC_KERNEL_L_MAX>, generated for the build's rank limit

namespace fc {

constexpr float kMinEdgeLength = 1.0e-4f;  // MIN_EDGE_LENGTH, src/flashcart/model/flashcart.py:22
constexpr int kMaxRadial = 32;

template <int L>
__device__ __forceinline__ void expand_all(float x, float y, float z, float* out) {
  static_for<L + 1>([&](auto ic) {
    constexpr int l = decltype(ic)::value;
    Expand<l>::fwd(x, y, z, out + l * l);
  });
}

template <int L>
__device__ __forceinline__ void expand_all_bwd(float x, float y, float z, const float* g, float* gv) {
  static_for<L + 1>([&](auto ic) {
    constexpr int l = decltype(ic)::value;
    if constexpr (l > 0) Expand<l>::bwd(x, y, z, g + l * l, gv);
  });
}

// ---------------------------------------------------------------------------
// Radial basis + envelope (value and derivative with respect to d), following
// src/flashcart/nn/radial.py. The derivative conventions are those of PyTorch
// autograd on the reference expressions (clamp passes the gradient on the closed
// interval, torch.sinc' = 0 at 0).
// ---------------------------------------------------------------------------
struct RadialParams {
  int basis, n_radial, poly_order;
  float r_min, r_max;
};

__device__ __forceinline__ void radial_eval(const RadialParams& p, float d, float* feats, float* dfeats) {
  const int n = p.n_radial;
  if (p.basis == FC_BASIS_BESSEL) {
    // sqrt(2/r_max) * w_n * sinc(w_n d / pi), w_n = n pi / r_max
    const float pre = sqrtf(2.0f / p.r_max);
    for (int k = 0; k < n; ++k) {
      const float w = (float)M_PI / p.r_max * (float)(k + 1);
      const float u = d * w / (float)M_PI;  // argument of torch.sinc
      const float pu = (float)M_PI * u;
      float s, ds;
      if (fabsf(pu) < 0.05f) {
        // Taylor series of sin(t)/t and of pi * d/dt[sin(t)/t] (the direct forms cancel for small t)
        const float t2 = pu * pu;
        s = 1.0f - t2 * (1.0f / 6.0f) * (1.0f - t2 * (1.0f / 20.0f));
        ds = (float)M_PI * pu * (-1.0f / 3.0f + t2 * (1.0f / 30.0f) * (1.0f - t2 * (1.0f / 28.0f)));
      } else {
        const float sn = sinf(pu), cs = cosf(pu);
        s = sn / pu;
        ds = (pu * cs - sn) / (pu * u);
      }
      feats[k] = pre * w * s;
      if (dfeats) dfeats[k] = pre * w * ds * (w / (float)M_PI);
    }
    return;
  }
  // Chebyshev T_k of x(t), t = (d - r_min) / (r_max - r_min)
  const float span = p.r_max - p.r_min;
  const float t = (d - p.r_min) / span;
  float x, dx;
  if (p.basis == FC_BASIS_CHEBYSHEV_COSINE) {
    x = cosf(t * (float)M_PI);
    dx = -sinf(t * (float)M_PI) * (float)M_PI / span;
  } else {
    x = 2.0f * t - 1.0f;
    dx = 2.0f / span;
  }
  float tm2 = 1.0f, tm1 = x, dm2 = 0.0f, dm1 = 1.0f;  // T_{k-2}, T_{k-1} and d/dx
  feats[0] = 1.0f;
  if (dfeats) dfeats[0] = 0.0f;
  if (n > 1) {
    feats[1] = x;
    if (dfeats) dfeats[1] = dx;
  }
  for (int k = 2; k < n; ++k) {
    const float tk = 2.0f * x * tm1 - tm2;
    const float dk = 2.0f * tm1 + 2.0f * x * dm1 - dm2;
    feats[k] = tk;
    if (dfeats) dfeats[k] = dk * dx;
    tm2 = tm1; tm1 = tk; dm2 = dm1; dm1 = dk;
  }
}

// Values only (the forward kernels). The Bessel functions take sin(pi u) from sinpif: the same
// quantity as sinf(pi * u) without a general range reduction (the product pi * u, up to n_radial pi,
// sends sinf down its large-argument path).
// NR > 0: n_radial == NR at compile time (the loop unrolls, the values stay in registers).
template <int NR = 0>
__device__ __forceinline__ void radial_feats(const RadialParams& p, float d, float* feats) {
  const int n = NR > 0 ? NR : p.n_radial;
  if (p.basis != FC_BASIS_BESSEL) {  // Chebyshev T_k of x(t): the recurrence of radial_eval
    const float t = (d - p.r_min) / (p.r_max - p.r_min);
    const float x = p.basis == FC_BASIS_CHEBYSHEV_COSINE ? cosf(t * (float)M_PI) : 2.0f * t - 1.0f;
    float tm2 = 1.0f, tm1 = x;
    feats[0] = 1.0f;
    if (n > 1) feats[1] = x;
#pragma unroll
    for (int k = 2; k < n; ++k) {
      const float tk = 2.0f * x * tm1 - tm2;
      feats[k] = tk;
      tm2 = tm1;
      tm1 = tk;
    }
    return;
  }
  const float pre = sqrtf(2.0f / p.r_max);
#pragma unroll
  for (int k = 0; k < n; ++k) {
    const float w = (float)M_PI / p.r_max * (float)(k + 1);
    const float u = d * w / (float)M_PI;  // argument of torch.sinc
    const float pu = (float)M_PI * u;
    float sc;
    if (fabsf(pu) < 0.05f) {
      const float t2 = pu * pu;
      sc = 1.0f - t2 * (1.0f / 6.0f) * (1.0f - t2 * (1.0f / 20.0f));
    } else {
      sc = sinpif(u) / pu;
    }
    feats[k] = pre * w * sc;
  }
}

__device__ __forceinline__ float envelope_eval(const RadialParams& p, float d, float* denv) {
  // clamp(d, 0); t = d / r_max; f(t) = 1 - c1 t^p + c2 t^(p+1) - c3 t^(p+2); * [d < r_max]; clamp [0, 1].
  // f has a triple root at t = 1 and is evaluated in the exactly equal factored form
  //   f(t) = (1-t)^3 g(t),  g(t) = sum_{k<p} C(k+2,2) t^k,
  // which avoids the cancellation of the expanded form near the cutoff (terms ~50 summing to ~1e-4).
  const int po = p.poly_order;
  const float dc = fmaxf(d, 0.0f);
  const float t = dc / p.r_max;
  float g = 0.0f, dg = 0.0f;  // Horner for g and g'
  for (int k = po - 1; k >= 0; --k) {
    dg = fmaf(dg, t, g);
    g = fmaf(g, t, 0.5f * (float)((k + 1) * (k + 2)));
  }
  const float s = 1.0f - t;
  const float env = s * s * s * g;
  const float mask = dc < p.r_max ? 1.0f : 0.0f;
  const float v = env * mask;
  const float out = fminf(fmaxf(v, 0.0f), 1.0f);
  if (denv) {
    const float de = s * s * (s * dg - 3.0f * g) / p.r_max;
    const bool pass = (v >= 0.0f && v <= 1.0f) && (d >= 0.0f);
    *denv = pass ? mask * de : 0.0f;
  }
  return out;
}

__host__ __device__ inline RadialParams radial_params(const fc_radial_desc& d) {
  return RadialParams{d.basis, d.n_radial, d.poly_order, d.r_min, d.r_max};
}

// ---------------------------------------------------------------------------
// Irreps (Eq. 1 on given unit vectors)
// ---------------------------------------------------------------------------
template <int L>
__global__ void irreps_fwd_kernel(int64_t n, const float* __restrict__ x, float* __restrict__ out) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  float o[ncomp(L)];
  expand_all<L>(x[3 * i], x[3 * i + 1], x[3 * i + 2], o);
#pragma unroll
  for (int k = 0; k < ncomp(L); ++k) out[i * ncomp(L) + k] = o[k];
}

template <int L>
__global__ void irreps_bwd_kernel(int64_t n, const float* __restrict__ g, const float* __restrict__ x,
                                  float* __restrict__ gx) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  float gi[ncomp(L)];
#pragma unroll
  for (int k = 0; k < ncomp(L); ++k) gi[k] = g[i * ncomp(L) + k];
  float v[3] = {0.f, 0.f, 0.f};
  expand_all_bwd<L>(x[3 * i], x[3 * i + 1], x[3 * i + 2], gi, v);
  gx[3 * i] = v[0];
  gx[3 * i + 1] = v[1];
  gx[3 * i + 2] = v[2];
}

__global__ void radial_fwd_kernel(RadialParams p, int64_t n, const float* __restrict__ d,
                                  float* __restrict__ feats, float* __restrict__ env) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  const float di = d[i];
  if (feats && p.basis != FC_BASIS_NONE) {
    float f[kMaxRadial];
    radial_feats(p, di, f);
    for (int k = 0; k < p.n_radial; ++k) feats[i * p.n_radial + k] = f[k];
  }
  if (env) env[i] = envelope_eval(p, di, nullptr);
}

__global__ void radial_bwd_kernel(RadialParams p, int64_t n, const float* __restrict__ d,
                                  const float* __restrict__ gf, const float* __restrict__ ge,
                                  float* __restrict__ gd) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  const float di = d[i];
  float acc = 0.f;
  if (gf && p.basis != FC_BASIS_NONE) {
    float f[kMaxRadial], df[kMaxRadial];
    radial_eval(p, di, f, df);
    for (int k = 0; k < p.n_radial; ++k) acc = fmaf(gf[i * p.n_radial + k], df[k], acc);
  }
  if (ge) {
    float de;
    envelope_eval(p, di, &de);
    acc = fmaf(ge[i], de, acc);
  }
  gd[i] = acc;
}

// ---------------------------------------------------------------------------
// Fused edge geometry
// ---------------------------------------------------------------------------
__device__ __forceinline__ void edge_vector(int64_t e, const float* pos, const float* shift, const int32_t* ii,
                                            const int32_t* jj, const float* vectors, float* v) {
  if (pos) {
    const int64_t i = ii[e], j = jj[e];
#pragma unroll
    for (int k = 0; k < 3; ++k) v[k] = pos[3 * j + k] - pos[3 * i + k] + (shift ? shift[3 * e + k] : 0.f);
  } else {
#pragma unroll
    for (int k = 0; k < 3; ++k) v[k] = vectors[3 * e + k];
  }
}

// Rows of W floats per edge (the block's edges e0 .. e0 + nb - 1) written through LDS: each thread
// puts its row at stride W + 1 (odd: the row writes hit distinct banks), then the block stores the
// nb * W floats as one contiguous run, consecutive lanes on consecutive floats. A row per thread
// written straight to memory would be W stores whose lanes sit W floats apart.
constexpr int kEdgeBlock = 256;

// W <= MAXW; the row is a register array, read at compile-time indices only.
template <int MAXW>
__device__ __forceinline__ void block_store_rows(float* st, const float (&row)[MAXW], int W, bool active, int64_t e0,
                                                 int nb, float* __restrict__ out) {
  const int t = threadIdx.x;
  if (active) {
#pragma unroll
    for (int k = 0; k < MAXW; ++k)
      if (k < W) st[t * (W + 1) + k] = row[k];
  }
  __syncthreads();
  float* o = out + e0 * W;
  for (int idx = t; idx < nb * W; idx += kEdgeBlock) {
    const int r = idx / W;
    o[idx] = st[r * (W + 1) + (idx - r * W)];
  }
  __syncthreads();  // the buffer is reused by the next call
}

// NR > 0: exactly NR radial functions (the loops over them unroll); NR == 0: any count.
template <int L, int NR>
__global__ void __launch_bounds__(kEdgeBlock) edge_fwd_kernel(RadialParams p, int64_t n, const float* __restrict__ pos,
                                                            const float* __restrict__ shift,
                                                            const int32_t* __restrict__ ii,
                                                            const int32_t* __restrict__ jj,
                                                            const float* __restrict__ vectors,
                                                            float* __restrict__ attrs, float* __restrict__ feats,
                                                            float* __restrict__ env) {
  extern __shared__ float st[];  // kEdgeBlock x (widest row + 1) floats, sized at launch
  const int64_t e0 = (int64_t)blockIdx.x * kEdgeBlock;
  const int64_t e = e0 + threadIdx.x;
  const bool active = e < n;  // no early return: every thread takes part in the block stores
  const int nb = n - e0 < kEdgeBlock ? (int)(n - e0) : kEdgeBlock;
  float v[3] = {1.f, 0.f, 0.f};
  if (active) edge_vector(e, pos, shift, ii, jj, vectors, v);
  const float d = sqrtf(v[0] * v[0] + v[1] * v[1] + v[2] * v[2]);
  const float inv = 1.0f / fmaxf(d, kMinEdgeLength);
  if (attrs) {
    float o[ncomp(L)];
    expand_all<L>(v[0] * inv, v[1] * inv, v[2] * inv, o);
    block_store_rows(st, o, ncomp(L), active, e0, nb, attrs);
  }
  if (feats && p.basis != FC_BASIS_NONE) {
    if constexpr (NR > 0) {
      float f[NR];
      radial_feats<NR>(p, d, f);
      block_store_rows(st, f, NR, active, e0, nb, feats);
    } else {
      float f[kMaxRadial];
      radial_feats(p, d, f);
      block_store_rows(st, f, p.n_radial, active, e0, nb, feats);
    }
  }
  if (env && active) env[e] = p.poly_order > 0 ? envelope_eval(p, d, nullptr) : 1.0f;
}

template <int L>
__global__ void edge_bwd_kernel(RadialParams p, int64_t n, const float* __restrict__ pos,
                                const float* __restrict__ shift, const int32_t* __restrict__ ii,
                                const int32_t* __restrict__ jj, const float* __restrict__ vectors,
                                const float* __restrict__ ga, const float* __restrict__ gf,
                                const float* __restrict__ ge, float* __restrict__ gvec) {
  const int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (e >= n) return;
  float v[3];
  edge_vector(e, pos, shift, ii, jj, vectors, v);
  const float d = sqrtf(v[0] * v[0] + v[1] * v[1] + v[2] * v[2]);
  const float dcl = fmaxf(d, kMinEdgeLength);
  const float inv = 1.0f / dcl;
  const float r[3] = {v[0] * inv, v[1] * inv, v[2] * inv};
  float gr[3] = {0.f, 0.f, 0.f};
  if (ga) {
    float g[ncomp(L)];
#pragma unroll
    for (int k = 0; k < ncomp(L); ++k) g[k] = ga[e * ncomp(L) + k];
    expand_all_bwd<L>(r[0], r[1], r[2], g, gr);
  }
  // direction = v / clamp_min(d, eps): dL/dv += gr / dcl, dL/dd -= (gr . v) / dcl^2 when d >= eps
  float gd = 0.f;
  if (gf && p.basis != FC_BASIS_NONE) {
    float f[kMaxRadial], df[kMaxRadial];
    radial_eval(p, d, f, df);
    for (int k = 0; k < p.n_radial; ++k) gd = fmaf(gf[e * p.n_radial + k], df[k], gd);
  }
  if (ge && p.poly_order > 0) {
    float de;
    envelope_eval(p, d, &de);
    gd = fmaf(ge[e], de, gd);
  }
  if (d >= kMinEdgeLength) gd -= (gr[0] * v[0] + gr[1] * v[1] + gr[2] * v[2]) * inv * inv;
  const float nd = d > 0.f ? gd / d : 0.f;  // d|v|/dv = v / |v|
#pragma unroll
  for (int k = 0; k < 3; ++k) gvec[3 * e + k] = gr[k] * inv + nd * v[k];
}

// ---------------------------------------------------------------------------
// Second derivatives (force-loss training): the backward of the edge-geometry backward.
// ---------------------------------------------------------------------------
template <int L>
__device__ __forceinline__ void expand_all_jvp(float x, float y, float z, const float* du, float* dt) {
  static_for<L + 1>([&](auto ic) {
    constexpr int l = decltype(ic)::value;
    Expand<l>::jvp(x, y, z, du, dt + l * l);
  });
}

template <int L>
__device__ __forceinline__ void expand_all_hvp(float x, float y, float z, const float* g, const float* du, float* h) {
  static_for<L + 1>([&](auto ic) {
    constexpr int l = decltype(ic)::value;
    if constexpr (l > 1) Expand<l>::hvp(x, y, z, g + l * l, du, h);
  });
}

// Backward of irreps_bwd (gx = J(x)^T g): along a cotangent v of gx,
//   d/dg = J(x) v            (the directional derivative of every component),
//   d/dx = sum_a g_a H_a(x) v (Hessian-vector products of the components).
// Either output may be NULL (not wanted).
template <int L>
__global__ void irreps_dbwd_kernel(int64_t n, const float* __restrict__ g, const float* __restrict__ x,
                                   const float* __restrict__ v, float* __restrict__ d_g, float* __restrict__ d_x) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  const float x0 = x[3 * i], x1 = x[3 * i + 1], x2 = x[3 * i + 2];
  const float du[3] = {v[3 * i], v[3 * i + 1], v[3 * i + 2]};
  if (d_g) {
    float dt[ncomp(L)];
    expand_all_jvp<L>(x0, x1, x2, du, dt);
#pragma unroll
    for (int k = 0; k < ncomp(L); ++k) d_g[i * ncomp(L) + k] = dt[k];
  }
  if (d_x) {
    float gi[ncomp(L)];
#pragma unroll
    for (int k = 0; k < ncomp(L); ++k) gi[k] = g[i * ncomp(L) + k];
    float h[3] = {0.f, 0.f, 0.f};
    expand_all_hvp<L>(x0, x1, x2, gi, du, h);
    d_x[3 * i] = h[0];
    d_x[3 * i + 1] = h[1];
    d_x[3 * i + 2] = h[2];
  }
}

// First and second derivatives of the radial basis with respect to d.
__device__ __forceinline__ void radial_d12(const RadialParams& p, float d, float* df, float* d2f) {
  const int n = p.n_radial;
  if (p.basis == FC_BASIS_BESSEL) {
    // f = sqrt(2/r_max) sin(w d) / d = pre w sinc(t), t = w d: f' = pre w^2 sinc'(t), f'' = pre w^3 sinc''(t)
    const float pre = sqrtf(2.0f / p.r_max);
    for (int k = 0; k < n; ++k) {
      const float w = (float)M_PI / p.r_max * (float)(k + 1);
      const float t = w * d;
      float s1, s2;
      if (fabsf(t) < 0.05f) {  // Taylor series (the closed forms cancel for small t)
        const float t2 = t * t;
        s1 = t * (-1.0f / 3.0f + t2 * (1.0f / 30.0f));
        s2 = -1.0f / 3.0f + t2 * (1.0f / 10.0f);
      } else {
        const float sn = sinf(t), cs = cosf(t), it = 1.0f / t;
        s1 = (cs - sn * it) * it;
        s2 = ((2.0f * it * it - 1.0f) * sn - 2.0f * cs * it) * it;
      }
      df[k] = pre * w * w * s1;
      d2f[k] = pre * w * w * w * s2;
    }
    return;
  }
  // Chebyshev T_k(x(t)), t = (d - r_min) / span: F' = T_k' x', F'' = T_k'' x'^2 + T_k' x''
  const float span = p.r_max - p.r_min;
  const float t = (d - p.r_min) / span;
  float x, x1, x2;
  if (p.basis == FC_BASIS_CHEBYSHEV_COSINE) {
    const float a = t * (float)M_PI;
    x = cosf(a);
    x1 = -sinf(a) * (float)M_PI / span;
    x2 = -x * (float)(M_PI * M_PI) / (span * span);
  } else {
    x = 2.0f * t - 1.0f;
    x1 = 2.0f / span;
    x2 = 0.0f;
  }
  float tm2 = 1.0f, tm1 = x, dm2 = 0.0f, dm1 = 1.0f, sm2 = 0.0f, sm1 = 0.0f;  // T, T', T'' of k-2, k-1
  df[0] = 0.0f;
  d2f[0] = 0.0f;
  if (n > 1) {
    df[1] = x1;
    d2f[1] = x2;
  }
  for (int k = 2; k < n; ++k) {
    const float tk = 2.0f * x * tm1 - tm2;
    const float dk = 2.0f * tm1 + 2.0f * x * dm1 - dm2;
    const float sk = 4.0f * dm1 + 2.0f * x * sm1 - sm2;
    df[k] = dk * x1;
    d2f[k] = sk * x1 * x1 + dk * x2;
    tm2 = tm1; tm1 = tk; dm2 = dm1; dm1 = dk; sm2 = sm1; sm1 = sk;
  }
}

// First and second derivatives of the envelope with respect to d (zero where the clamps or
// the cutoff mask hold it constant, as the first derivative of envelope_eval).
__device__ __forceinline__ void envelope_d12(const RadialParams& p, float d, float* de, float* d2e) {
  const int po = p.poly_order;
  const float dc = fmaxf(d, 0.0f);
  const float t = dc / p.r_max;
  float g = 0.0f, dg = 0.0f, d2g = 0.0f;  // Horner for g, g', g''
  for (int k = po - 1; k >= 0; --k) {
    d2g = fmaf(d2g, t, 2.0f * dg);
    dg = fmaf(dg, t, g);
    g = fmaf(g, t, 0.5f * (float)((k + 1) * (k + 2)));
  }
  const float s = 1.0f - t;
  const float mask = dc < p.r_max ? 1.0f : 0.0f;
  const float v = s * s * s * g * mask;
  const bool pass = (v >= 0.0f && v <= 1.0f) && (d >= 0.0f);
  const float h = s * dg - 3.0f * g;  // P = s^3 g: dP/dt = s^2 h, d2P/dt2 = -2 s h + s^2 (s g'' - 4 g')
  *de = pass ? mask * s * s * h / p.r_max : 0.0f;
  *d2e = pass ? mask * (-2.0f * s * h + s * s * (s * d2g - 4.0f * dg)) / (p.r_max * p.r_max) : 0.0f;
}

// With the edge vector v, d = |v|, u = v / max(d, eps), a = dA/du^T g_attrs and
// s = g_feats . F'(d) + g_env P'(d), the first-order backward is
//   gvec = (a - (u.a) u) / d + s u   (d >= eps),   a / eps + s v / d   (0 < d < eps).
// Its derivative along the cotangent c of gvec gives d_vec (the Hessian-vector product of
// g . geometry), and the derivative of the geometry along c gives the gradients of the
// upstream gradients: d_g_attrs = dA/du du, d_g_feats = F'(d) dd, d_g_env = P'(d) dd.
template <int L>
__global__ void edge_dbwd_kernel(RadialParams p, int64_t n, const float* __restrict__ pos,
                                 const float* __restrict__ shift, const int32_t* __restrict__ ii,
                                 const int32_t* __restrict__ jj, const float* __restrict__ vectors,
                                 const float* __restrict__ ga, const float* __restrict__ gf,
                                 const float* __restrict__ ge, const float* __restrict__ cvec,
                                 float* __restrict__ d_ga, float* __restrict__ d_gf, float* __restrict__ d_ge,
                                 float* __restrict__ d_vec) {
  const int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (e >= n) return;
  float v[3];
  edge_vector(e, pos, shift, ii, jj, vectors, v);
  const float d = sqrtf(v[0] * v[0] + v[1] * v[1] + v[2] * v[2]);
  const bool big = d >= kMinEdgeLength;
  const float inv = 1.0f / fmaxf(d, kMinEdgeLength);
  const float u[3] = {v[0] * inv, v[1] * inv, v[2] * inv};
  const float c[3] = {cvec[3 * e], cvec[3 * e + 1], cvec[3 * e + 2]};
  const float dd = d > 0.f ? (v[0] * c[0] + v[1] * c[1] + v[2] * c[2]) / d : 0.f;  // tangent of d
  float du[3];  // tangent of u
#pragma unroll
  for (int k = 0; k < 3; ++k) du[k] = big ? (c[k] - dd * u[k]) * inv : c[k] * inv;
  float a[3] = {0.f, 0.f, 0.f}, da[3] = {0.f, 0.f, 0.f};
  if (ga) {
    float g[ncomp(L)];
#pragma unroll
    for (int k = 0; k < ncomp(L); ++k) g[k] = ga[e * ncomp(L) + k];
    expand_all_bwd<L>(u[0], u[1], u[2], g, a);
    expand_all_hvp<L>(u[0], u[1], u[2], g, du, da);
  }
  if (d_ga) {
    float dt[ncomp(L)];
    expand_all_jvp<L>(u[0], u[1], u[2], du, dt);
#pragma unroll
    for (int k = 0; k < ncomp(L); ++k) d_ga[e * ncomp(L) + k] = dt[k];
  }
  float s = 0.f, s2 = 0.f;
  if (p.basis != FC_BASIS_NONE && (gf || d_gf)) {
    float df[kMaxRadial], d2f[kMaxRadial];
    radial_d12(p, d, df, d2f);
    for (int k = 0; k < p.n_radial; ++k) {
      if (gf) {
        s = fmaf(gf[e * p.n_radial + k], df[k], s);
        s2 = fmaf(gf[e * p.n_radial + k], d2f[k], s2);
      }
      if (d_gf) d_gf[e * p.n_radial + k] = df[k] * dd;
    }
  }
  if (p.poly_order > 0 && (ge || d_ge)) {
    float de, d2e;
    envelope_d12(p, d, &de, &d2e);
    if (ge) {
      s = fmaf(ge[e], de, s);
      s2 = fmaf(ge[e], d2e, s2);
    }
    if (d_ge) d_ge[e] = de * dd;
  }
  if (!d_vec) return;
  float out[3];
  if (big) {
    const float ua = u[0] * a[0] + u[1] * a[1] + u[2] * a[2];
    const float dua = du[0] * a[0] + du[1] * a[1] + du[2] * a[2] + u[0] * da[0] + u[1] * da[1] + u[2] * da[2];
#pragma unroll
    for (int k = 0; k < 3; ++k)
      out[k] = (da[k] - dua * u[k] - ua * du[k]) * inv - (a[k] - ua * u[k]) * inv * inv * dd + s2 * dd * u[k] +
               s * du[k];
  } else if (d > 0.f) {
    const float id = 1.0f / d;
#pragma unroll
    for (int k = 0; k < 3; ++k) out[k] = da[k] * inv + (s2 * dd - s * dd * id) * id * v[k] + s * id * c[k];
  } else {
#pragma unroll
    for (int k = 0; k < 3; ++k) out[k] = da[k] * inv;
  }
#pragma unroll
  for (int k = 0; k < 3; ++k) d_vec[3 * e + k] = out[k];
}

template <template <int> class K, class... Args>
int launch_by_l(int l, int64_t n, hipStream_t s, Args... args) {
  if (n == 0) return FC_OK;
  const int bs = 256;
  dim3 grid((unsigned)((n + bs - 1) / bs)), block(bs);
  switch (l) {
    case 0: hipLaunchKernelGGL(K<0>::fn, grid, block, 0, s, n, args...); break;
    case 1: hipLaunchKernelGGL(K<1>::fn, grid, block, 0, s, n, args...); break;
    case 2: hipLaunchKernelGGL(K<2>::fn, grid, block, 0, s, n, args...); break;
    case 3: hipLaunchKernelGGL(K<3>::fn, grid, block, 0, s, n, args...); break;
#if FC_KERNEL_L_MAX >= 4
    case 4: hipLaunchKernelGGL(K<4>::fn, grid, block, 0, s, n, args...); break;
#endif
    default: return FC_ERR_UNSUPPORTED_L;
  }
  FC_LAUNCH_CHECK();
  return FC_OK;
}

template <int L> struct IrrepsFwd { static constexpr auto fn = irreps_fwd_kernel<L>; };
template <int L> struct IrrepsBwd { static constexpr auto fn = irreps_bwd_kernel<L>; };
template <int L> struct IrrepsDbwd { static constexpr auto fn = irreps_dbwd_kernel<L>; };

static int check_radial(const fc_radial_desc* d) {
  if (!d) return FC_ERR_NULL;
  if (d->basis < 0 || d->basis > FC_BASIS_NONE) return FC_ERR_BAD_DESC;
  if (d->basis != FC_BASIS_NONE && (d->n_radial < 1 || d->n_radial > kMaxRadial)) return FC_ERR_BAD_DESC;
  if (d->poly_order != 0 && d->poly_order < 2) return FC_ERR_BAD_DESC;
  if (!(d->r_max > d->r_min) || !(d->r_max > 0.f)) return FC_ERR_BAD_DESC;
  return FC_OK;
}

template <int L>
int launch_edge_fwd(const RadialParams& p, int64_t n, const float* pos, const float* shift, const int32_t* ii,
                    const int32_t* jj, const float* vec, float* attrs, float* feats, float* env, hipStream_t s) {
  const int bs = kEdgeBlock;
  int w = attrs ? ncomp(L) : 0;
  if (feats && p.basis != FC_BASIS_NONE && p.n_radial > w) w = p.n_radial;
  const size_t lds = sizeof(float) * (size_t)kEdgeBlock * (size_t)(w + 1);
  if (p.basis != FC_BASIS_NONE && p.n_radial == 8)  // the packaged default count
    hipLaunchKernelGGL((edge_fwd_kernel<L, 8>), dim3((unsigned)((n + bs - 1) / bs)), dim3(bs), lds, s, p, n, pos,
                       shift, ii, jj, vec, attrs, feats, env);
  else
    hipLaunchKernelGGL((edge_fwd_kernel<L, 0>), dim3((unsigned)((n + bs - 1) / bs)), dim3(bs), lds, s, p, n, pos,
                       shift, ii, jj, vec, attrs, feats, env);
  FC_LAUNCH_CHECK();
  return FC_OK;
}

template <int L>
int launch_edge_bwd(const RadialParams& p, int64_t n, const float* pos, const float* shift, const int32_t* ii,
                    const int32_t* jj, const float* vec, const float* ga, const float* gf, const float* ge,
                    float* gvec, hipStream_t s) {
  const int bs = 256;
  hipLaunchKernelGGL(edge_bwd_kernel<L>, dim3((unsigned)((n + bs - 1) / bs)), dim3(bs), 0, s, p, n, pos, shift,
                     ii, jj, vec, ga, gf, ge, gvec);
  FC_LAUNCH_CHECK();
  return FC_OK;
}

// x as an opaque value: the library builds with -ffp-contract=fast (pragmas ignored), and a
// product passed through here cannot be fused into an FMA with the sum that takes it.
__device__ __forceinline__ float rounded(float x) {
  asm volatile("" : "+v"(x));
  return x;
}

// Periodic translation of each edge, one thread per edge: out[e] = (S0 a + S1 b) + S2 c with
// (a, b, c) the rows of the edge's cell, each product and sum rounded on its own (no contraction),
// so the translation of -S is the exact negation of that of S. A structure index outside
// [0, n_cells) or a receiver outside [0, n_nodes) gives NaN rows.
__global__ void shift_vectors_kernel(int64_t n, int n_cells, const int64_t* __restrict__ shifts,
                                     const float* __restrict__ cell, const int32_t* __restrict__ idx_i,
                                     const int32_t* __restrict__ batch, int64_t n_nodes, float* __restrict__ out) {
  const int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (e >= n) return;
  int b = 0;
  if (n_cells > 1) {
    const int32_t i = idx_i[e];
    b = (i >= 0 && i < n_nodes) ? batch[i] : -1;
  }
  const float s0 = (float)shifts[3 * e], s1 = (float)shifts[3 * e + 1], s2 = (float)shifts[3 * e + 2];
  float* o = out + 3 * e;
  if (b < 0 || b >= n_cells) {
    o[0] = o[1] = o[2] = __builtin_nanf("");
    return;
  }
  const float* c = cell + 9 * (int64_t)b;
#pragma unroll
  for (int k = 0; k < 3; ++k)
    o[k] = (rounded(s0 * c[k]) + rounded(s1 * c[3 + k])) + rounded(s2 * c[6 + k]);
}

}  // namespace fc

using namespace fc;

extern "C" int fc_irreps_fwd(int64_t n, int32_t l_max, const float* x, float* out, void* stream) {
  if (n < 0) return FC_ERR_SHAPE;
  if (n > 0 && (!x || !out)) return FC_ERR_NULL;
  return launch_by_l<IrrepsFwd>(l_max, n, (hipStream_t)stream, x, out);
}

extern "C" int fc_irreps_bwd(int64_t n, int32_t l_max, const float* g, const float* x, float* gx, void* stream) {
  if (n < 0) return FC_ERR_SHAPE;
  if (n > 0 && (!g || !x || !gx)) return FC_ERR_NULL;
  return launch_by_l<IrrepsBwd>(l_max, n, (hipStream_t)stream, g, x, gx);
}

extern "C" int fc_irreps_dbwd(int64_t n, int32_t l_max, const float* g, const float* x, const float* v,
                              float* d_g, float* d_x, void* stream) {
  if (n < 0) return FC_ERR_SHAPE;
  if (n > 0 && (!x || !v || (d_x && !g))) return FC_ERR_NULL;
  if (!d_g && !d_x) return FC_OK;
  return launch_by_l<IrrepsDbwd>(l_max, n, (hipStream_t)stream, g, x, v, d_g, d_x);
}

extern "C" int fc_radial_fwd(const fc_radial_desc* desc, int64_t n, const float* d, float* feats, float* env,
                             void* stream) {
  int st = check_radial(desc);
  if (st != FC_OK) return st;
  if (n == 0) return FC_OK;
  if (!d) return FC_ERR_NULL;
  if (env && desc->poly_order == 0) return FC_ERR_BAD_DESC;
  const int bs = 256;
  hipLaunchKernelGGL(radial_fwd_kernel, dim3((unsigned)((n + bs - 1) / bs)), dim3(bs), 0, (hipStream_t)stream,
                     radial_params(*desc), n, d, feats, env);
  FC_LAUNCH_CHECK();
  return FC_OK;
}

extern "C" int fc_radial_bwd(const fc_radial_desc* desc, int64_t n, const float* d, const float* g_feats,
                             const float* g_env, float* grad_d, void* stream) {
  int st = check_radial(desc);
  if (st != FC_OK) return st;
  if (n == 0) return FC_OK;
  if (!d || !grad_d) return FC_ERR_NULL;
  if (g_env && desc->poly_order == 0) return FC_ERR_BAD_DESC;
  const int bs = 256;
  hipLaunchKernelGGL(radial_bwd_kernel, dim3((unsigned)((n + bs - 1) / bs)), dim3(bs), 0, (hipStream_t)stream,
                     radial_params(*desc), n, d, g_feats, g_env, grad_d);
  FC_LAUNCH_CHECK();
  return FC_OK;
}

extern "C" int fc_edge_geometry_fwd(const fc_edge_desc* desc, int64_t n, const float* pos, const float* shift,
                                    const int32_t* ii, const int32_t* jj, const float* vectors, float* attrs,
                                    float* feats, float* env, void* stream) {
  if (!desc) return FC_ERR_NULL;
  int st = check_radial(&desc->radial);
  if (st != FC_OK) return st;
  if (n == 0) return FC_OK;
  if (pos ? (!ii || !jj) : !vectors) return FC_ERR_NULL;
  const RadialParams p = radial_params(desc->radial);
  hipStream_t s = (hipStream_t)stream;
  switch (desc->l_max) {
    case 0: return launch_edge_fwd<0>(p, n, pos, shift, ii, jj, vectors, attrs, feats, env, s);
    case 1: return launch_edge_fwd<1>(p, n, pos, shift, ii, jj, vectors, attrs, feats, env, s);
    case 2: return launch_edge_fwd<2>(p, n, pos, shift, ii, jj, vectors, attrs, feats, env, s);
    case 3: return launch_edge_fwd<3>(p, n, pos, shift, ii, jj, vectors, attrs, feats, env, s);
#if FC_KERNEL_L_MAX >= 4
    case 4: return launch_edge_fwd<4>(p, n, pos, shift, ii, jj, vectors, attrs, feats, env, s);
#endif
  }
  return FC_ERR_UNSUPPORTED_L;
}

extern "C" int fc_edge_geometry_bwd(const fc_edge_desc* desc, int64_t n, const float* pos, const float* shift,
                                    const int32_t* ii, const int32_t* jj, const float* vectors,
                                    const float* ga, const float* gf, const float* ge, float* gvec,
                                    void* stream) {
  if (!desc) return FC_ERR_NULL;
  int st = check_radial(&desc->radial);
  if (st != FC_OK) return st;
  if (n == 0) return FC_OK;
  if (!gvec || (pos ? (!ii || !jj) : !vectors)) return FC_ERR_NULL;
  const RadialParams p = radial_params(desc->radial);
  hipStream_t s = (hipStream_t)stream;
  switch (desc->l_max) {
    case 0: return launch_edge_bwd<0>(p, n, pos, shift, ii, jj, vectors, ga, gf, ge, gvec, s);
    case 1: return launch_edge_bwd<1>(p, n, pos, shift, ii, jj, vectors, ga, gf, ge, gvec, s);
    case 2: return launch_edge_bwd<2>(p, n, pos, shift, ii, jj, vectors, ga, gf, ge, gvec, s);
    case 3: return launch_edge_bwd<3>(p, n, pos, shift, ii, jj, vectors, ga, gf, ge, gvec, s);
#if FC_KERNEL_L_MAX >= 4
    case 4: return launch_edge_bwd<4>(p, n, pos, shift, ii, jj, vectors, ga, gf, ge, gvec, s);
#endif
  }
  return FC_ERR_UNSUPPORTED_L;
}

extern "C" int fc_edge_geometry_dbwd(const fc_edge_desc* desc, int64_t n, const float* pos, const float* shift,
                                     const int32_t* ii, const int32_t* jj, const float* vectors,
                                     const float* ga, const float* gf, const float* ge, const float* cot_vec,
                                     float* d_ga, float* d_gf, float* d_ge, float* d_vec, void* stream) {
  if (!desc) return FC_ERR_NULL;
  int st = check_radial(&desc->radial);
  if (st != FC_OK) return st;
  if (desc->l_max < 0 || desc->l_max > FC_KERNEL_L_MAX) return FC_ERR_UNSUPPORTED_L;
  if (n == 0) return FC_OK;
  if (!cot_vec || (pos ? (!ii || !jj) : !vectors)) return FC_ERR_NULL;
  const RadialParams p = radial_params(desc->radial);
  const dim3 grid((unsigned)((n + 255) / 256)), block(256);
  hipStream_t s = (hipStream_t)stream;
#define FC_EDGE_DBWD(LL)                                                                                   \
  hipLaunchKernelGGL(edge_dbwd_kernel<LL>, grid, block, 0, s, p, n, pos, shift, ii, jj, vectors, ga, gf, ge, \
                     cot_vec, d_ga, d_gf, d_ge, d_vec)
  switch (desc->l_max) {
    case 0: FC_EDGE_DBWD(0); break;
    case 1: FC_EDGE_DBWD(1); break;
    case 2: FC_EDGE_DBWD(2); break;
    case 3: FC_EDGE_DBWD(3); break;
#if FC_KERNEL_L_MAX >= 4
    case 4: FC_EDGE_DBWD(4); break;
#endif
  }
#undef FC_EDGE_DBWD
  FC_LAUNCH_CHECK();
  return FC_OK;
}

extern "C" int fc_shift_vectors(int64_t n_edges, int32_t n_cells, const int64_t* shifts, const float* cell,
                                const int32_t* idx_i, const int32_t* batch, int64_t n_nodes, float* out,
                                void* stream) {
  if (n_edges < 0 || n_cells < 1 || n_nodes < 0) return FC_ERR_SHAPE;
  if (n_edges == 0) return FC_OK;
  if (!shifts || !cell || !out) return FC_ERR_NULL;
  if (n_cells > 1 && (!idx_i || !batch)) return FC_ERR_NULL;
  const int bs = 256;
  hipLaunchKernelGGL(shift_vectors_kernel, dim3((unsigned)((n_edges + bs - 1) / bs)), dim3(bs), 0,
                     (hipStream_t)stream, n_edges, n_cells, shifts, cell, idx_i, batch, n_nodes, out);
  FC_LAUNCH_CHECK();
  return FC_OK;
}
