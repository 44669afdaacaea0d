// Equivariant linear maps and dense layers on the fp32 matrix cores (MFMA).
//
// Per rank l the map is a GEMM with M = n*(2l+1) rows (one per node and
// component), K = in_features*in_paths[l], N = out_features, and the same weight
// matrix for every component (reference src/flashcart/o3/_linear.py:64-110).
// Rows are addressed as (node, component) so the packed (n, in_dim) feature rows
// are read in place, and all ranks run in one launch (blockIdx.z = rank).
//
// Tiling (gfx950): 64x64 output tile per 256-thread workgroup, four wave64s each
// owning a 32x32 sub-tile built from 2x2 v_mfma_f32_16x16x4f32 blocks; K is
// staged through LDS in steps of 16 (k-major, padded against bank conflicts).
// fp32 inputs, fp32 accumulation: no reduced-precision inputs anywhere.
#include "fc_common.h"

namespace fc {

typedef float floatx4 __attribute__((ext_vector_type(4)));

constexpr int BM = 64, BN = 64, BK = 16, LDP = 4;
constexpr float kSiluScale = 1.6765324703310907f;  // RescaledSiLULayer, src/flashcart/nn/layers.py:23

struct GemmRank {
  const float* A;   // row r = (n, c): A + n*a_row + c*a_comp, K contiguous floats
  const float* B;   // weight
  float* D;         // row r: D + n*d_row + c*d_comp, N contiguous floats
  const float* P;   // optional A-side multiplier source (dense dgrad: pre-activation, same layout as A)
  float* pre;       // optional pre-activation output (dense fwd, same layout as D)
  int64_t a_row, a_comp, d_row, d_comp;
  int64_t M;        // rows = n * comps
  int32_t comps, K, N;
  float scale;
};

struct GemmBatch {
  GemmRank r[4];
  const float* bias;  // dense fwd only (rank 0)
  int32_t trans_b;    // 1: B(k, o) = W[o*K + k] (forward); 0: B(k, o) = W[k*N + o] (input gradient)
  int32_t act;        // 0: none, 1: rescaled SiLU epilogue (fwd) / derivative prologue (dgrad)
  int32_t act_bwd;
};

__device__ __forceinline__ float sigmoidf_(float x) { return 1.0f / (1.0f + __expf(-x)); }

__global__ void __launch_bounds__(256) gemm_kernel(GemmBatch gb) {
  const GemmRank& g = gb.r[blockIdx.z];
  const int64_t r0 = (int64_t)blockIdx.x * BM;
  const int c0 = blockIdx.y * BN;
  if (r0 >= g.M || c0 >= g.N) return;
  __shared__ float As[BK][BM + LDP];
  __shared__ float Bs[BK][BN + LDP];
  const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
  const int wm = wave >> 1, wn = wave & 1;

  floatx4 acc[2][2];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j) acc[i][j] = floatx4{0.f, 0.f, 0.f, 0.f};

  // A-load mapping: 64 rows x 16 k, 4 consecutive k per thread
  const int a_row = t >> 2, a_k = (t & 3) * 4;
  const int64_t gr = r0 + a_row;
  const float* arow = nullptr;
  const float* prow = nullptr;
  if (gr < g.M) {
    const int64_t n = gr / g.comps, c = gr % g.comps;
    arow = g.A + n * g.a_row + c * g.a_comp;
    if (g.P) prow = g.P + n * g.a_row + c * g.a_comp;
  }

  for (int k0 = 0; k0 < g.K; k0 += BK) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int k = k0 + a_k + i;
      float v = 0.f;
      if (arow && k < g.K) {
        v = arow[k];
        if (gb.act_bwd && prow) {
          const float x = prow[k], s = sigmoidf_(x);
          v *= kSiluScale * s * (1.0f + x * (1.0f - s));
        }
      }
      As[a_k + i][a_row] = v;
    }
    if (gb.trans_b) {
      const int o = t >> 2, kk = (t & 3) * 4;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int k = k0 + kk + i, col = c0 + o;
        Bs[kk + i][o] = (k < g.K && col < g.N) ? g.B[(int64_t)col * g.K + k] : 0.f;
      }
    } else {
      const int k = t >> 4, o4 = (t & 15) * 4;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int kg = k0 + k, col = c0 + o4 + i;
        Bs[k][o4 + i] = (kg < g.K && col < g.N) ? g.B[(int64_t)kg * g.N + col] : 0.f;
      }
    }
    __syncthreads();
#pragma unroll
    for (int kk = 0; kk < BK; kk += 4) {
      float a[2], b[2];
#pragma unroll
      for (int i = 0; i < 2; ++i) a[i] = As[kk + (lane >> 4)][wm * 32 + i * 16 + (lane & 15)];
#pragma unroll
      for (int j = 0; j < 2; ++j) b[j] = Bs[kk + (lane >> 4)][wn * 32 + j * 16 + (lane & 15)];
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j) acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(a[i], b[j], acc[i][j], 0, 0, 0);
    }
    __syncthreads();
  }

  // Epilogue: D[4*(lane/16) + v][lane%16] of each 16x16 block.
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const int64_t row = r0 + wm * 32 + i * 16 + 4 * (lane >> 4) + v;
        const int col = c0 + wn * 32 + j * 16 + (lane & 15);
        if (row < g.M && col < g.N) {
          const int64_t n = row / g.comps, c = row % g.comps;
          float val = acc[i][j][v] * g.scale;
          if (gb.bias) val += gb.bias[col];
          if (g.pre) g.pre[n * g.d_row + c * g.d_comp + col] = val;
          if (gb.act == 1) val = kSiluScale * val * sigmoidf_(val);
          g.D[n * g.d_row + c * g.d_comp + col] = val;
        }
      }
}

int launch_gemm(const GemmBatch& gb, int n_ranks, hipStream_t s) {
  int64_t max_m = 0;
  int max_n = 0;
  for (int l = 0; l < n_ranks; ++l) {
    if (gb.r[l].M > max_m) max_m = gb.r[l].M;
    if (gb.r[l].N > max_n) max_n = gb.r[l].N;
  }
  if (max_m == 0 || max_n == 0 || n_ranks == 0) return FC_OK;
  const int64_t gx = (max_m + BM - 1) / BM;
  if (gx > 0x7fffffff) return FC_ERR_SHAPE;
  dim3 grid((unsigned)gx, (unsigned)((max_n + BN - 1) / BN), (unsigned)n_ranks);
  hipLaunchKernelGGL(gemm_kernel, grid, dim3(256), 0, s, gb);
  FC_LAUNCH_CHECK();
  return FC_OK;
}

int fill(int64_t n, float v, float* dst, hipStream_t s);

__global__ void fill_rows_kernel(int64_t rows, int64_t row_stride, int64_t off, int64_t width, float* dst) {
  const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (t >= rows * width) return;
  dst[(t / width) * row_stride + off + (t % width)] = 0.f;
}

int zero_columns(int64_t rows, int64_t row_stride, int64_t off, int64_t width, float* dst, hipStream_t s) {
  if (rows * width == 0) return FC_OK;
  const int bs = 256;
  hipLaunchKernelGGL(fill_rows_kernel, dim3((unsigned)((rows * width + bs - 1) / bs)), dim3(bs), 0, s, rows,
                     row_stride, off, width, dst);
  FC_LAUNCH_CHECK();
  return FC_OK;
}

static int check_linear(const fc_linear_desc* d) {
  if (!d) return FC_ERR_NULL;
  if (d->in_l_max < 0 || d->out_l_max < 0) return FC_ERR_BAD_DESC;
  if (d->in_l_max > 3 || d->out_l_max > 3) return FC_ERR_UNSUPPORTED_L;
  if (d->in_features < 1 || d->out_features < 1) return FC_ERR_BAD_DESC;
  const int common = d->in_l_max < d->out_l_max ? d->in_l_max : d->out_l_max;
  for (int l = 0; l <= d->in_l_max; ++l)
    if (d->in_paths[l] < 1) return FC_ERR_BAD_DESC;
  for (int l = 0; l <= common; ++l)
    if (!d->weight[l]) return FC_ERR_NULL;
  return FC_OK;
}

struct LinearLayout {
  int64_t in_dim, out_dim, in_off[4], out_off[4];
  int common;
};

static LinearLayout linear_layout(const fc_linear_desc* d) {
  LinearLayout L{};
  L.common = d->in_l_max < d->out_l_max ? d->in_l_max : d->out_l_max;
  int64_t o = 0;
  for (int l = 0; l <= d->in_l_max; ++l) {
    L.in_off[l] = o;
    o += (int64_t)(2 * l + 1) * d->in_features * d->in_paths[l];
  }
  L.in_dim = o;
  o = 0;
  for (int l = 0; l <= d->out_l_max; ++l) {
    L.out_off[l] = o;
    o += (int64_t)(2 * l + 1) * d->out_features;
  }
  L.out_dim = o;
  return L;
}

}  // namespace fc

using namespace fc;

extern "C" int fc_linear_fwd(const fc_linear_desc* d, int64_t n, const float* x, float alpha, float* out,
                             void* stream) {
  int st = check_linear(d);
  if (st != FC_OK) return st;
  if (n == 0) return FC_OK;
  if (!x || !out) return FC_ERR_NULL;
  hipStream_t s = (hipStream_t)stream;
  const LinearLayout L = linear_layout(d);
  GemmBatch gb{};
  gb.trans_b = 1;
  for (int l = 0; l <= L.common; ++l) {
    GemmRank& g = gb.r[l];
    const int K = d->in_features * d->in_paths[l];
    g.A = x + L.in_off[l];
    g.a_row = L.in_dim;
    g.a_comp = K;
    g.B = d->weight[l];
    g.D = out + L.out_off[l];
    g.d_row = L.out_dim;
    g.d_comp = d->out_features;
    g.comps = 2 * l + 1;
    g.M = n * g.comps;
    g.K = K;
    g.N = d->out_features;
    g.scale = alpha * d->scale[l];
  }
  st = launch_gemm(gb, L.common + 1, s);
  if (st != FC_OK) return st;
  if (L.common < d->out_l_max)
    return zero_columns(n, L.out_dim, L.out_off[L.common + 1], L.out_dim - L.out_off[L.common + 1], out, s);
  return FC_OK;
}

extern "C" int fc_linear_dgrad(const fc_linear_desc* d, int64_t n, const float* go, float alpha, float* gx,
                               void* stream) {
  int st = check_linear(d);
  if (st != FC_OK) return st;
  if (n == 0) return FC_OK;
  if (!go || !gx) return FC_ERR_NULL;
  hipStream_t s = (hipStream_t)stream;
  const LinearLayout L = linear_layout(d);
  GemmBatch gb{};
  gb.trans_b = 0;
  for (int l = 0; l <= L.common; ++l) {
    GemmRank& g = gb.r[l];
    const int Kin = d->in_features * d->in_paths[l];
    g.A = go + L.out_off[l];
    g.a_row = L.out_dim;
    g.a_comp = d->out_features;
    g.B = d->weight[l];
    g.D = gx + L.in_off[l];
    g.d_row = L.in_dim;
    g.d_comp = Kin;
    g.comps = 2 * l + 1;
    g.M = n * g.comps;
    g.K = d->out_features;
    g.N = Kin;
    g.scale = alpha * d->scale[l];
  }
  st = launch_gemm(gb, L.common + 1, s);
  if (st != FC_OK) return st;
  if (L.common < d->in_l_max)
    return zero_columns(n, L.in_dim, L.in_off[L.common + 1], L.in_dim - L.in_off[L.common + 1], gx, s);
  return FC_OK;
}

extern "C" int fc_dense_fwd(int64_t n, int32_t k, int32_t m, const float* x, const float* w, float scale,
                            const float* bias, int32_t act, float* pre_act, float* out, void* stream) {
  if (n < 0 || k < 1 || m < 1 || act < 0 || act > 1) return FC_ERR_BAD_DESC;
  if (n == 0) return FC_OK;
  if (!x || !w || !out) return FC_ERR_NULL;
  GemmBatch gb{};
  gb.trans_b = 1;
  gb.bias = bias;
  gb.act = act;
  GemmRank& g = gb.r[0];
  g.A = x; g.a_row = k; g.a_comp = 0;
  g.B = w;
  g.D = out; g.d_row = m; g.d_comp = 0;
  g.pre = pre_act;
  g.comps = 1; g.M = n; g.K = k; g.N = m; g.scale = scale;
  return launch_gemm(gb, 1, (hipStream_t)stream);
}

extern "C" int fc_dense_dgrad(int64_t n, int32_t k, int32_t m, const float* go, const float* pre_act,
                              const float* w, float scale, int32_t act, float* gx, void* stream) {
  if (n < 0 || k < 1 || m < 1 || act < 0 || act > 1) return FC_ERR_BAD_DESC;
  if (n == 0) return FC_OK;
  if (!go || !w || !gx || (act == 1 && !pre_act)) return FC_ERR_NULL;
  GemmBatch gb{};
  gb.trans_b = 0;
  gb.act_bwd = act;
  GemmRank& g = gb.r[0];
  g.A = go; g.a_row = m; g.a_comp = 0;
  g.P = act ? pre_act : nullptr;
  g.B = w;
  g.D = gx; g.d_row = k; g.d_comp = 0;
  g.comps = 1; g.M = n; g.K = m; g.N = k; g.scale = scale;
  return launch_gemm(gb, 1, (hipStream_t)stream);
}
