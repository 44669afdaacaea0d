// Equivariant linear maps and dense layers on the fp32 matrix cores (MFMA).
//
// Per rank l the equivariant map is a GEMM with M = n*(2l+1) rows (one per node and
// component), K = in_features*in_paths[l], N = out_features, and one weight matrix
// for every component (reference src/flashcart/o3/_linear.py:64-110). Rows are
// addressed as (node, component), so the packed (n, in_dim) feature rows are read in
// place; all ranks run in one launch.
//
// Tiling (gfx950, wave64): 256-thread workgroups, BM x BN output tiles, waves arranged
// WM x WN, each wave accumulating (BM/WM) x (BN/WN) with v_mfma_f32_32x32x2f32 blocks.
// The K dimension is staged through LDS k-major (conflict-free operand reads) in BK
// steps, with the next tile prefetched into registers during the MFMAs. Blocks are
// ordered N-tile fastest and remapped so that consecutive tiles of one row block land
// on the same XCD (the hardware deals workgroups round-robin over the 8 XCDs), so the
// A rows are fetched from HBM once and then hit that XCD's L2.
// fp32 inputs, fp32 accumulation: no reduced-precision operands.
#include "fc_common.h"

namespace fc {

typedef float floatx16 __attribute__((ext_vector_type(16)));

constexpr float kSiluScale = 1.6765324703310907f;  // RescaledSiLULayer, src/flashcart/nn/layers.py:23

struct GemmRank {
  const float* A;   // row r = (n, c): A + n*a_row + c*a_comp, K contiguous floats
  const float* B;   // weight
  float* D;         // row r: D + n*d_row + c*d_comp, N contiguous floats
  const float* P;   // dense dgrad: pre-activation (same layout as A), multiplies A by act'(P)
  float* pre;       // dense fwd: pre-activation output (same layout as D)
  int64_t a_row, a_comp, d_row, d_comp;
  int32_t M;        // rows = n * comps
  int32_t comps, K, N;
  float scale;
  int32_t tiles_m, tiles_n, tile_base;  // tile grid of this rank, first linear tile id
};

struct GemmBatch {
  GemmRank r[4];
  int32_t n_ranks, total_tiles;
  const float* bias;  // dense fwd only
  int32_t trans_b;    // 1: B(k, o) = W[o*K + k] (forward); 0: B(k, o) = W[k*N + o] (input gradient)
  int32_t act;        // 1: rescaled SiLU epilogue (fwd)
  int32_t act_bwd;    // 1: rescaled SiLU derivative prologue on A (dgrad)
};

__device__ __forceinline__ float sigmoidf_(float x) { return 1.0f / (1.0f + __expf(-x)); }

template <int BM, int BN, int BK, int WM, int WN>
__global__ void __launch_bounds__(256) gemm_kernel(GemmBatch gb) {
  static_assert(WM * WN == 4, "four waves");
  constexpr int TM = BM / WM, TN = BN / WN;  // per-wave tile
  constexpr int FM = TM / 32, FN = TN / 32;  // 32x32 MFMA blocks per wave
  constexpr int PADA = 4, PADB = 4;
  constexpr int A_LOADS = BM * BK / (256 * 4);  // float4 per thread
  constexpr int B_LOADS = BN * BK / (256 * 4);
  static_assert(A_LOADS >= 1 && B_LOADS >= 1, "tile too small for 256 threads");
  __shared__ float As[BK][BM + PADA];
  __shared__ float Bs[BK][BN + PADB];
  __shared__ int64_t d_off[BM];  // output row offsets of this tile (-1 past the end)

  // XCD-aware remap: hardware block b runs on XCD b % 8; give each XCD a contiguous tile range.
  const int nb = gridDim.x;
  const int b = blockIdx.x;
  int tile = b;
  if (nb >= 8 && nb % 8 == 0) tile = (b % 8) * (nb / 8) + b / 8;
  if (tile >= gb.total_tiles) return;
  int ri = 0;
#pragma unroll
  for (int q = 1; q < 4; ++q)
    if (q < gb.n_ranks && tile >= gb.r[q].tile_base) ri = q;
  const GemmRank& g = gb.r[ri];
  const int local = tile - g.tile_base;
  const int tm = local / g.tiles_n, tn = local % g.tiles_n;
  const int r0 = tm * BM, c0 = tn * BN;

  const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
  const int wm = wave / WN, wn = wave % WN;
  for (int m = t; m < BM; m += 256) {
    const int row = r0 + m;
    int64_t off = -1;
    if (row < g.M) {
      const int n = row / g.comps, c = row - n * g.comps;
      off = (int64_t)n * g.d_row + (int64_t)c * g.d_comp;
    }
    d_off[m] = off;
  }

  // ---- global-load mapping (float4 along K for A; along K or N for B)
  // A: BM rows x BK cols, row-major K; thread loads A_LOADS float4s.
  constexpr int A_TPR = BK / 4;  // threads per row
  const float* a_ptr[A_LOADS];
  const float* p_ptr[A_LOADS];
  int a_k4[A_LOADS], a_m[A_LOADS];
#pragma unroll
  for (int i = 0; i < A_LOADS; ++i) {
    const int idx = t + i * 256;
    a_m[i] = idx / A_TPR;
    a_k4[i] = (idx % A_TPR) * 4;
    const int row = r0 + a_m[i];
    a_ptr[i] = nullptr;
    p_ptr[i] = nullptr;
    if (row < g.M) {
      const int n = row / g.comps, c = row - n * g.comps;
      a_ptr[i] = g.A + (int64_t)n * g.a_row + (int64_t)c * g.a_comp;
      if (g.P) p_ptr[i] = g.P + (int64_t)n * g.a_row + (int64_t)c * g.a_comp;
    }
  }
  const bool a_vec = ((g.K & 3) == 0) && ((g.a_row & 3) == 0) && ((g.a_comp & 3) == 0) &&
                     (((uintptr_t)g.A & 15) == 0);

  float4 ra[A_LOADS], rb[B_LOADS];
  auto load_a = [&](int k0) {
#pragma unroll
    for (int i = 0; i < A_LOADS; ++i) {
      const int k = k0 + a_k4[i];
      float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
      if (a_ptr[i]) {
        if (a_vec && k + 3 < g.K) {
          v = *reinterpret_cast<const float4*>(a_ptr[i] + k);
        } else {
          if (k < g.K) v.x = a_ptr[i][k];
          if (k + 1 < g.K) v.y = a_ptr[i][k + 1];
          if (k + 2 < g.K) v.z = a_ptr[i][k + 2];
          if (k + 3 < g.K) v.w = a_ptr[i][k + 3];
        }
        if (gb.act_bwd && p_ptr[i]) {
          float pv[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
          for (int j = 0; j < 4; ++j)
            if (k + j < g.K) pv[j] = p_ptr[i][k + j];
          float* vv = reinterpret_cast<float*>(&v);
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            const float s = sigmoidf_(pv[j]);
            vv[j] *= kSiluScale * s * (1.0f + pv[j] * (1.0f - s));
          }
        }
      }
      ra[i] = v;
    }
  };
  // B: BK x BN tile. trans_b: W[col*K + k] (k contiguous); else W[k*N + col] (col contiguous).
  auto load_b = [&](int k0) {
#pragma unroll
    for (int i = 0; i < B_LOADS; ++i) {
      const int idx = t + i * 256;
      float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
      float* vv = reinterpret_cast<float*>(&v);
      if (gb.trans_b) {
        const int col = c0 + idx / (BK / 4), k = k0 + (idx % (BK / 4)) * 4;
        if (col < g.N) {
          const float* w = g.B + (int64_t)col * g.K;
#pragma unroll
          for (int j = 0; j < 4; ++j)
            if (k + j < g.K) vv[j] = w[k + j];
        }
      } else {
        const int k = k0 + idx / (BN / 4), col = c0 + (idx % (BN / 4)) * 4;
        if (k < g.K) {
          const float* w = g.B + (int64_t)k * g.N;
#pragma unroll
          for (int j = 0; j < 4; ++j)
            if (col + j < g.N) vv[j] = w[col + j];
        }
      }
      rb[i] = v;
    }
  };
  auto store_tiles = [&]() {
#pragma unroll
    for (int i = 0; i < A_LOADS; ++i) {
      const float* vv = reinterpret_cast<const float*>(&ra[i]);
#pragma unroll
      for (int j = 0; j < 4; ++j) As[a_k4[i] + j][a_m[i]] = vv[j];
    }
#pragma unroll
    for (int i = 0; i < B_LOADS; ++i) {
      const int idx = t + i * 256;
      const float* vv = reinterpret_cast<const float*>(&rb[i]);
      if (gb.trans_b) {
        const int col = idx / (BK / 4), k = (idx % (BK / 4)) * 4;
#pragma unroll
        for (int j = 0; j < 4; ++j) Bs[k + j][col] = vv[j];
      } else {
        const int k = idx / (BN / 4), col = (idx % (BN / 4)) * 4;
#pragma unroll
        for (int j = 0; j < 4; ++j) Bs[k][col + j] = vv[j];
      }
    }
  };

  floatx16 acc[FM][FN];
#pragma unroll
  for (int i = 0; i < FM; ++i)
#pragma unroll
    for (int j = 0; j < FN; ++j)
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[i][j][v] = 0.f;

  load_a(0);
  load_b(0);
  for (int k0 = 0; k0 < g.K; k0 += BK) {
    __syncthreads();
    store_tiles();
    __syncthreads();
    if (k0 + BK < g.K) {
      load_a(k0 + BK);
      load_b(k0 + BK);
    }
#pragma unroll
    for (int kk = 0; kk < BK; kk += 2) {
      float a[FM], bv[FN];
#pragma unroll
      for (int i = 0; i < FM; ++i) a[i] = As[kk + (lane >> 5)][wm * TM + i * 32 + (lane & 31)];
#pragma unroll
      for (int j = 0; j < FN; ++j) bv[j] = Bs[kk + (lane >> 5)][wn * TN + j * 32 + (lane & 31)];
#pragma unroll
      for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j) acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(a[i], bv[j], acc[i][j], 0, 0, 0);
    }
  }

  // ---- epilogue: D[row][col] with row = 8*(v/4) + 4*(lane/32) + v%4, col = lane%32 per 32x32 block
  float bias_v[FN];
#pragma unroll
  for (int j = 0; j < FN; ++j) {
    const int col = c0 + wn * TN + j * 32 + (lane & 31);
    bias_v[j] = (gb.bias && col < g.N) ? gb.bias[col] : 0.f;
  }
#pragma unroll
  for (int i = 0; i < FM; ++i) {
#pragma unroll
    for (int v = 0; v < 16; ++v) {
      const int64_t off = d_off[wm * TM + i * 32 + 8 * (v >> 2) + 4 * (lane >> 5) + (v & 3)];
      if (off < 0) continue;
      float* drow = g.D + off;
      float* prow = g.pre ? g.pre + off : nullptr;
#pragma unroll
      for (int j = 0; j < FN; ++j) {
        const int col = c0 + wn * TN + j * 32 + (lane & 31);
        if (col >= g.N) continue;
        float val = fmaf(acc[i][j][v], g.scale, bias_v[j]);
        if (prow) prow[col] = val;
        if (gb.act == 1) val = kSiluScale * val * sigmoidf_(val);
        drow[col] = val;
      }
    }
  }
}

template <int BM, int BN, int BK, int WM, int WN>
int launch_gemm_cfg(GemmBatch gb, int n_ranks, hipStream_t s) {
  int64_t total = 0;
  for (int l = 0; l < n_ranks; ++l) {
    GemmRank& g = gb.r[l];
    g.tiles_m = (g.M + BM - 1) / BM;
    g.tiles_n = (g.N + BN - 1) / BN;
    g.tile_base = (int32_t)total;
    total += (int64_t)g.tiles_m * g.tiles_n;
  }
  if (total == 0) return FC_OK;
  if (total > 0x7fffffff) return FC_ERR_SHAPE;
  gb.n_ranks = n_ranks;
  gb.total_tiles = (int32_t)total;
  const int64_t grid = (total + 7) / 8 * 8;  // a multiple of 8 enables the XCD remap
  hipLaunchKernelGGL((gemm_kernel<BM, BN, BK, WM, WN>), dim3((unsigned)grid), dim3(256), 0, s, gb);
  FC_LAUNCH_CHECK();
  return FC_OK;
}

int launch_gemm(GemmBatch gb, int n_ranks, hipStream_t s) {
  int max_n = 0;
  int64_t max_m = 0;
  for (int l = 0; l < n_ranks; ++l) {
    if (gb.r[l].N > max_n) max_n = gb.r[l].N;
    if (gb.r[l].M > max_m) max_m = gb.r[l].M;
    if (gb.r[l].M < 0) return FC_ERR_SHAPE;
  }
  if (max_m == 0 || max_n == 0 || n_ranks == 0) return FC_OK;
  if (max_n <= 64) return launch_gemm_cfg<128, 64, 16, 4, 1>(gb, n_ranks, s);
  return launch_gemm_cfg<128, 128, 16, 2, 2>(gb, n_ranks, s);
}

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
  if (n * 7 > 0x7fffffff) return FC_ERR_SHAPE;
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
    g.M = (int32_t)(n * g.comps);
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
  if (n * 7 > 0x7fffffff) return FC_ERR_SHAPE;
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
    g.M = (int32_t)(n * g.comps);
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
  if (n > 0x7fffffff) return FC_ERR_SHAPE;
  GemmBatch gb{};
  gb.trans_b = 1;
  gb.bias = bias;
  gb.act = act;
  GemmRank& g = gb.r[0];
  g.A = x; g.a_row = k; g.a_comp = 0;
  g.B = w;
  g.D = out; g.d_row = m; g.d_comp = 0;
  g.pre = pre_act;
  g.comps = 1; g.M = (int32_t)n; g.K = k; g.N = m; g.scale = scale;
  return launch_gemm(gb, 1, (hipStream_t)stream);
}

extern "C" int fc_dense_dgrad(int64_t n, int32_t k, int32_t m, const float* go, const float* pre_act,
                              const float* w, float scale, int32_t act, float* gx, void* stream) {
  if (n < 0 || k < 1 || m < 1 || act < 0 || act > 1) return FC_ERR_BAD_DESC;
  if (n == 0) return FC_OK;
  if (!go || !w || !gx || (act == 1 && !pre_act)) return FC_ERR_NULL;
  if (n > 0x7fffffff) return FC_ERR_SHAPE;
  GemmBatch gb{};
  gb.trans_b = 0;
  gb.act_bwd = act;
  GemmRank& g = gb.r[0];
  g.A = go; g.a_row = m; g.a_comp = 0;
  g.P = act ? pre_act : nullptr;
  g.B = w;
  g.D = gx; g.d_row = k; g.d_comp = 0;
  g.comps = 1; g.M = (int32_t)n; g.K = m; g.N = k; g.scale = scale;
  return launch_gemm(gb, 1, (hipStream_t)stream);
}
