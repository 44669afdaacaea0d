// Equivariant linear maps and dense layers on the fp32 matrix cores (MFMA).
//
// Per rank l the equivariant map is a GEMM with M = n*(2l+1) rows (one per node and
// component), K = in_features*in_paths[l], N = out_features, and one weight matrix
// for every component (reference src/flashcart/o3/_linear.py:64-110). Rows are
// addressed as (node, component), so the packed (n, in_dim) feature rows are read in
// place; all ranks run in one launch.
//
// Two kernels. gemm_pipe_kernel serves every launch whose
// ranks have K % 32 == 0 and 16-byte aligned rows and need no activation: direct global->LDS
// loads into a three-stage ring, persistent workgroups, v_mfma_f32_16x16x4f32 blocks.
// gemm_kernel serves the rest (activation prologue/epilogue of the dense layers, ragged K):
// Tiling (gfx950, wave64): 256-thread workgroups, BM x BN output tiles, waves arranged
// WM x WN, each wave accumulating (BM/WM) x (BN/WN) with v_mfma_f32_32x32x2f32 blocks.
// K advances in steps of 32 through LDS (a single buffer with two barriers per step in
// the tile shapes launched, which leaves room for four workgroups per CU): the next
// step's global loads are in flight while the current step's 16 MFMA k-pairs run.
// Full K steps load through one branch-free path (row pointers clamped
// to valid rows and masked afterwards): per-lane divergence between vector and scalar
// loads made the compiler wait on outstanding loads inside the load sequence.
// A rows (and B rows when the weight is k-contiguous, the forward) sit in LDS in the
// order the MFMA consumes them: k-step s takes k = 2s (lanes 0-31) and k = 2s+1
// (lanes 32-63), so position (k % 2) * 16 + k / 2 puts each half-wave's 16 values of
// the step sequence next to each other and a lane fetches four k-steps with one
// 128-bit LDS read; the row pitch of 36 floats makes those reads conflict-free (row
// stride 9 x 16 B). A column-contiguous weight (the input gradient) is stored k-major
// with 128-bit writes instead and read one k-step at a time.
// Blocks are ordered N-tile fastest and remapped so that consecutive tiles of one row
// block land on the same XCD (the hardware deals workgroups round-robin over the 8
// XCDs), so the A rows are fetched from HBM once and then hit that XCD's L2.
// fp32 inputs, fp32 accumulation: no reduced-precision operands.
#include "fc_common.h"
#include <type_traits>  // std::true_type

namespace fc {

typedef float floatx16 __attribute__((ext_vector_type(16)));

constexpr float kSiluScale = 1.6765324703310907f;  // RescaledSiLULayer, src/flashcart/nn/layers.py:23

struct GemmRank {
  const float* A;   // row r = (n, c): A + n*a_row + c*a_comp, K contiguous floats
  const float* B;   // weight
  float* D;         // row r: D + n*d_row + c*d_comp, N contiguous floats
  const float* P;   // dense dgrad: pre-activation (same layout as A), multiplies A by act'(P)
  float* pre;       // dense fwd: pre-activation output (same layout as D)
  const float* R;   // residual added to the result (same layout as D; may be D itself)
  int64_t a_row, a_comp, d_row, d_comp;
  const int32_t* a_lo;  // pair sum (gb.pair_sum) with gathered halves: A row r's halves are rows a_lo[r]
  const int32_t* a_hi;  // and a_hi[r] of A (a_row floats apart); NULL: A row r holds both halves
  int32_t M;        // rows = n * comps
  int32_t comps, K, N;
  float scale;
  int32_t tiles_m, tiles_n, tile_base;  // tile grid of this rank, first linear tile id
};

struct GemmBatch {
  GemmRank r[FC_MAX_RANKS];
  int32_t n_ranks, total_tiles;
  const float* bias;  // dense fwd only
  int32_t trans_b;    // 1: B(k, o) = W[o*K + k] (forward); 0: B(k, o) = W[k*N + o] (input gradient)
  int32_t act;        // 1: rescaled SiLU epilogue (fwd)
  int32_t act_bwd;    // 1: rescaled SiLU derivative prologue on A (dgrad)
  int32_t pair_sum;   // 1: A rows hold two K-long halves, multiplied as their sum (pipelined kernel only)
};

__device__ __forceinline__ float sigmoidf_(float x) { return 1.0f / (1.0f + __expf(-x)); }

constexpr int GEMM_BK = 32;
constexpr int GEMM_PITCH = GEMM_BK + 4;

// LDS position of k (0..31) inside an operand row.
__device__ __forceinline__ constexpr int kpos(int k) { return (k & 1) * 16 + (k >> 1); }

template <int BM, int BN, int WM, int WN, int NBUF, bool KB>
__global__ void __launch_bounds__(256) gemm_kernel(GemmBatch gb) {
  static_assert(WM * WN == 4, "four waves");
  constexpr int BK = GEMM_BK, LP = GEMM_PITCH;
  constexpr int TM = BM / WM, TN = BN / WN;  // per-wave tile
  constexpr int FM = TM / 32, FN = TN / 32;  // 32x32 MFMA blocks per wave
  constexpr int A_LOADS = BM * BK / 1024;    // float4 per thread and K step
  constexpr int B_LOADS = BN * BK / 1024;
  static_assert(A_LOADS >= 1 && B_LOADS >= 1, "tile too small for 256 threads");
  __shared__ __attribute__((aligned(16))) float As[NBUF][BM * LP];
  constexpr int BSZ = KB ? BK * (BN + 4) : BN * LP;
  __shared__ __attribute__((aligned(16))) float Bs[NBUF][BSZ];
  __shared__ int64_t d_off[BM];  // output row offsets of this tile (-1 past the end)

  // XCD-aware remap: hardware block b runs on XCD b % 8; give each XCD a contiguous tile range.
  const int nb = gridDim.x;
  const int b = blockIdx.x;
  int tile = b;
  if (nb >= 8 && nb % 8 == 0) tile = (b % 8) * (nb / 8) + b / 8;
  if (tile >= gb.total_tiles) return;
  int ri = 0;
#pragma unroll
  for (int q = 1; q < FC_MAX_RANKS; ++q)
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

  // ---- global loads: 8 threads per operand row, one float4 (4 consecutive k) each.
  // Row pointers are clamped to valid rows and masked afterwards, so that full K steps
  // take one branch-free path (no per-lane divergence between vector and scalar loads).
  const int lk4 = (t & 7) * 4;  // k offset of this thread inside a K step
  const float* a_ptr[A_LOADS];
  const float* p_ptr[A_LOADS];
  bool a_ok[A_LOADS];
  const bool use_p = gb.act_bwd && g.P;
#pragma unroll
  for (int i = 0; i < A_LOADS; ++i) {
    const int row0 = r0 + (t >> 3) + 32 * i;
    a_ok[i] = row0 < g.M;
    const int row = a_ok[i] ? row0 : g.M - 1;
    const int n = row / g.comps, c = row - n * g.comps;
    a_ptr[i] = g.A + (int64_t)n * g.a_row + (int64_t)c * g.a_comp;
    p_ptr[i] = use_p ? g.P + (int64_t)n * g.a_row + (int64_t)c * g.a_comp : nullptr;
  }
  const bool a_vec = ((g.K & 3) == 0) && ((g.a_row & 3) == 0) && ((g.a_comp & 3) == 0) &&
                     (((uintptr_t)g.A & 15) == 0) && (!use_p || (((uintptr_t)g.P & 15) == 0));
  const bool b_vec = gb.trans_b ? (((g.K & 3) == 0) && (((uintptr_t)g.B & 15) == 0))
                                : (((g.N & 3) == 0) && (((uintptr_t)g.B & 15) == 0));
  // B operand rows: trans_b -> output column c0 + (t>>3) + 32 i (k contiguous);
  // otherwise k row k0 + t/(BN/4) + (1024/BN) i, 4 consecutive columns from bcol.
  const float* b_ptr[B_LOADS];
  bool b_ok[B_LOADS];
  const int bcol = c0 + (t % (BN / 4)) * 4;
#pragma unroll
  for (int i = 0; i < B_LOADS; ++i) {
    if (gb.trans_b) {
      const int col0 = c0 + (t >> 3) + 32 * i;
      b_ok[i] = col0 < g.N;
      b_ptr[i] = g.B + (int64_t)(b_ok[i] ? col0 : g.N - 1) * g.K;
    } else {
      b_ok[i] = bcol + 3 < g.N;
      b_ptr[i] = g.B + (b_ok[i] ? bcol : 0);
    }
  }

  auto slow4 = [&](const float* p, int k, int kmax) -> float4 {
    float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
    if (k < kmax) v.x = p[k];
    if (k + 1 < kmax) v.y = p[k + 1];
    if (k + 2 < kmax) v.z = p[k + 2];
    if (k + 3 < kmax) v.w = p[k + 3];
    return v;
  };
  const float4 zero4 = make_float4(0.f, 0.f, 0.f, 0.f);

  float4 ra[A_LOADS], rb[B_LOADS];
  auto load_step = [&](int k0) {
    const bool full = k0 + BK <= g.K;  // uniform
    float4 pa[A_LOADS];
    if (full && a_vec) {
#pragma unroll
      for (int i = 0; i < A_LOADS; ++i) ra[i] = *reinterpret_cast<const float4*>(a_ptr[i] + k0 + lk4);
      if (use_p) {
#pragma unroll
        for (int i = 0; i < A_LOADS; ++i) pa[i] = *reinterpret_cast<const float4*>(p_ptr[i] + k0 + lk4);
      }
    } else {
#pragma unroll
      for (int i = 0; i < A_LOADS; ++i) {
        ra[i] = slow4(a_ptr[i], k0 + lk4, g.K);
        if (use_p) pa[i] = slow4(p_ptr[i], k0 + lk4, g.K);
      }
    }
#pragma unroll
    for (int i = 0; i < A_LOADS; ++i) {
      if (use_p) {
        const float pp[4] = {pa[i].x, pa[i].y, pa[i].z, pa[i].w};
        float* vv = reinterpret_cast<float*>(&ra[i]);
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const float s = sigmoidf_(pp[j]);
          vv[j] *= kSiluScale * s * (1.0f + pp[j] * (1.0f - s));
        }
      }
      if (!a_ok[i]) ra[i] = zero4;
    }
    if (gb.trans_b) {
      if (full && b_vec) {
#pragma unroll
        for (int i = 0; i < B_LOADS; ++i) rb[i] = *reinterpret_cast<const float4*>(b_ptr[i] + k0 + lk4);
      } else {
#pragma unroll
        for (int i = 0; i < B_LOADS; ++i) rb[i] = slow4(b_ptr[i], k0 + lk4, g.K);
      }
#pragma unroll
      for (int i = 0; i < B_LOADS; ++i)
        if (!b_ok[i]) rb[i] = zero4;
    } else {
#pragma unroll
      for (int i = 0; i < B_LOADS; ++i) {
        const int k = k0 + (t / (BN / 4)) + (1024 / BN) * i;
        if (full && b_vec && b_ok[i]) {
          rb[i] = *reinterpret_cast<const float4*>(b_ptr[i] + (int64_t)k * g.N);
        } else {
          rb[i] = k < g.K ? slow4(g.B + (int64_t)k * g.N, bcol, g.N) : zero4;
        }
      }
    }
  };
  auto store_step = [&](int buf) {
    float* as = As[buf];
    float* bs = Bs[buf];
    const int p0 = kpos(lk4);  // lk4 even: (v.x, v.z) at p0, (v.y, v.w) at p0 + 16
#pragma unroll
    for (int i = 0; i < A_LOADS; ++i) {
      float* r = as + ((t >> 3) + 32 * i) * LP;
      *reinterpret_cast<float2*>(r + p0) = make_float2(ra[i].x, ra[i].z);
      *reinterpret_cast<float2*>(r + p0 + 16) = make_float2(ra[i].y, ra[i].w);
    }
#pragma unroll
    for (int i = 0; i < B_LOADS; ++i) {
      if (gb.trans_b) {
        float* r = bs + ((t >> 3) + 32 * i) * LP;
        *reinterpret_cast<float2*>(r + p0) = make_float2(rb[i].x, rb[i].z);
        *reinterpret_cast<float2*>(r + p0 + 16) = make_float2(rb[i].y, rb[i].w);
      } else {
        const int kk = (t / (BN / 4)) + (1024 / BN) * i, col = (t % (BN / 4)) * 4;
        if constexpr (KB) {
          *reinterpret_cast<float4*>(bs + kk * (BN + 4) + col) = rb[i];
        } else {
          const int p = kpos(kk);
          bs[(col + 0) * LP + p] = rb[i].x;
          bs[(col + 1) * LP + p] = rb[i].y;
          bs[(col + 2) * LP + p] = rb[i].z;
          bs[(col + 3) * LP + p] = rb[i].w;
        }
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

  const int half = (lane >> 5) * 16;
  const int nk = (g.K + BK - 1) / BK;
  load_step(0);
  store_step(0);
  __syncthreads();
  for (int kt = 0; kt < nk; ++kt) {
    const int cur = NBUF == 2 ? (kt & 1) : 0;
    if (kt + 1 < nk) load_step((kt + 1) * BK);
    const float* as = As[cur] + (wm * TM + (lane & 31)) * LP + half;
    const float* bs = KB ? Bs[cur] + (lane >> 5) * (BN + 4) + wn * TN + (lane & 31)
                         : Bs[cur] + (wn * TN + (lane & 31)) * LP + half;
#pragma unroll
    for (int s4 = 0; s4 < 4; ++s4) {
      float4 a4[FM], b4[FN];
#pragma unroll
      for (int i = 0; i < FM; ++i) a4[i] = *reinterpret_cast<const float4*>(as + i * 32 * LP + s4 * 4);
#pragma unroll
      for (int j = 0; j < FN; ++j) {
        if constexpr (KB) {  // k-step s = 4 s4 + q reads row 2 s + lane/32
          const float* p = bs + j * 32 + (8 * s4) * (BN + 4);
          b4[j] = make_float4(p[0], p[2 * (BN + 4)], p[4 * (BN + 4)], p[6 * (BN + 4)]);
        } else {
          b4[j] = *reinterpret_cast<const float4*>(bs + j * 32 * LP + s4 * 4);
        }
      }
#pragma unroll
      for (int q = 0; q < 4; ++q)
#pragma unroll
        for (int i = 0; i < FM; ++i)
#pragma unroll
          for (int j = 0; j < FN; ++j)
            acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(reinterpret_cast<const float*>(&a4[i])[q],
                                                             reinterpret_cast<const float*>(&b4[j])[q], acc[i][j],
                                                             0, 0, 0);
    }
    if constexpr (NBUF == 1) __syncthreads();
    if (kt + 1 < nk) store_step(NBUF == 2 ? cur ^ 1 : 0);
    __syncthreads();
  }

  // ---- epilogue: D[row][col] with row = 8*(v/4) + 4*(lane/32) + v%4, col = lane%32 per 32x32 block
  float bias_v[FN];
#pragma unroll
  for (int j = 0; j < FN; ++j) {
    const int col = c0 + wn * TN + j * 32 + (lane & 31);
    bias_v[j] = (gb.bias && col < g.N) ? gb.bias[col] : 0.f;
  }
  // The residual may alias D (in-place accumulation), so a lane reads its residual values
  // before storing to them; loading them inside the store loop would serialise every load
  // behind the preceding stores.
  if (r0 + BM <= g.M && c0 + BN <= g.N && !g.pre && gb.act == 0) {
    // interior tile with a plain epilogue (scale, bias, residual): no bound checks, and
    // residual reads in groups of 4 rows so the values in flight stay in few registers
    const int cl = c0 + wn * TN + (lane & 31);
#pragma unroll
    for (int i = 0; i < FM; ++i) {
#pragma unroll
      for (int v4 = 0; v4 < 16; v4 += 4) {  // rows 8 (v4/4) + 4 (lane/32) + q of the 32-row block
        int64_t offs[4];
        float rvi[4][FN];
#pragma unroll
        for (int q = 0; q < 4; ++q) offs[q] = d_off[wm * TM + i * 32 + 8 * (v4 >> 2) + 4 * (lane >> 5) + q];
        if (g.R) {
#pragma unroll
          for (int q = 0; q < 4; ++q)
#pragma unroll
            for (int j = 0; j < FN; ++j) rvi[q][j] = g.R[offs[q] + cl + j * 32];
        }
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          float* drow = g.D + offs[q] + cl;
#pragma unroll
          for (int j = 0; j < FN; ++j) {
            float val = fmaf(acc[i][j][v4 + q], g.scale, bias_v[j]);
            if (g.R) val += rvi[q][j];
            drow[j * 32] = val;
          }
        }
      }
    }
    return;
  }
  float rv[FM][16][FN];
  if (g.R) {
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        const int64_t off = d_off[wm * TM + i * 32 + 8 * (v >> 2) + 4 * (lane >> 5) + (v & 3)];
#pragma unroll
        for (int j = 0; j < FN; ++j) {
          const int col = c0 + wn * TN + j * 32 + (lane & 31);
          rv[i][v][j] = (off >= 0 && col < g.N) ? g.R[off + col] : 0.f;
        }
      }
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
        if (g.R) val += rv[i][v][j];
        drow[col] = val;
      }
    }
  }
}

// ---------------------------------------------------------------------------------------
// Pipelined GEMM. Operands travel global -> LDS by direct loads (global_load_lds_dwordx4:
// no register staging, no LDS store phase) into a ring of three stages, so every wave has
// the next two K steps in flight while it multiplies the current one, with one barrier per
// K step. Persistent workgroups (two per CU) walk their tiles as one stream of K steps:
// the first steps of the next tile load during the current tile's epilogue. Used when every
// rank has K % 32 == 0, 16-byte aligned operand rows and no A prologue (act_bwd) or
// activation epilogue.
//
// LDS layout per stage: A, and B when k-contiguous (trans_b), as rows of 8 chunks of 4
// floats (one 32-float K step); chunk c of row r sits at position c ^ ((r / 2) % 8), so the
// rows read together at one chunk fall in distinct banks (SQ_LDS_BANK_CONFLICT reads 0; the
// (r % 8)-based swizzle it replaces stalled the LDS ~0.55 of the busy cycles). A k-major B (the input
// gradient) sits as 32 rows of BN floats; chunk p of row k at p ^ pipe_kswz(k), which puts the
// rows that the lane groups of one k step read (4 apart) in different parts of the bank row.
// K-step mapping: MFMA k-pair q (0..3) of quad s4 (0..3) takes k = 8 s4 + 4 h + q in lane
// half h, in A and B alike, so each lane reads four k values as one 128-bit chunk.

__device__ __forceinline__ int pipe_swz(int r) { return (r >> 1) & 7; }
// k-major B rows: the lane groups reading one k step sit 4 rows apart (2 groups for 32x32x2
// blocks, 4 for 16x16x4); XOR-ing the chunk index by the group puts each group's 128-byte
// (32x32) or 64-byte (16x16) column run in its own part of the bank row.
template <int MI>
__device__ __forceinline__ int pipe_kswz(int k) {
  return MI == 32 ? ((k >> 2) & 1) << 3 : ((k >> 2) & 3) << 2;
}

// One 16-byte direct load per lane into LDS at lds + 16 * lane (lds: byte offset, wave-uniform).
// Issued as inline assembly so that the compiler does not track it: it would otherwise wait for
// every outstanding direct load before any LDS read, which defeats the ring. The kernel orders
// these loads itself (explicit vmcnt waits and barriers below); the 'memory' clobber keeps the
// compiler from moving other memory accesses across them. M0 written by a scalar move needs
// one wait state before the load that reads it.
// M0 is a reserved register to the compiler; no other code of these kernels uses it (no
// indirect register indexing, no compiler-issued direct loads), so clobbering it is safe here.
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
__device__ __forceinline__ void lds_dma16(const float* src, uint32_t lds_off) {
  asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, off" ::"v"(src), "s"(lds_off)
               : "memory", "m0");
}

// The same with a wave-uniform 64-bit base in scalar registers and a 32-bit per-lane byte
// offset (no per-lane 64-bit address arithmetic per load).
__device__ __forceinline__ void lds_dma16_s(const float* base, uint32_t voff, uint32_t lds_off) {
  asm volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, %1" ::"v"(voff), "s"(base),
               "s"(lds_off)
               : "memory", "m0");
}

// A pointer that is the same in every lane, moved to scalar registers (the asm operands of
// lds_dma16_s must be scalar).
__device__ __forceinline__ const float* uniform_ptr(const float* p) {
  const uint64_t v = (uint64_t)(uintptr_t)p;
  const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)v);
  const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)(v >> 32));
  return (const float*)(uintptr_t)(((uint64_t)hi << 32) | lo);
}

// LDS byte address of a __shared__ array (a compile-time constant for a named array)
__device__ __forceinline__ uint32_t lds_addr(const float* p) {
  return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) float*)(p);
}
#pragma clang diagnostic pop

// barrier after which LDS reads see what other waves (and their completed direct loads) wrote;
// the empty asm stops the compiler from moving LDS accesses across it
__device__ __forceinline__ void pipe_barrier() {
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

// s_waitcnt immediate (gfx9 encoding): vector-memory count <= vm, LDS count <= lgkm, no export wait
#define FC_WAITCNT_IMM(vm, lgkm) (((vm) & 0xF) | ((((vm) >> 4) & 3) << 14) | (0x7 << 4) | (((lgkm) & 0xF) << 8))

struct PipeTile {
  int ri, r0, c0, K;
};

// PS (pair sum): every A row is the sum of two halves of K floats, A[r, 0:K] and A[r, K:2K], or
// rows a_lo[r] and a_hi[r] of A when the rank gives those index arrays; both halves go to LDS by
// direct loads and are added as the MFMA operands are read, so the MFMA work is that of K (the
// radial output layer's input gradient over edge pairs, whose two edges share the layer's
// output row).
template <int BM, int BN, int WM, int WN, int MI, bool KB, bool PS = false>
__global__ void __launch_bounds__(256, ((PS ? 2 : 1) * BM + BN) * 32 * 4 * 3 <= 80 * 1024 ? 2 : 1) gemm_pipe_kernel(GemmBatch gb) {
  static_assert(WM * WN == 4, "four waves");
  static_assert(MI == 32 || MI == 16, "MFMA block: 32x32x2 or 16x16x4");
  constexpr int TM = BM / WM, TN = BN / WN;
  constexpr int FM = TM / MI, FN = TN / MI;  // MFMA blocks per wave
  constexpr int NV = MI == 32 ? 16 : 4;      // accumulator values per lane and block
  typedef float accv __attribute__((ext_vector_type(NV)));
  constexpr int A_DMA = BM * 8 / 256;  // 16-byte chunks per thread and K step
  constexpr int B_DMA = BN * 8 / 256;
  constexpr int AH = PS ? 2 : 1;       // A halves
  constexpr int L = AH * A_DMA + B_DMA;  // direct loads per wave and K step
  static_assert(A_DMA >= 1 && B_DMA >= 1 && L <= 15, "tile shape");
  constexpr int BQ = BN / 4;           // chunks per k-major B row
  __shared__ __attribute__((aligned(16))) float As0[AH * BM * 32];
  __shared__ __attribute__((aligned(16))) float As1[AH * BM * 32];
  __shared__ __attribute__((aligned(16))) float As2[AH * BM * 32];
  __shared__ __attribute__((aligned(16))) float Bs0[BN * 32];
  __shared__ __attribute__((aligned(16))) float Bs1[BN * 32];
  __shared__ __attribute__((aligned(16))) float Bs2[BN * 32];

  const int t = threadIdx.x, lane = t & 63, wave = t >> 6, h = lane >> 5;
  const int wm = wave / WN, wn = wave % WN;
  const int G = gridDim.x, b = blockIdx.x;
  // Tiles of this workgroup: a contiguous range holding 1/G of the batch's K steps (ranks
  // differ in K, so equal tile counts would not be equal work). Workgroups of one XCD
  // (hardware block b runs on XCD b % 8) take neighbouring ranges, so an XCD's L2 serves
  // one contiguous run of A rows.
  const int v = (G >= 8 && G % 8 == 0) ? (b % 8) * (G / 8) + b / 8 : b;
  int64_t work = 0;
#pragma unroll
  for (int q = 0; q < FC_MAX_RANKS; ++q)
    if (q < gb.n_ranks) work += (int64_t)gb.r[q].tiles_m * gb.r[q].tiles_n * (gb.r[q].K / 32);
  // first tile whose first K step (counted over the whole batch) is at or after step s
  auto tile_at = [&](int64_t s) -> int {
    int64_t base = 0;
#pragma unroll
    for (int q = 0; q < FC_MAX_RANKS; ++q) {
      if (q >= gb.n_ranks) break;
      const GemmRank& g = gb.r[q];
      const int64_t ks = g.K / 32, n = (int64_t)g.tiles_m * g.tiles_n;
      if (n > 0 && s <= base + (n - 1) * ks) {
        const int64_t d = s - base;
        return g.tile_base + (int)(d <= 0 ? 0 : (d + ks - 1) / ks);
      }
      base += n * ks;
    }
    return gb.total_tiles;
  };
  // (uniform; kept in scalar registers so the tile loop's bookkeeping stays scalar)
  const int t_first = __builtin_amdgcn_readfirstlane(tile_at(((int64_t)v * work + G - 1) / G));
  const int t_end = __builtin_amdgcn_readfirstlane(tile_at(((int64_t)(v + 1) * work + G - 1) / G));
  constexpr int t_step = 1;
  auto decode = [&](int tile) -> PipeTile {
    int ri = 0;
#pragma unroll
    for (int q = 1; q < FC_MAX_RANKS; ++q)
      if (q < gb.n_ranks && tile >= gb.r[q].tile_base) ri = q;
    ri = __builtin_amdgcn_readfirstlane(ri);  // uniform: keeps the rank's fields in scalar loads
    const GemmRank& g = gb.r[ri];
    const int local = tile - g.tile_base;
    if (g.tiles_n == 1) return PipeTile{ri, local * BM, 0, g.K};  // uniform: no division
    return PipeTile{ri, (local / g.tiles_n) * BM, (local % g.tiles_n) * BN, g.K};
  };

  // ---- producer: direct loads of K steps in tile order
  // Without pair sums every load of a tile addresses a uniform base (the tile's first A row,
  // its first B column) plus a 32-bit lane offset fixed for the tile (pipe_ok bounds them);
  // the pair-sum mode's gathered rows span the whole A, so it keeps 64-bit lane addresses.
  constexpr bool SADDR = !PS;
  int p_tile = t_first, p_k = 0, n_issued = 0;
  PipeTile pt{0, 0, 0, 32};
  const float* a_src[SADDR ? 1 : A_DMA];
  const float* a_src2[PS ? A_DMA : 1];  // second halves
  const float* b_src[SADDR ? 1 : B_DMA];
  const float* a_base = nullptr;
  const float* b_base = nullptr;
  uint32_t a_off[SADDR ? A_DMA : 1], b_off[SADDR ? B_DMA : 1];  // bytes
  auto p_setup = [&]() {
    if (p_tile >= t_end) return;
    pt = decode(p_tile);
    const GemmRank& g = gb.r[pt.ri];
    if constexpr (SADDR) {
      const int n0 = pt.r0 / g.comps, c00 = pt.r0 - n0 * g.comps;
      const float inv_comps = 1.0f / (float)g.comps;
      a_base = uniform_ptr(g.A + (int64_t)n0 * g.a_row);
      b_base = uniform_ptr(KB ? g.B : g.B + (int64_t)pt.c0 * g.K);
#pragma unroll
      for (int j = 0; j < A_DMA; ++j) {
        const int s = (j * 4 + wave) * 64 + lane;
        const int row = s >> 3, c = (s & 7) ^ pipe_swz(row);
        const int grow = min(pt.r0 + row, g.M - 1);
        // node and component counted from node n0: y / comps for y < BM + comps (exact in
        // float, as in the epilogue)
        const int y = c00 + (grow - pt.r0);
        const int dn = (int)(((float)y + 0.5f) * inv_comps), cc = y - dn * g.comps;
        a_off[j] = 4u * (uint32_t)((int64_t)dn * g.a_row + (int64_t)cc * g.a_comp + 4 * c);
      }
#pragma unroll
      for (int j = 0; j < B_DMA; ++j) {
        const int s = (j * 4 + wave) * 64 + lane;
        if constexpr (KB) {
          const int kk = s / BQ, p = (s % BQ) ^ pipe_kswz<MI>(kk);
          const int col = min(pt.c0 + 4 * p, g.N - 4);
          b_off[j] = 4u * (uint32_t)((int64_t)kk * g.N + col);
        } else {
          const int col = s >> 3, c = (s & 7) ^ pipe_swz(col);
          const int gcol = min(pt.c0 + col, g.N - 1);
          b_off[j] = 4u * (uint32_t)((int64_t)(gcol - pt.c0) * g.K + 4 * c);
        }
      }
      return;
    }
#pragma unroll
    for (int j = 0; j < A_DMA; ++j) {
      const int s = (j * 4 + wave) * 64 + lane;
      const int row = s >> 3, c = (s & 7) ^ pipe_swz(row);
      const int grow = min(pt.r0 + row, g.M - 1);
      if constexpr (PS) {
        if (g.a_lo) {
          // Gathered halves. Using these loads waits for every outstanding vector load, the
          // direct loads of the ring included (once per tile).
          a_src[j] = g.A + (int64_t)g.a_lo[grow] * g.a_row + 4 * c;
          a_src2[j] = g.A + (int64_t)g.a_hi[grow] * g.a_row + 4 * c;
          continue;
        }
      }
      const int n = grow / g.comps, cc = grow - n * g.comps;
      a_src[j] = g.A + (int64_t)n * g.a_row + (int64_t)cc * g.a_comp + 4 * c;
      if constexpr (PS) a_src2[j] = a_src[j] + g.K;
    }
#pragma unroll
    for (int j = 0; j < B_DMA; ++j) {
      const int s = (j * 4 + wave) * 64 + lane;
      if constexpr (KB) {
        const int kk = s / BQ, p = (s % BQ) ^ pipe_kswz<MI>(kk);
        const int col = min(pt.c0 + 4 * p, g.N - 4);
        b_src[j] = g.B + (int64_t)kk * g.N + col;
      } else {
        const int col = s >> 3, c = (s & 7) ^ pipe_swz(col);
        const int gcol = min(pt.c0 + col, g.N - 1);
        b_src[j] = g.B + (int64_t)gcol * g.K + 4 * c;
      }
    }
  };
  // LDS byte addresses of the stage being filled (as, bs); this wave's 16-byte chunks of a
  // direct load land at + 1024 (j * 4 + wave), kept in scalar registers
  const uint32_t wave_lds = 1024u * (uint32_t)__builtin_amdgcn_readfirstlane(wave);
  auto p_issue = [&](uint32_t as, uint32_t bs) {
    if (p_tile >= t_end) return;
    const int64_t bstep = KB ? (int64_t)p_k * gb.r[pt.ri].N : (int64_t)p_k;
    if constexpr (SADDR) {
      const float* sa = uniform_ptr(a_base + p_k);
      const float* sb = uniform_ptr(b_base + bstep);
#pragma unroll
      for (int j = 0; j < A_DMA; ++j) lds_dma16_s(sa, a_off[j], as + 4096u * j + wave_lds);
#pragma unroll
      for (int j = 0; j < B_DMA; ++j) lds_dma16_s(sb, b_off[j], bs + 4096u * j + wave_lds);
    } else {
#pragma unroll
    for (int j = 0; j < A_DMA; ++j) lds_dma16(a_src[j] + p_k, as + 4096u * j + wave_lds);
    if constexpr (PS) {
#pragma unroll
      for (int j = 0; j < A_DMA; ++j) lds_dma16(a_src2[j] + p_k, as + 4u * BM * 32 + 4096u * j + wave_lds);
    }
#pragma unroll
    for (int j = 0; j < B_DMA; ++j) lds_dma16(b_src[j] + bstep, bs + 4096u * j + wave_lds);
    }
    ++n_issued;
    p_k += 32;
    if (p_k >= pt.K) {
      p_k = 0;
      p_tile += t_step;
      p_setup();
    }
  };

  // ---- consumer
  int c_tile = t_first, c_k = 0, n_done = 0;
  PipeTile ct{0, 0, 0, 32};
  if (c_tile < t_end) ct = decode(c_tile);
  accv acc[FM][FN];
#pragma unroll
  for (int i = 0; i < FM; ++i)
#pragma unroll
    for (int j = 0; j < FN; ++j)
#pragma unroll
      for (int v = 0; v < NV; ++v) acc[i][j][v] = 0.f;

  // K mapping inside a 32-float step: 32x32x2 blocks take k = 8 s + 4 (lane / 32) + q in
  // k-pair q of quad s (4 quads); 16x16x4 blocks take k = 16 s + 4 (lane / 16) + q in k-quad
  // q of half s (2 halves). Either way a lane reads its four k values as one chunk.
  constexpr int NS = MI == 32 ? 4 : 2;
  const int kg = MI == 32 ? h : (lane >> 4);  // lane group along k
  // FIRST: the tile's first K step, whose first MFMA of each block starts from zero (the
  // accumulators need no clearing between tiles)
  auto compute = [&](const float* as, const float* bs, auto first_c) {
    constexpr bool FIRST = decltype(first_c)::value;
#pragma unroll
    for (int s4 = 0; s4 < NS; ++s4) {
      float4 a4[FM], b4[FN];
      const int ch = (MI == 32 ? 2 : 4) * s4 + kg;
#pragma unroll
      for (int i = 0; i < FM; ++i) {
        const int row = wm * TM + i * MI + (lane & (MI - 1));
        a4[i] = *reinterpret_cast<const float4*>(as + row * 32 + 4 * (ch ^ pipe_swz(row)));
        if constexpr (PS) {
          const float4 hi = *reinterpret_cast<const float4*>(as + BM * 32 + row * 32 + 4 * (ch ^ pipe_swz(row)));
          a4[i].x += hi.x; a4[i].y += hi.y; a4[i].z += hi.z; a4[i].w += hi.w;
        }
      }
#pragma unroll
      for (int j = 0; j < FN; ++j) {
        const int col = wn * TN + j * MI + (lane & (MI - 1));
        if constexpr (KB) {
          const int k = 4 * ch;  // rows k..k+3 share (k / 4) % 2
          const float* p = bs + k * BN + 4 * ((col >> 2) ^ pipe_kswz<MI>(k)) + (col & 3);
          b4[j] = make_float4(p[0], p[BN], p[2 * BN], p[3 * BN]);
        } else {
          b4[j] = *reinterpret_cast<const float4*>(bs + col * 32 + 4 * (ch ^ pipe_swz(col)));
        }
      }
#pragma unroll
      for (int q = 0; q < 4; ++q)
#pragma unroll
        for (int i = 0; i < FM; ++i)
#pragma unroll
          for (int j = 0; j < FN; ++j) {
            const float a = reinterpret_cast<const float*>(&a4[i])[q];
            const float b = reinterpret_cast<const float*>(&b4[j])[q];
            const accv c = (FIRST && s4 == 0 && q == 0) ? accv{} : acc[i][j];
            if constexpr (MI == 32) acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(a, b, c, 0, 0, 0);
            else acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
          }
    }
  };

  // Residual values are all loaded before the first store: a load into a register that a
  // pending store still reads would make the compiler wait for every outstanding load,
  // including the direct loads of the next K steps.
  auto epilogue = [&]() {
    const GemmRank& g = gb.r[ct.ri];
    const int M = g.M, N = g.N, comps = g.comps;
    const float scale = g.scale;
    // Rows are addressed from the tile's first node (a uniform base) with 32-bit byte
    // offsets (pipe_ok bounds them), columns j > 0 as immediate offsets: the stores and
    // residual loads need no per-access 64-bit address arithmetic.
    const int n0 = ct.r0 / comps, c00 = ct.r0 - n0 * comps;
    const float inv_comps = 1.0f / (float)comps;
    gfloat* const Dt = uniform_gptr(g.D + (int64_t)n0 * g.d_row);
    const bool has_r = g.R != nullptr;
    const gfloat* const Rt = uniform_gptr(has_r ? g.R + (int64_t)n0 * g.d_row : g.D);
    const int col0 = ct.c0 + wn * TN + (lane & (MI - 1));  // this lane's column in block j = 0
    const bool all_cols = ct.c0 + BN <= N;                  // uniform
    float bias_v[FN];
#pragma unroll
    for (int j = 0; j < FN; ++j) bias_v[j] = (gb.bias && col0 + j * MI < N) ? gb.bias[col0 + j * MI] : 0.f;
    // block rows of acc value v = 4 vg + q: 8 vg + 4 (lane / 32) + q (32x32), 4 (lane / 16) + q (16x16)
    uint32_t roff[FM][NV];
    bool rok[FM][NV];
#pragma unroll
    for (int i = 0; i < FM; ++i) {
#pragma unroll
      for (int vg = 0; vg < NV / 4; ++vg) {
        const int rl = wm * TM + i * MI + (MI == 32 ? 8 * vg + 4 * h : 4 * (lane >> 4));
        // node and component of row r0 + rl, counted from node n0: y / comps for y < BM + comps
        // (exact in float: (y + 1/2) / comps is at least 1 / (2 comps) from an integer)
        const int y = c00 + rl;
        int dn = (int)(((float)y + 0.5f) * inv_comps), c = y - dn * comps;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          rok[i][4 * vg + q] = ct.r0 + rl + q < M;
          roff[i][4 * vg + q] = 4u * (uint32_t)(dn * (int)g.d_row + c * (int)g.d_comp + col0);
          if (++c == comps) {
            c = 0;
            ++dn;
          }
        }
      }
    }
    auto d_at = [&](uint32_t off, int j) { return reinterpret_cast<gfloat*>(reinterpret_cast<gchar*>(Dt) + off) + j * MI; };
    auto r_at = [&](uint32_t off, int j) {
      return reinterpret_cast<const gfloat*>(reinterpret_cast<const gchar*>(Rt) + off) + j * MI;
    };
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
      for (int j = 0; j < FN; ++j)
#pragma unroll
        for (int v = 0; v < NV; ++v) acc[i][j][v] = fmaf(acc[i][j][v], scale, bias_v[j]);
    if (has_r) {
      // every residual value is loaded (rows out of range read the tile's first row, columns
      // out of range nothing) before the first store: a load into a register that a pending
      // store still reads makes the compiler wait for all outstanding loads, the direct loads
      // of the next K steps included
      float rv[FM][NV][FN];
#pragma unroll
      for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int v = 0; v < NV; ++v)
#pragma unroll
          for (int j = 0; j < FN; ++j)
            rv[i][v][j] = (all_cols || col0 + j * MI < N) ? *r_at(rok[i][v] ? roff[i][v] : 0u, j) : 0.f;
#pragma unroll
      for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int v = 0; v < NV; ++v)
#pragma unroll
          for (int j = 0; j < FN; ++j) acc[i][j][v] += rv[i][v][j];
    }
    // nontemporal stores: the output streams to HBM without displacing the operands the next
    // tiles read from L2 (K = 128 maps 77 -> 81 TFLOP/s alone; 25k-atom step 26.31 -> 26.14 ms)
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
      for (int v = 0; v < NV; ++v) {
        if (!rok[i][v]) continue;
#pragma unroll
        for (int j = 0; j < FN; ++j)
          if (all_cols || col0 + j * MI < N) __builtin_nontemporal_store(acc[i][j][v], d_at(roff[i][v], j));
      }
  };

  // One K step: wait for this wave's loads of the step (the step issued after it may stay in
  // flight), barrier (every wave's loads have landed and every wave is done with the stage
  // the new loads overwrite), refill that stage, multiply, and finish the tile at its end.
  bool more = c_tile < t_end;
  auto step = [&](const float* as, const float* bs, uint32_t pas, uint32_t pbs) {
    if (n_issued - n_done >= 2) __builtin_amdgcn_s_waitcnt(FC_WAITCNT_IMM(L, 0));
    else __builtin_amdgcn_s_waitcnt(FC_WAITCNT_IMM(0, 0));
    pipe_barrier();
    p_issue(pas, pbs);
    if (c_k == 0) compute(as, bs, std::true_type{});
    else compute(as, bs, std::false_type{});
    ++n_done;
    c_k += 32;
    if (c_k >= ct.K) {
      epilogue();
      c_k = 0;
      c_tile += t_step;
      more = c_tile < t_end;
      if (more) ct = decode(c_tile);
    }
  };

  p_setup();
  p_issue(lds_addr(As0), lds_addr(Bs0));
  p_issue(lds_addr(As1), lds_addr(Bs1));
  while (more) {
    step(As0, Bs0, lds_addr(As2), lds_addr(Bs2));
    if (!more) break;
    step(As1, Bs1, lds_addr(As0), lds_addr(Bs0));
    if (!more) break;
    step(As2, Bs2, lds_addr(As1), lds_addr(Bs1));
  }
}

static int device_cu_count() {
  static int cus[64] = {0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  if (cus[dev] <= 0) {
    int v = 0;
    if (hipDeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || v <= 0) v = 256;
    cus[dev] = v;
  }
  return cus[dev];
}

static bool pipe_ok(const GemmBatch& gb, int n_ranks) {
  if (gb.act || gb.act_bwd) return false;
  for (int l = 0; l < n_ranks; ++l) {
    const GemmRank& g = gb.r[l];
    if (g.pre || g.P || g.K < 32 || (g.K & 31) || (g.a_row & 3) || (g.a_comp & 3)) return false;
    // 32-bit byte offsets of a tile's loads from its first A row / B column (128-row tiles)
    if ((int64_t)129 * g.a_row + (int64_t)g.comps * g.a_comp + g.K >= (int64_t(1) << 30)) return false;
    if ((int64_t)128 * g.K >= (int64_t(1) << 30) || (int64_t)32 * g.N + g.N >= (int64_t(1) << 30)) return false;
    // and of the epilogue's stores from the tile's first output node
    if ((int64_t)129 * g.d_row + (int64_t)g.comps * g.d_comp + g.N >= (int64_t(1) << 30)) return false;
    if (g.d_row > 0x7fffffff || g.d_comp > 0x7fffffff) return false;
    if (((uintptr_t)g.A & 15) || ((uintptr_t)g.B & 15)) return false;
    if (!gb.trans_b && (g.N & 3)) return false;
  }
  return true;
}

template <int BM, int BN, int WM, int WN, int MI, bool PS = false>
int launch_pipe_cfg(GemmBatch gb, int n_ranks, hipStream_t s) {
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
  int64_t grid = 2 * (int64_t)device_cu_count();
  if (grid > total) grid = total;
  if (grid >= 8) grid -= grid % 8;
  if (gb.trans_b) hipLaunchKernelGGL((gemm_pipe_kernel<BM, BN, WM, WN, MI, false, PS>), dim3((unsigned)grid), dim3(256), 0, s, gb);
  else hipLaunchKernelGGL((gemm_pipe_kernel<BM, BN, WM, WN, MI, true, PS>), dim3((unsigned)grid), dim3(256), 0, s, gb);
  FC_LAUNCH_CHECK();
  return FC_OK;
}

template <int BM, int BN, int WM, int WN, int NBUF>
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
  if (gb.trans_b) hipLaunchKernelGGL((gemm_kernel<BM, BN, WM, WN, NBUF, false>), dim3((unsigned)grid), dim3(256), 0, s, gb);
  else hipLaunchKernelGGL((gemm_kernel<BM, BN, WM, WN, NBUF, true>), dim3((unsigned)grid), dim3(256), 0, s, gb);
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
  // Measured on the model's shapes (M = n (2l+1) rows, K and N of 128 or paths x 128):
  // 128 x 64 tiles (waves stacked along M) for the wider input gradients, 64 x 128
  // (waves side by side along N) for the forward. Both hold four workgroups per CU, whose
  // prologues and epilogues overlap each other's MFMA work better than two 128 x 128 tiles.
  // Maps at most 64 wide (the 64-channel models, radial hidden layers) take 64 x 64
  // tiles: twice the workgroups, so short-K launches fill the chip.
  // Measured on the model's shapes (MI355X, fp32): the pipelined kernel with 16x16x4 blocks
  // runs 3-13% faster than the register-staged one; 128 x 64 tiles for maps at most 64 wide
  // (the radial output layer's input gradient: 112 vs 99 TFLOP/s), 64 x 128 otherwise.
  // Launches with fewer 128-row tiles than two per CU (the 1,536-atom water box) take 64 x 64
  // tiles instead, for twice the workgroups.
  if (gb.pair_sum) {  // forward layout, at most 64 output columns, pipelined kernel only
    if (!gb.trans_b || max_n > 64 || !pipe_ok(gb, n_ranks)) return FC_ERR_SHAPE;
    return launch_pipe_cfg<64, 64, 2, 2, 16, true>(gb, n_ranks, s);
  }
  if (pipe_ok(gb, n_ranks)) {
    if (max_n <= 64) {
      int64_t tiles128 = 0;
      for (int l = 0; l < n_ranks; ++l) tiles128 += (gb.r[l].M + 127) / 128;
      if (tiles128 < 2 * (int64_t)device_cu_count()) return launch_pipe_cfg<64, 64, 2, 2, 16>(gb, n_ranks, s);
      return launch_pipe_cfg<128, 64, 4, 1, 16>(gb, n_ranks, s);
    }
    return launch_pipe_cfg<64, 128, 2, 2, 16>(gb, n_ranks, s);
  }
  if (max_n <= 64) return launch_gemm_cfg<64, 64, 2, 2, 1>(gb, n_ranks, s);
  if (!gb.trans_b) return launch_gemm_cfg<128, 64, 4, 1, 1>(gb, n_ranks, s);
  return launch_gemm_cfg<64, 128, 1, 4, 1>(gb, n_ranks, s);
}

// dst[r, off:off+width] = src ? src[r, off:off+width] : 0 (same row stride): one wave per
// row, lanes along the columns (no per-element division)
__global__ void fill_rows_kernel(int64_t rows, int64_t row_stride, int64_t off, int64_t width,
                                 const float* __restrict__ src, float* __restrict__ dst) {
  const int64_t r = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (r >= rows) return;
  const int64_t base = r * row_stride + off;
  for (int64_t c = threadIdx.x & 63; c < width; c += 64) dst[base + c] = src ? src[base + c] : 0.f;
}

// Output columns the map does not produce: zero, or the residual's values.
int fill_columns(int64_t rows, int64_t row_stride, int64_t off, int64_t width, const float* residual, float* dst,
                 hipStream_t s) {
  if (rows * width == 0 || residual == dst) return FC_OK;
  hipLaunchKernelGGL(fill_rows_kernel, dim3((unsigned)((rows + 3) / 4)), dim3(256), 0, s, rows, row_stride, off, width,
                     residual, dst);
  FC_LAUNCH_CHECK();
  return FC_OK;
}

static int check_linear(const fc_linear_desc* d) {
  if (!d) return FC_ERR_NULL;
  if (d->in_l_max < 0 || d->out_l_max < 0) return FC_ERR_BAD_DESC;
  if (d->in_l_max >= FC_MAX_RANKS || d->out_l_max >= FC_MAX_RANKS) return FC_ERR_UNSUPPORTED_L;
  if (d->in_features < 1 || d->out_features < 1) return FC_ERR_BAD_DESC;
  const int common = d->in_l_max < d->out_l_max ? d->in_l_max : d->out_l_max;
  for (int l = 0; l <= d->in_l_max; ++l)
    if (d->in_paths[l] < 1) return FC_ERR_BAD_DESC;
  for (int l = 0; l <= common; ++l)
    if (!d->weight[l]) return FC_ERR_NULL;
  return FC_OK;
}

struct LinearLayout {
  int64_t in_dim, out_dim, in_off[FC_MAX_RANKS], out_off[FC_MAX_RANKS];
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

extern "C" int fc_linear_fwd(const fc_linear_desc* d, int64_t n, const float* x, float alpha,
                             const float* residual, float* out, void* stream) {
  int st = check_linear(d);
  if (st != FC_OK) return st;
  if (n == 0) return FC_OK;
  if (!x || !out) return FC_ERR_NULL;
  if (n * (2 * FC_MAX_RANKS - 1) > 0x7fffffff) return FC_ERR_SHAPE;
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
    g.R = residual ? residual + L.out_off[l] : nullptr;
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
    return fill_columns(n, L.out_dim, L.out_off[L.common + 1], L.out_dim - L.out_off[L.common + 1], residual, out,
                        s);
  return FC_OK;
}

extern "C" int fc_linear_dgrad(const fc_linear_desc* d, int64_t n, const float* go, float alpha,
                               const float* residual, float* gx, void* stream) {
  int st = check_linear(d);
  if (st != FC_OK) return st;
  if (n == 0) return FC_OK;
  if (!go || !gx) return FC_ERR_NULL;
  if (n * (2 * FC_MAX_RANKS - 1) > 0x7fffffff) return FC_ERR_SHAPE;
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
    g.R = residual ? residual + L.in_off[l] : nullptr;
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
    return fill_columns(n, L.in_dim, L.in_off[L.common + 1], L.in_dim - L.in_off[L.common + 1], residual, gx, s);
  return FC_OK;
}

namespace fc {

// ---- Wide output, K = 64: out (n x m) = scale * x (n x 64) @ W^T, W (m x 64), m >> 64 (the
// radial MLP's output layer, m = paths x channels). Writing the output is as costly as the
// MFMA work here, so each workgroup keeps its 128 x 64 block of x in LDS and walks the
// output columns in chunks of 64: the next weight chunk is loaded while the current one
// is multiplied, and the previous chunk's results are stored in between the MFMAs.
// MFMA step s (of 32) contracts k = s in lanes 0-31 and k = 32 + s in lanes 32-63, so
// rows sit in LDS in natural k order (a float4 from global memory is written as is, no
// register shuffle) and a lane reads four steps with one 128-bit load; the pitch of 68
// floats (17 x 16 B) keeps those reads conflict-free. Four waves stacked along the rows,
// 32 x 64 outputs each per chunk.
constexpr int WIDE_BM = 128, WIDE_BN = 64, WIDE_K = 64, WIDE_P = 68;

// Output part shared by the wide kernels: the x block of rows r0 .. r0 + 127 is in As
// (natural k order, pitch WIDE_P); Bs holds two weight-chunk buffers. Ends with no
// barrier pending; every thread of the workgroup must call it.
template <bool GUARD>
__device__ __forceinline__ void wide_body(const float* As, float (*Bs)[WIDE_BN * WIDE_P], int64_t n, int m,
                                          const float* __restrict__ w, float scale, float* __restrict__ out,
                                          int64_t r0) {
  const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
  auto put4 = [&](float* base, int q, int k4, float4 v) {
    *reinterpret_cast<float4*>(base + q * WIDE_P + k4) = v;
  };
  float4 rb[4];
  auto load_b = [&](int c0) {  // 64 weight rows x 16 float4, 4 per thread
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int e = t + 256 * i, q = e >> 4, k4 = (e & 15) * 4;
      const int col = c0 + q < m ? c0 + q : m - 1;
      rb[i] = *reinterpret_cast<const float4*>(w + (int64_t)col * WIDE_K + k4);
    }
  };
  // the weight chunk goes to LDS scaled, out = x (W scale)^T (the order of F.linear(x, W * s))
  auto store_b = [&](int buf) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int e = t + 256 * i;
      put4(Bs[buf], e >> 4, (e & 15) * 4,
           make_float4(rb[i].x * scale, rb[i].y * scale, rb[i].z * scale, rb[i].w * scale));
    }
  };
  load_b(0);
  store_b(0);
  __syncthreads();

  const int half = (lane >> 5) * (WIDE_K / 2);  // k offset of this half-wave
  const float* as = As + (wave * 32 + (lane & 31)) * WIDE_P + half;
  const int nch = (m + WIDE_BN - 1) / WIDE_BN;
  // output rows of this lane: r0 + 32 wave + 8 (v/4) + 4 (lane/32) + v%4
  const int64_t rl = r0 + wave * 32 + 4 * (lane >> 5);
  // Unguarded blocks: the element offset of row v (of this lane's 16) from the block's first
  // element is fixed for the whole block, so a store is a wave-uniform base (the block and the
  // chunk's column) plus a precomputed 32-bit offset, with no per-store address arithmetic.
  // (The caller keeps 128 m 4 below 2^31.)
  uint32_t voff[GUARD ? 1 : 16];  // bytes
  if constexpr (!GUARD) {
#pragma unroll
    for (int v = 0; v < 16; ++v)
      voff[v] = (uint32_t)((wave * 32 + 4 * (lane >> 5) + 8 * (v >> 2) + (v & 3)) * m + (lane & 31)) * 4u;
  }
  float* const blk = out + r0 * m;
  // results of output row v (of this lane's 16) and column block j of a chunk at column c0
  auto store_one = [&](const floatx16 (&res)[2], int c0, int v, int j) {
    if constexpr (GUARD) {
      const int64_t row = rl + 8 * (v >> 2) + (v & 3);
      const int col = c0 + j * 32 + (lane & 31);
      if (row < n && col < m) out[row * m + col] = res[j][v];
    } else {
      *reinterpret_cast<float*>(reinterpret_cast<char*>(blk + c0 + j * 32) + voff[v]) = res[j][v];
    }
  };
  // One chunk into `cur`; the previous chunk's results (`prv`, complete by now) are
  // stored in between this chunk's MFMAs, so the wave keeps the matrix core fed while
  // its stores issue (two accumulator sets used alternately).
  auto chunk = [&](int ch, floatx16 (&cur)[2], const floatx16 (&prv)[2], bool have_prev) {
    const int c0 = ch * WIDE_BN, buf = ch & 1;
    if (ch + 1 < nch) load_b(c0 + WIDE_BN);
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int v = 0; v < 16; ++v) cur[j][v] = 0.f;
    const float* bs = Bs[buf] + (lane & 31) * WIDE_P + half;
    // operands of MFMA group s4 + 1 are read from LDS while group s4 multiplies
    float4 a4n = *reinterpret_cast<const float4*>(as), b4n[2];
#pragma unroll
    for (int j = 0; j < 2; ++j) b4n[j] = *reinterpret_cast<const float4*>(bs + j * 32 * WIDE_P);
#pragma unroll
    for (int s4 = 0; s4 < 8; ++s4) {  // 32 MFMA steps, four per 128-bit read
      const float4 a4 = a4n;
      float4 b4[2] = {b4n[0], b4n[1]};
      if (s4 + 1 < 8) {
        const int o = 4 * (s4 + 1);
        a4n = *reinterpret_cast<const float4*>(as + o);
#pragma unroll
        for (int j = 0; j < 2; ++j) b4n[j] = *reinterpret_cast<const float4*>(bs + j * 32 * WIDE_P + o);
      }
      __builtin_amdgcn_sched_barrier(0);  // keep those reads ahead of this group's MFMAs
#pragma unroll
      for (int q = 0; q < 4; ++q)
#pragma unroll
        for (int j = 0; j < 2; ++j) {
          cur[j] = __builtin_amdgcn_mfma_f32_32x32x2f32(reinterpret_cast<const float*>(&a4)[q],
                                                        reinterpret_cast<const float*>(&b4[j])[q], cur[j], 0, 0, 0);
          if (have_prev && (q & 1) == 0) store_one(prv, c0 - WIDE_BN, 2 * s4 + (q >> 1), j);
        }
    }
    if (ch + 1 < nch) {
      store_b(buf ^ 1);  // the other buffer was last read in the previous chunk
      __syncthreads();
    }
  };
  floatx16 r0acc[2], r1acc[2];
  for (int ch = 0; ch < nch; ch += 2) {
    chunk(ch, r0acc, r1acc, ch > 0);
    if (ch + 1 < nch) chunk(ch + 1, r1acc, r0acc, true);
  }
  const int last = nch - 1;
#pragma unroll
  for (int v = 0; v < 16; ++v)
#pragma unroll
    for (int j = 0; j < 2; ++j) store_one((last & 1) ? r1acc : r0acc, last * WIDE_BN, v, j);
}

// GUARD = false: every row and column of the block is in range (m a multiple of 64), so
// the stores are unconditional and the compiler can count them as outstanding rather
// than wait for them before the next weight chunk is written to LDS. The last, partial
// row block runs as a separate GUARD = true launch. (The radial MLP forward instead takes
// the guarded body for its partial block inside the one launch; there it costs no spills.)
template <bool GUARD>
__global__ void __launch_bounds__(256, 2) gemm_wide_kernel(int64_t n, int m, const float* __restrict__ x,
                                                            const float* __restrict__ w, float scale,
                                                            float* __restrict__ out, int64_t first_block) {
  __shared__ __attribute__((aligned(16))) float As[WIDE_BM * WIDE_P];
  __shared__ __attribute__((aligned(16))) float Bs[2][WIDE_BN * WIDE_P];
  const int t = threadIdx.x;
  const int64_t r0 = (first_block + blockIdx.x) * WIDE_BM;
  // x block: 128 rows x 16 float4, 8 per thread; rows past n read row n-1 (never stored)
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const int e = t + 256 * i, q = e >> 4, k4 = (e & 15) * 4;
    int64_t row = r0 + q;
    row = row < n ? row : n - 1;
    *reinterpret_cast<float4*>(As + q * WIDE_P + k4) = *reinterpret_cast<const float4*>(x + row * WIDE_K + k4);
  }
  wide_body<GUARD>(As, Bs, n, m, w, scale, out, r0);
}

// ---- Radial MLP with two hidden layers of 64 (reference InteractionLayer.radial_mlp,
// src/flashcart/nn/layers.py:258-267, applied at :357-363):
//   pre1 = s0 x W0^T, h1 = silu(pre1), pre2 = s1 h1 W1^T, h2 = silu(pre2), out = s2 h2 W2^T
// with silu the rescaled SiLU and x (n, n_in), n_in <= 64. The forward forms h1 and h2 of a
// 128-row block in LDS and hands h2 to the wide output part, so neither hidden layer goes
// through HBM. The backward (input gradient only) recomputes the hidden layers from x
// (n_in floats per row) instead of reading saved pre-activations.

// acc[j] (j < NJ) = A rows of this wave (as) x weight rows of column block j (bs + 32 j
// rows), k = 0..63: MFMA step s contracts k = s (lanes 0-31) and k = 32 + s (lanes 32-63).
// Only the first ns4 groups of four steps run: with K <= 32 the rest multiply zero padding
// (K = n_in, the first hidden layer), so ns4 = ceil(K / 4) there and 8 otherwise.
template <int NJ>
__device__ __forceinline__ void mfma_k64(const float* as, const float* bs, floatx16 (&acc)[2], int ns4 = 8) {
#pragma unroll
  for (int j = 0; j < NJ; ++j)
#pragma unroll
    for (int v = 0; v < 16; ++v) acc[j][v] = 0.f;
  // operands of group s4 + 1 are read from LDS while group s4 multiplies
  float4 a4n = *reinterpret_cast<const float4*>(as), b4n[NJ];
#pragma unroll
  for (int j = 0; j < NJ; ++j) b4n[j] = *reinterpret_cast<const float4*>(bs + j * 32 * WIDE_P);
#pragma unroll
  for (int s4 = 0; s4 < 8; ++s4) {
    if (s4 >= ns4) break;  // uniform
    const float4 a4 = a4n;
    float4 b4[NJ];
#pragma unroll
    for (int j = 0; j < NJ; ++j) b4[j] = b4n[j];
    if (s4 + 1 < ns4) {
      a4n = *reinterpret_cast<const float4*>(as + 4 * (s4 + 1));
#pragma unroll
      for (int j = 0; j < NJ; ++j) b4n[j] = *reinterpret_cast<const float4*>(bs + j * 32 * WIDE_P + 4 * (s4 + 1));
    }
    __builtin_amdgcn_sched_barrier(0);  // keep those reads ahead of this group's MFMAs
#pragma unroll
    for (int q = 0; q < 4; ++q)
#pragma unroll
      for (int j = 0; j < NJ; ++j)
        acc[j] = __builtin_amdgcn_mfma_f32_32x32x2f32(reinterpret_cast<const float*>(&a4)[q],
                                                      reinterpret_cast<const float*>(&b4[j])[q], acc[j], 0, 0, 0);
  }
}

// The same product with B stored the other way round: bt = W + (lane & 31) + half * WIDE_P for a
// weight square W[k][j] (k-major rows), so lane j of block jb reads W[k][jb * 32 + j] for its four
// k values (four scalar LDS reads, the same bytes as one float4): the input gradients multiply by
// the weight matrices the forward staged, without staging their transposes.
template <int NJ>
__device__ __forceinline__ void mfma_k64_t(const float* as, const float* bt, floatx16 (&acc)[2]) {
#pragma unroll
  for (int j = 0; j < NJ; ++j)
#pragma unroll
    for (int v = 0; v < 16; ++v) acc[j][v] = 0.f;
  auto read_b = [&](int s4, float4 (&b)[NJ]) {
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
      const float* p = bt + 4 * s4 * WIDE_P + j * 32;
      b[j] = make_float4(p[0], p[WIDE_P], p[2 * WIDE_P], p[3 * WIDE_P]);
    }
  };
  float4 a4n = *reinterpret_cast<const float4*>(as), b4n[NJ];
  read_b(0, b4n);
#pragma unroll
  for (int s4 = 0; s4 < 8; ++s4) {
    const float4 a4 = a4n;
    float4 b4[NJ];
#pragma unroll
    for (int j = 0; j < NJ; ++j) b4[j] = b4n[j];
    if (s4 + 1 < 8) {
      a4n = *reinterpret_cast<const float4*>(as + 4 * (s4 + 1));
      read_b(s4 + 1, b4n);
    }
    __builtin_amdgcn_sched_barrier(0);  // keep those reads ahead of this group's MFMAs
#pragma unroll
    for (int q = 0; q < 4; ++q)
#pragma unroll
      for (int j = 0; j < NJ; ++j)
        acc[j] = __builtin_amdgcn_mfma_f32_32x32x2f32(reinterpret_cast<const float*>(&a4)[q],
                                                      reinterpret_cast<const float*>(&b4[j])[q], acc[j], 0, 0, 0);
  }
}

// Row (within the wave's 32 rows) of accumulator element v of this lane.
__device__ __forceinline__ int acc_row(int v, int lane) { return 8 * (v >> 2) + 4 * (lane >> 5) + (v & 3); }

__device__ __forceinline__ float silu_r(float z) { return kSiluScale * z * sigmoidf_(z); }
__device__ __forceinline__ float silu_r_grad(float z) {
  const float sg = sigmoidf_(z);
  return kSiluScale * sg * (1.0f + z * (1.0f - sg));
}

// x block (rows r0 .. r0 + 127 that exist; they are contiguous in x) -> As, zero-padded to 64
// columns; rows past n stay zero (never stored). W0 (64 x n_in) -> B0 and W1 (64 x 64) -> B1 as
// weight rows (zero-padded k). Every thread issues all of its global loads before its first LDS
// store, so the load latency is paid once.
__device__ __forceinline__ void mlp_stage_x(float* As, int64_t n, int n_in, const float* __restrict__ x, int64_t r0) {
  const int t = threadIdx.x;
  const int rows = n - r0 < WIDE_BM ? (int)(n - r0) : WIDE_BM;
  const int cnt = rows * n_in;
  const float* xb = x + r0 * n_in;
  // row of element e: e / n_in, exact in float for e < 2^13 ((e + 1/2) / n_in is at least
  // 1 / (2 n_in) from an integer), without an integer division per element
  const float inv_in = 1.0f / (float)n_in;
  // in chunks of eight values per thread (one chunk for up to 16 inputs), so few registers stay
  // reserved for the staging
  for (int base = 0; base < WIDE_BM * n_in; base += 8 * 256) {
    float v[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int e = base + t + 256 * i;
      v[i] = e < cnt ? xb[e] : 0.f;
    }
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int e = base + t + 256 * i;
      if (e < WIDE_BM * n_in) {
        const int q = (int)(((float)e + 0.5f) * inv_in);
        As[q * WIDE_P + (e - q * n_in)] = v[i];
      }
    }
  }
  for (int e = t; e < WIDE_BM * (WIDE_K - n_in); e += 256) {
    const int q = e / (WIDE_K - n_in);
    As[q * WIDE_P + n_in + (e - q * (WIDE_K - n_in))] = 0.f;
  }
}

__device__ __forceinline__ void mlp_stage_weights(float* B0, float* B1, int n_in, const float* __restrict__ w0,
                                                  const float* __restrict__ w1) {
  const int t = threadIdx.x;
  float a[16], b[16];
#pragma unroll
  for (int i = 0; i < 16; ++i) {  // element e = (r, c) of a 64 x 64 square, c = e & 63 along memory
    const int e = t + 256 * i, r = e >> 6, c = e & 63;
    a[i] = w1[r * 64 + c];
    b[i] = c < n_in ? w0[r * n_in + c] : 0.f;
  }
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    const int e = t + 256 * i, r = e >> 6, c = e & 63;
    B0[r * WIDE_P + c] = b[i];  // W0 row r (output), k = c
    B1[r * WIDE_P + c] = a[i];  // W1 row r, k = c
  }
}

// The wave's 32 x 64 accumulator block -> f(value) into its own rows of As.
template <class F>
__device__ __forceinline__ void acc_to_rows(const floatx16 (&acc)[2], float* As, int wave, int lane, F f) {
#pragma unroll
  for (int j = 0; j < 2; ++j)
#pragma unroll
    for (int v = 0; v < 16; ++v)
      As[(wave * 32 + acc_row(v, lane)) * WIDE_P + j * 32 + (lane & 31)] = f(acc[j][v]);
}

// HIDDEN: stop after the second hidden layer and write its activation h2 (n x 64) instead of
// the output layer (the first interaction layer's species density takes h2 itself).
template <bool GUARD, bool HIDDEN = false>
__global__ void __launch_bounds__(256, 2) radial_mlp_fwd_kernel(int64_t n, int n_in, const float* __restrict__ x,
                                                                 const float* __restrict__ w0, float s0,
                                                                 const float* __restrict__ w1, float s1, int m,
                                                                 const float* __restrict__ w2, float s2,
                                                                 float* __restrict__ out, int64_t first_block) {
  __shared__ __attribute__((aligned(16))) float As[WIDE_BM * WIDE_P];
  __shared__ __attribute__((aligned(16))) float Bs[2][WIDE_BN * WIDE_P];
  const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
  const int64_t r0 = (first_block + blockIdx.x) * WIDE_BM;
  mlp_stage_x(As, n, n_in, x, r0);
  mlp_stage_weights(Bs[0], Bs[1], n_in, w0, w1);
  __syncthreads();
  const int half = (lane >> 5) * (WIDE_K / 2);
  const float* as = As + (wave * 32 + (lane & 31)) * WIDE_P + half;
  floatx16 acc[2];
  const int ns4_in = n_in <= 32 ? (n_in + 3) / 4 : 8;
  mfma_k64<2>(as, Bs[0] + (lane & 31) * WIDE_P + half, acc, ns4_in);
  __syncthreads();  // every wave's reads of the x rows are done (each wave rewrites only its own rows)
  acc_to_rows(acc, As, wave, lane, [&](float a) { return silu_r(a * s0); });
  __syncthreads();
  mfma_k64<2>(as, Bs[1] + (lane & 31) * WIDE_P + half, acc);
  if constexpr (HIDDEN) {
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        const int64_t row = r0 + wave * 32 + acc_row(v, lane);
        if (row < n) out[row * 64 + j * 32 + (lane & 31)] = silu_r(acc[j][v] * s1);
      }
    return;
  }
  __syncthreads();  // reads of h1 and of both weight buffers done before they are overwritten
  acc_to_rows(acc, As, wave, lane, [&](float a) { return silu_r(a * s1); });
  __syncthreads();
  if (GUARD || r0 + WIDE_BM > n) wide_body<true>(As, Bs, n, m, w2, s2, out, r0);
  else wide_body<false>(As, Bs, n, m, w2, s2, out, r0);
}

// Input gradient of the two hidden layers: given gh2 = dL/dh2 (n, 64),
//   dpre2 = gh2 * silu'(pre2), dh1 = s1 dpre2 W1, dpre1 = dh1 * silu'(pre1), dx = s0 dpre1 W0.
// PAIRS: gh2 holds two rows per input row (rows 2r and 2r + 1, summed).
template <bool PAIRS = false>
__global__ void __launch_bounds__(256, 2) radial_mlp_bwd_kernel(int64_t n, int n_in, const float* __restrict__ x,
                                                                 const float* __restrict__ w0, float s0,
                                                                 const float* __restrict__ w1, float s1,
                                                                 const float* __restrict__ gh2,
                                                                 float* __restrict__ gx) {
  __shared__ __attribute__((aligned(16))) float As[WIDE_BM * WIDE_P];
  __shared__ __attribute__((aligned(16))) float B0[WIDE_BN * WIDE_P];
  __shared__ __attribute__((aligned(16))) float B1[WIDE_BN * WIDE_P];
  const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
  // Persistent: workgroup b takes row blocks b, b + G, ...; the weights are staged once, and the
  // next block's dL/dh2 loads while the current block's last two products run.
  const int64_t nblk = (n + WIDE_BM - 1) / WIDE_BM;
  int64_t blk = blockIdx.x;
  if (blk >= nblk) return;  // uniform
  // this lane's dL/dh2 values of block b (accumulator layout); rows past n contribute nothing
  auto load_g2 = [&](int64_t b, float (&g)[2][16]) {
    const int64_t rb = b * WIDE_BM;
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        const int64_t row = rb + wave * 32 + acc_row(v, lane);
        if constexpr (PAIRS)
          g[j][v] = row < n ? gh2[2 * row * 64 + j * 32 + (lane & 31)] + gh2[(2 * row + 1) * 64 + j * 32 + (lane & 31)]
                            : 0.f;
        else
          g[j][v] = row < n ? gh2[row * 64 + j * 32 + (lane & 31)] : 0.f;
      }
  };
  float g2[2][16];
  load_g2(blk, g2);
  mlp_stage_weights(B0, B1, n_in, w0, w1);
  const int half = (lane >> 5) * (WIDE_K / 2);
  const float* as = As + (wave * 32 + (lane & 31)) * WIDE_P + half;
  // dh1 = dpre2 W1 and dx = dpre1 W0 read the weight rows staged for the forward layers
  const float* w1t = B1 + (lane & 31) + half * WIDE_P;
  const float* w0t = B0 + (lane & 31) + half * WIDE_P;
  const int ns4_in = n_in <= 32 ? (n_in + 3) / 4 : 8;
  const int nj = n_in <= 32 ? 1 : 2;  // dx has n_in columns: one 32-column block when n_in <= 32
  for (; blk < nblk; blk += gridDim.x) {
    const int64_t r0 = blk * WIDE_BM;
    mlp_stage_x(As, n, n_in, x, r0);
    __syncthreads();  // x rows (and, the first time, the weights) staged
    floatx16 acc[2], d1[2];
    mfma_k64<2>(as, B0 + (lane & 31) * WIDE_P + half, acc, ns4_in);
    // one sigmoid per pre-activation serves both silu'(pre1) (kept) and h1 = silu(pre1) (to LDS)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        const float z = acc[j][v] * s0, sg = sigmoidf_(z);
        d1[j][v] = kSiluScale * sg * (1.0f + z * (1.0f - sg));
        acc[j][v] = kSiluScale * z * sg;
      }
    __syncthreads();
    acc_to_rows(acc, As, wave, lane, [](float a) { return a; });
    __syncthreads();
    mfma_k64<2>(as, B1 + (lane & 31) * WIDE_P + half, acc);
    // dpre2 = gh2 * silu'(pre2)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[j][v] = g2[j][v] * silu_r_grad(acc[j][v] * s1);
    if (blk + gridDim.x < nblk) load_g2(blk + gridDim.x, g2);  // in flight during the rest of this block
    __syncthreads();  // reads of h1 done: stage dpre2
    acc_to_rows(acc, As, wave, lane, [](float a) { return a; });
    __syncthreads();
    mfma_k64_t<2>(as, w1t, acc);
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[j][v] = acc[j][v] * s1 * d1[j][v];
    __syncthreads();
    acc_to_rows(acc, As, wave, lane, [](float a) { return a; });
    __syncthreads();
    if (nj == 1) mfma_k64_t<1>(as, w0t, acc);
    else mfma_k64_t<2>(as, w0t, acc);
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        const int64_t row = r0 + wave * 32 + acc_row(v, lane);
        const int col = j * 32 + (lane & 31);
        if (j < nj && row < n && col < n_in) gx[row * n_in + col] = acc[j][v] * s0;
      }
    __syncthreads();  // every wave's reads of this block's rows done before the next block's x
  }
}

}  // namespace fc

extern "C" int fc_dense_fwd(int64_t n, int32_t k, int32_t m, const float* x, const float* w, float scale,
                            const float* bias, int32_t act, float* pre_act, float* out, void* stream) {
  if (n < 0 || k < 1 || m < 1 || act < 0 || act > 1) return FC_ERR_BAD_DESC;
  if (n == 0) return FC_OK;
  if (!x || !w || !out) return FC_ERR_NULL;
  if (n > 0x7fffffff) return FC_ERR_SHAPE;
  if (k == WIDE_K && m >= 4 * WIDE_BN && !bias && act == 0 && ((uintptr_t)x & 15) == 0 && ((uintptr_t)w & 15) == 0) {
    const int64_t blocks = (n + WIDE_BM - 1) / WIDE_BM;
    // unguarded blocks address their 128 rows with 32-bit byte offsets: 128 m 4 < 2^31
    const int64_t full = (m % WIDE_BN == 0 && (int64_t)m < (int64_t(1) << 22)) ? n / WIDE_BM : 0;
    if (full > 0) {
      hipLaunchKernelGGL(gemm_wide_kernel<false>, dim3((unsigned)full), dim3(256), 0, (hipStream_t)stream, n, m, x,
                         w, scale, out, (int64_t)0);
      FC_LAUNCH_CHECK();
    }
    if (blocks > full) {
      hipLaunchKernelGGL(gemm_wide_kernel<true>, dim3((unsigned)(blocks - full)), dim3(256), 0, (hipStream_t)stream,
                         n, m, x, w, scale, out, full);
      FC_LAUNCH_CHECK();
    }
    return FC_OK;
  }
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

extern "C" int fc_dense_fwd_pairsum(int64_t n, int32_t k, int32_t m, const float* x, const int32_t* rows_lo,
                                    const int32_t* rows_hi, const float* w, float scale, float* out, void* stream) {
  if (n < 0 || k < 1 || m < 1 || m > 64) return FC_ERR_BAD_DESC;
  if (n == 0) return FC_OK;
  if (!x || !w || !out) return FC_ERR_NULL;
  if ((rows_lo == nullptr) != (rows_hi == nullptr)) return FC_ERR_NULL;
  if (n > 0x7fffffff || (k & 31) || (m & 3) || ((uintptr_t)x & 15) || ((uintptr_t)w & 15)) return FC_ERR_SHAPE;
  GemmBatch gb{};
  gb.trans_b = 1;
  gb.pair_sum = 1;
  GemmRank& g = gb.r[0];
  g.A = x; g.a_row = (rows_lo ? 1 : 2) * (int64_t)k; g.a_comp = 0;
  g.a_lo = rows_lo; g.a_hi = rows_hi;
  g.B = w;
  g.D = out; g.d_row = m; g.d_comp = 0;
  g.comps = 1; g.M = (int32_t)n; g.K = k; g.N = m; g.scale = scale;
  return launch_gemm(gb, 1, (hipStream_t)stream);
}

extern "C" int fc_radial_mlp_fwd(int64_t n, int32_t n_in, const float* x, const float* w0, float s0,
                                 const float* w1, float s1, int32_t m, const float* w2, float s2, float* out,
                                 void* stream) {
  if (n < 0 || n_in < 1 || n_in > WIDE_K || m < 1) return FC_ERR_BAD_DESC;
  if (n == 0) return FC_OK;
  if (!x || !w0 || !w1 || !w2 || !out) return FC_ERR_NULL;
  if (((uintptr_t)w2 & 15) != 0) return FC_ERR_SHAPE;  // weight chunks load as float4
  const int64_t blocks = (n + WIDE_BM - 1) / WIDE_BM;
  if (blocks > 0x7fffffff) return FC_ERR_SHAPE;
  // one launch (the partial last row block is guarded inside it); unguarded blocks address their
  // 128 rows with 32-bit byte offsets: 128 m 4 < 2^31
  if (m % WIDE_BN == 0 && (int64_t)m < (int64_t(1) << 22))
    hipLaunchKernelGGL(radial_mlp_fwd_kernel<false>, dim3((unsigned)blocks), dim3(256), 0, (hipStream_t)stream, n,
                       (int)n_in, x, w0, s0, w1, s1, (int)m, w2, s2, out, (int64_t)0);
  else
    hipLaunchKernelGGL(radial_mlp_fwd_kernel<true>, dim3((unsigned)blocks), dim3(256), 0, (hipStream_t)stream, n,
                       (int)n_in, x, w0, s0, w1, s1, (int)m, w2, s2, out, (int64_t)0);
  FC_LAUNCH_CHECK();
  return FC_OK;
}

extern "C" int fc_radial_mlp_hidden_fwd(int64_t n, int32_t n_in, const float* x, const float* w0, float s0,
                                        const float* w1, float s1, float* h2, void* stream) {
  if (n < 0 || n_in < 1 || n_in > WIDE_K) return FC_ERR_BAD_DESC;
  if (n == 0) return FC_OK;
  if (!x || !w0 || !w1 || !h2) return FC_ERR_NULL;
  const int64_t blocks = (n + WIDE_BM - 1) / WIDE_BM;
  if (blocks > 0x7fffffff) return FC_ERR_SHAPE;
  hipLaunchKernelGGL((radial_mlp_fwd_kernel<true, true>), dim3((unsigned)blocks), dim3(256), 0, (hipStream_t)stream, n,
                     (int)n_in, x, w0, s0, w1, s1, 64, (const float*)nullptr, 1.0f, h2, (int64_t)0);
  FC_LAUNCH_CHECK();
  return FC_OK;
}

// persistent workgroups of the radial MLP backward: two per CU (their LDS), at most one per block
static int64_t mlp_bwd_grid(int64_t blocks) {
  const int64_t g = 2 * (int64_t)device_cu_count();
  return blocks < g ? blocks : g;
}

extern "C" int fc_radial_mlp_bwd(int64_t n, int32_t n_in, const float* x, const float* w0, float s0,
                                 const float* w1, float s1, const float* grad_h2, float* grad_x, void* stream) {
  if (n < 0 || n_in < 1 || n_in > WIDE_K) return FC_ERR_BAD_DESC;
  if (n == 0) return FC_OK;
  if (!x || !w0 || !w1 || !grad_h2 || !grad_x) return FC_ERR_NULL;
  const int64_t blocks = (n + WIDE_BM - 1) / WIDE_BM;
  if (blocks > 0x7fffffff) return FC_ERR_SHAPE;
  hipLaunchKernelGGL(radial_mlp_bwd_kernel<false>, dim3((unsigned)mlp_bwd_grid(blocks)), dim3(256), 0,
                     (hipStream_t)stream, n, (int)n_in, x, w0, s0, w1, s1, grad_h2, grad_x);
  FC_LAUNCH_CHECK();
  return FC_OK;
}

extern "C" int fc_radial_mlp_bwd_pairsum(int64_t n, int32_t n_in, const float* x, const float* w0, float s0,
                                         const float* w1, float s1, const float* grad_h2, float* grad_x,
                                         void* stream) {
  if (n < 0 || n_in < 1 || n_in > WIDE_K) return FC_ERR_BAD_DESC;
  if (n == 0) return FC_OK;
  if (!x || !w0 || !w1 || !grad_h2 || !grad_x) return FC_ERR_NULL;
  const int64_t blocks = (n + WIDE_BM - 1) / WIDE_BM;
  if (blocks > 0x7fffffff) return FC_ERR_SHAPE;
  hipLaunchKernelGGL(radial_mlp_bwd_kernel<true>, dim3((unsigned)mlp_bwd_grid(blocks)), dim3(256), 0,
                     (hipStream_t)stream, n, (int)n_in, x, w0, s0, w1, s1, grad_h2, grad_x);
  FC_LAUNCH_CHECK();
  return FC_OK;
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

namespace fc {

// ---- Elementwise products with the rescaled SiLU's derivatives (second-order backward of the
// dense layers): out1 = a f'(pre) + add, out2 = a b f''(pre), with f(x) = kSiluScale x sigmoid(x),
//   f'(x)  = kSiluScale s (1 + x (1 - s)),   f''(x) = kSiluScale s (1 - s) (2 + x (1 - 2 s)),
// s = sigmoid(x). One pass over the operands for both products (one sigmoid per element).
__device__ __forceinline__ void silu_mix_one(float a, float b, float p, float add, bool w1, bool w2, float* o1,
                                             float* o2) {
  const float s = sigmoidf_(p);
  if (w1) *o1 = fmaf(a, kSiluScale * s * (1.0f + p * (1.0f - s)), add);
  if (w2) *o2 = a * b * (kSiluScale * s * (1.0f - s) * (2.0f + p * (1.0f - 2.0f * s)));
}

__global__ void __launch_bounds__(256) silu_grad_mix_kernel(int64_t n, const float* __restrict__ a,
                                                            const float* __restrict__ b,
                                                            const float* __restrict__ pre,
                                                            const float* __restrict__ add, float* __restrict__ out1,
                                                            float* __restrict__ out2, bool vec) {
  const bool w1 = out1 != nullptr, w2 = out2 != nullptr;
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  const int64_t t0 = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (vec) {  // n % 4 == 0 and every pointer 16-byte aligned
    for (int64_t q = t0; q < n / 4; q += stride) {
      const float4 av = reinterpret_cast<const float4*>(a)[q];
      const float4 pv = reinterpret_cast<const float4*>(pre)[q];
      const float4 bv = w2 ? reinterpret_cast<const float4*>(b)[q] : make_float4(0.f, 0.f, 0.f, 0.f);
      const float4 dv = (w1 && add) ? reinterpret_cast<const float4*>(add)[q] : make_float4(0.f, 0.f, 0.f, 0.f);
      float4 r1, r2;
      silu_mix_one(av.x, bv.x, pv.x, dv.x, w1, w2, &r1.x, &r2.x);
      silu_mix_one(av.y, bv.y, pv.y, dv.y, w1, w2, &r1.y, &r2.y);
      silu_mix_one(av.z, bv.z, pv.z, dv.z, w1, w2, &r1.z, &r2.z);
      silu_mix_one(av.w, bv.w, pv.w, dv.w, w1, w2, &r1.w, &r2.w);
      if (w1) reinterpret_cast<float4*>(out1)[q] = r1;
      if (w2) reinterpret_cast<float4*>(out2)[q] = r2;
    }
    return;
  }
  for (int64_t i = t0; i < n; i += stride) {
    float r1, r2;
    silu_mix_one(a[i], w2 ? b[i] : 0.f, pre[i], (w1 && add) ? add[i] : 0.f, w1, w2, &r1, &r2);
    if (w1) out1[i] = r1;
    if (w2) out2[i] = r2;
  }
}

}  // namespace fc

extern "C" int fc_silu_grad_mix(int64_t n, const float* a, const float* b, const float* pre, const float* add,
                                float* out1, float* out2, void* stream) {
  using namespace fc;
  if (n < 0) return FC_ERR_BAD_DESC;
  if (n == 0 || (!out1 && !out2)) return FC_OK;
  if (!a || !pre || (out2 && !b)) return FC_ERR_NULL;
  auto al = [](const void* p) { return p == nullptr || ((uintptr_t)p & 15) == 0; };
  const bool vec = (n & 3) == 0 && al(a) && al(b) && al(pre) && al(add) && al(out1) && al(out2);
  const int64_t work = vec ? n / 4 : n;
  const int64_t cap = (int64_t)device_cu_count() * 8;
  const int64_t blocks = (work + 255) / 256 < cap ? (work + 255) / 256 : cap;
  hipLaunchKernelGGL(silu_grad_mix_kernel, dim3((unsigned)blocks), dim3(256), 0, (hipStream_t)stream, n, a, b, pre,
                     add, out1, out2, vec);
  FC_LAUNCH_CHECK();
  return FC_OK;
}

namespace fc {

// ---- Weight gradients (training): dW[o, j] = scale * sum_r A'[r, o] * B[r, j] over every row
// r = (node, component) of a rank, with A = grad_out (A' = A * act'(pre) for a dense layer
// with the fused SiLU) and B = the layer input; optionally db[o] = sum_r A'[r, o].
// The contraction runs over rows, so the MFMA operands are row slices: step s contracts
// rows 2s (lanes 0-31) and 2s+1 (lanes 32-63), lane % 32 indexing o in the A operand and j
// in the B operand. Both stage tiles therefore sit in LDS row-major exactly as loaded
// (32 rows per stage, float4 global loads, no transposition), and the rows of a rank block
// are read in place from the packed feature rows (no gather copy).
// The row range is split over workgroups for parallelism (rows_per_split each); with more
// than one split every workgroup writes its unscaled partial block to a workspace and a
// second kernel sums the partials in split order, so results do not depend on scheduling.
struct WgradProblem {
  const float* A;  // row r = (n, c): A + n*a_row + c*a_comp, O floats
  const float* P;  // pre-activation in A's layout (SiLU derivative prologue) or null
  const float* B;  // row r: B + n*b_row + c*b_comp, J floats
  float* D;        // (O, J) row-major
  float* Db;       // (O) bias gradient or null
  int64_t a_row, a_comp, b_row, b_comp;
  int64_t R, rows_per_split;
  int32_t comps, O, J;
  float scale;
  int32_t tiles_o, tiles_j, splits, wg_base;
  int64_t part_off, partb_off;  // workspace offsets (floats) of the partial blocks
};

// One block of partial sums to reduce: dst[k] = scale * sum_s src[s * stride + k], k < count.
struct WgradSection {
  const float* src;
  float* dst;
  int64_t count, stride, base;  // base: first element in the reduce grid (multiple of 256)
  int32_t splits;
  float scale;
};

struct WgradBatch {
  WgradProblem p[FC_MAX_RANKS];
  WgradSection sec[2 * FC_MAX_RANKS];
  int32_t n, total_wg, n_sec;
  int64_t total_elems;
  float* part;
};

__device__ __forceinline__ float silu_grad_(float p) {
  const float s = sigmoidf_(p);
  return kSiluScale * s * (1.0f + p * (1.0f - s));
}

// Four consecutive floats of row r starting at column col (zero outside the row range and
// past the last column), times act'(pre) when P is given.
__device__ __forceinline__ float4 wgrad_fetch4(const float* p, int col, int ncol, bool vec) {
  if (vec) return *reinterpret_cast<const float4*>(p);
  return make_float4(p[0], col + 1 < ncol ? p[1] : 0.f, col + 2 < ncol ? p[2] : 0.f, col + 3 < ncol ? p[3] : 0.f);
}

// Row indices fit in 32 bits (the entry points check), so the (node, component) split of a
// row is a 32-bit division.
__device__ __forceinline__ float4 wgrad_load4(const float* base, const float* pbase, int64_t row_stride,
                                              int64_t comp_stride, int comps, int r, int r_end, int col,
                                              int ncol, bool vec) {
  if (r >= r_end || col >= ncol) return make_float4(0.f, 0.f, 0.f, 0.f);
  const int n = r / comps, c = r - n * comps;
  const int64_t off = (int64_t)n * row_stride + (int64_t)c * comp_stride + col;
  float4 v = wgrad_fetch4(base + off, col, ncol, vec);
  if (pbase) {
    const float4 p = wgrad_fetch4(pbase + off, col, ncol, vec);
    v.x *= silu_grad_(p.x); v.y *= silu_grad_(p.y); v.z *= silu_grad_(p.z); v.w *= silu_grad_(p.w);
  }
  return v;
}

template <int TO, int TJ>
__global__ void __launch_bounds__(256) wgrad_kernel(WgradBatch wb) {
  constexpr int RK = 32;                                  // rows per stage
  constexpr int WO = TO / 2, WJ = TJ / 2;                 // per-wave tile (waves 2 x 2)
  constexpr int FO = WO / 32, FJ = WJ / 32;               // 32 x 32 MFMA blocks per wave
  constexpr int A_TPR = TO / 4, B_TPR = TJ / 4;           // threads per stage row (one float4 each)
  constexpr int AL = RK * A_TPR / 256, BL = RK * B_TPR / 256;  // float4 per thread and stage
  __shared__ __attribute__((aligned(16))) float As[RK * TO];
  __shared__ __attribute__((aligned(16))) float Bs[RK * TJ];
  const int b = blockIdx.x;
  if (b >= wb.total_wg) return;
  int pi = 0;
#pragma unroll
  for (int q = 1; q < FC_MAX_RANKS; ++q)
    if (q < wb.n && b >= wb.p[q].wg_base) pi = q;
  const WgradProblem& g = wb.p[pi];
  const int local = b - g.wg_base;
  const int tiles = g.tiles_o * g.tiles_j;
  const int split = local / tiles, tile = local - split * tiles;
  const int to = tile / g.tiles_j, tj = tile - to * g.tiles_j;
  const int o0 = to * TO, j0 = tj * TJ;
  const int r_begin = (int)(split * g.rows_per_split);
  const int r_end = (int)(r_begin + g.rows_per_split < g.R ? r_begin + g.rows_per_split : g.R);
  const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
  const int wo = wave >> 1, wj = wave & 1;
  const bool a_vec = ((g.O & 3) == 0) && ((g.a_row & 3) == 0) && ((g.a_comp & 3) == 0) &&
                     (((uintptr_t)g.A & 15) == 0) && (!g.P || (((uintptr_t)g.P & 15) == 0));
  const bool b_vec = ((g.J & 3) == 0) && ((g.b_row & 3) == 0) && ((g.b_comp & 3) == 0) &&
                     (((uintptr_t)g.B & 15) == 0);
  const bool do_bias = g.Db && tj == 0 && wj == 0;

  float4 ra[AL], rb[BL];
  auto load = [&](int r0) {
#pragma unroll
    for (int i = 0; i < AL; ++i)
      ra[i] = wgrad_load4(g.A, g.P, g.a_row, g.a_comp, g.comps, r0 + t / A_TPR + i * (256 / A_TPR), r_end,
                          o0 + (t % A_TPR) * 4, g.O, a_vec);
#pragma unroll
    for (int i = 0; i < BL; ++i)
      rb[i] = wgrad_load4(g.B, nullptr, g.b_row, g.b_comp, g.comps, r0 + t / B_TPR + i * (256 / B_TPR), r_end,
                          j0 + (t % B_TPR) * 4, g.J, b_vec);
  };
  auto store = [&]() {
#pragma unroll
    for (int i = 0; i < AL; ++i)
      *reinterpret_cast<float4*>(As + (t / A_TPR + i * (256 / A_TPR)) * TO + (t % A_TPR) * 4) = ra[i];
#pragma unroll
    for (int i = 0; i < BL; ++i)
      *reinterpret_cast<float4*>(Bs + (t / B_TPR + i * (256 / B_TPR)) * TJ + (t % B_TPR) * 4) = rb[i];
  };

  floatx16 acc[FO][FJ];
#pragma unroll
  for (int i = 0; i < FO; ++i)
#pragma unroll
    for (int j = 0; j < FJ; ++j)
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[i][j][v] = 0.f;
  float bsum[FO];
#pragma unroll
  for (int i = 0; i < FO; ++i) bsum[i] = 0.f;

  load(r_begin);
  for (int r0 = r_begin; r0 < r_end; r0 += RK) {
    __syncthreads();  // the previous stage's reads are done
    store();
    __syncthreads();
    if (r0 + RK < r_end) load(r0 + RK);  // next stage in flight during this stage's MFMAs
    const float* as = As + wo * WO + (lane & 31);
    const float* bs = Bs + wj * WJ + (lane & 31);
#pragma unroll
    for (int s = 0; s < RK / 2; ++s) {
      const int rr = 2 * s + (lane >> 5);
      float av[FO], bv[FJ];
#pragma unroll
      for (int i = 0; i < FO; ++i) av[i] = as[rr * TO + i * 32];
#pragma unroll
      for (int j = 0; j < FJ; ++j) bv[j] = bs[rr * TJ + j * 32];
#pragma unroll
      for (int i = 0; i < FO; ++i)
#pragma unroll
        for (int j = 0; j < FJ; ++j) acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(av[i], bv[j], acc[i][j], 0, 0, 0);
      if (do_bias) {
#pragma unroll
        for (int i = 0; i < FO; ++i) bsum[i] += av[i];
      }
    }
  }

  // ---- epilogue: D[o][j] with o = 8*(v/4) + 4*(lane/32) + v%4, j = lane%32 per 32x32 block
  const bool direct = g.splits == 1;
  float* dst = direct ? g.D : wb.part + g.part_off + (int64_t)split * g.O * g.J;
  const float sc = direct ? g.scale : 1.0f;
#pragma unroll
  for (int i = 0; i < FO; ++i)
#pragma unroll
    for (int v = 0; v < 16; ++v) {
      const int o = o0 + wo * WO + i * 32 + 8 * (v >> 2) + 4 * (lane >> 5) + (v & 3);
      if (o >= g.O) continue;
#pragma unroll
      for (int j = 0; j < FJ; ++j) {
        const int jj = j0 + wj * WJ + j * 32 + (lane & 31);
        if (jj < g.J) dst[(int64_t)o * g.J + jj] = acc[i][j][v] * sc;
      }
    }
  if (do_bias) {
    float* bdst = direct ? g.Db : wb.part + g.partb_off + (int64_t)split * g.O;
#pragma unroll
    for (int i = 0; i < FO; ++i) {
      const float tot = bsum[i] + __shfl_xor(bsum[i], 32, 64);  // rows of both lane halves
      const int o = o0 + wo * WO + i * 32 + lane;
      if (lane < 32 && o < g.O) bdst[o] = tot;
    }
  }
}

// D = scale * sum over splits of the partial blocks (and Db = sum of the partial bias sums).
// Every workgroup covers 256 consecutive elements of one section (a weight or bias block;
// section starts are padded to multiples of 256): 64 threads x 4 elements per split lane,
// four split lanes (splits q, q+4, q+8, ...) whose sums are combined in a fixed order, so
// each thread keeps four independent loads in flight and the result is deterministic.
__global__ void __launch_bounds__(256) wgrad_reduce_kernel(WgradBatch wb) {
  __shared__ float red[4][256];
  const int64_t e0 = (int64_t)blockIdx.x * 256;
  int si = 0;
  for (int q = 1; q < wb.n_sec; ++q)
    if (e0 >= wb.sec[q].base) si = q;
  const WgradSection& sc = wb.sec[si];
  const int t = threadIdx.x, c = t & 63, lane_split = t >> 6;
  const int64_t k = e0 - sc.base + 4 * c;  // first of this thread's four elements
  float acc[4] = {0.f, 0.f, 0.f, 0.f};
  for (int sp = lane_split; sp < sc.splits; sp += 4) {
    const float* src = sc.src + (int64_t)sp * sc.stride;
#pragma unroll
    for (int q = 0; q < 4; ++q)
      if (k + q < sc.count) acc[q] += src[k + q];
  }
#pragma unroll
  for (int q = 0; q < 4; ++q) red[lane_split][4 * c + q] = acc[q];
  __syncthreads();
  if (lane_split == 0) {
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int i = 4 * c + q;
      if (k + q < sc.count) sc.dst[k + q] = ((red[0][i] + red[1][i]) + (red[2][i] + red[3][i])) * sc.scale;
    }
  }
}

// Tile shape, splits and workspace layout; returns the workspace size in floats.
static int64_t plan_wgrad(WgradBatch& wb, int* TO, int* TJ) {
  int max_o = 0, max_j = 0;
  for (int q = 0; q < wb.n; ++q) {
    if (wb.p[q].O > max_o) max_o = wb.p[q].O;
    if (wb.p[q].J > max_j) max_j = wb.p[q].J;
  }
  *TO = max_o >= 128 ? 128 : 64;
  *TJ = max_j >= 128 ? 128 : 64;
  int64_t work = 0;
  for (int q = 0; q < wb.n; ++q) {
    WgradProblem& g = wb.p[q];
    g.tiles_o = (g.O + *TO - 1) / *TO;
    g.tiles_j = (g.J + *TJ - 1) / *TJ;
    work += (int64_t)g.tiles_o * g.tiles_j * g.R;
  }
  // about 1024 workgroups, at least 256 rows each (a partial block costs as much as
  // reading 128 rows of both operands)
  int64_t rps = (work + 1023) / 1024;
  if (rps < 256) rps = 256;
  rps = (rps + 31) / 32 * 32;
  int64_t wg = 0, ws = 0;
  for (int q = 0; q < wb.n; ++q) {
    WgradProblem& g = wb.p[q];
    g.rows_per_split = rps;
    g.splits = (int32_t)(g.R > 0 ? (g.R + rps - 1) / rps : 1);
    g.wg_base = (int32_t)wg;
    wg += (int64_t)g.splits * g.tiles_o * g.tiles_j;
    if (g.splits > 1) {
      g.part_off = ws;
      ws += (int64_t)g.splits * g.O * g.J;
      g.partb_off = ws;
      if (g.Db) ws += (int64_t)g.splits * g.O;
    }
  }
  wb.total_wg = (int32_t)wg;
  return ws;
}

// The reduce grid: one section per weight (and bias) block that was split.
static void wgrad_sections(WgradBatch& wb) {
  wb.n_sec = 0;
  int64_t base = 0;
  auto add = [&](const float* src, float* dst, int64_t count, int64_t stride, int32_t splits, float scale) {
    WgradSection& sc = wb.sec[wb.n_sec++];
    sc.src = src; sc.dst = dst; sc.count = count; sc.stride = stride; sc.splits = splits; sc.scale = scale;
    sc.base = base;
    base += (count + 255) / 256 * 256;
  };
  for (int q = 0; q < wb.n; ++q) {
    const WgradProblem& g = wb.p[q];
    if (g.splits == 1) continue;
    const int64_t nw = (int64_t)g.O * g.J;
    add(wb.part + g.part_off, g.D, nw, nw, g.splits, g.scale);
    if (g.Db) add(wb.part + g.partb_off, g.Db, g.O, g.O, g.splits, 1.0f);
  }
  wb.total_elems = base;
}

static int launch_wgrad(WgradBatch wb, float* workspace, int64_t workspace_floats, hipStream_t s) {
  int TO, TJ;
  const int64_t need = plan_wgrad(wb, &TO, &TJ);
  if (wb.total_wg == 0) return FC_OK;
  if (need > 0 && (!workspace || workspace_floats < need)) return FC_ERR_WORKSPACE;
  wb.part = workspace;
  wgrad_sections(wb);
  const dim3 grid((unsigned)wb.total_wg), block(256);
  if (TO == 128 && TJ == 128) hipLaunchKernelGGL((wgrad_kernel<128, 128>), grid, block, 0, s, wb);
  else if (TO == 128) hipLaunchKernelGGL((wgrad_kernel<128, 64>), grid, block, 0, s, wb);
  else if (TJ == 128) hipLaunchKernelGGL((wgrad_kernel<64, 128>), grid, block, 0, s, wb);
  else hipLaunchKernelGGL((wgrad_kernel<64, 64>), grid, block, 0, s, wb);
  FC_LAUNCH_CHECK();
  if (need > 0) {
    hipLaunchKernelGGL(wgrad_reduce_kernel, dim3((unsigned)((wb.total_elems + 255) / 256)), dim3(256), 0, s, wb);
    FC_LAUNCH_CHECK();
  }
  return FC_OK;
}

static void linear_wgrad_batch(const fc_linear_desc* d, int64_t n, const float* go, const float* x, float alpha,
                               float* const* gw, WgradBatch& wb) {
  const LinearLayout L = linear_layout(d);
  wb = WgradBatch{};
  for (int l = 0; l <= L.common; ++l) {
    if (!gw || !gw[l]) continue;
    WgradProblem& g = wb.p[wb.n++];
    g.A = go + L.out_off[l];
    g.a_row = L.out_dim;
    g.a_comp = d->out_features;
    g.B = x + L.in_off[l];
    g.b_row = L.in_dim;
    g.b_comp = (int64_t)d->in_features * d->in_paths[l];
    g.D = gw[l];
    g.comps = 2 * l + 1;
    g.R = n * g.comps;
    g.O = d->out_features;
    g.J = d->in_features * d->in_paths[l];
    g.scale = alpha * d->scale[l];
  }
}

static void dense_wgrad_batch(int64_t n, int32_t k, int32_t m, const float* go, const float* pre_act, int32_t act,
                              const float* x, float scale, float* gw, float* gb, WgradBatch& wb) {
  wb = WgradBatch{};
  wb.n = 1;
  WgradProblem& g = wb.p[0];
  g.A = go; g.a_row = m; g.a_comp = 0;
  g.P = act ? pre_act : nullptr;
  g.B = x; g.b_row = k; g.b_comp = 0;
  g.D = gw; g.Db = gb;
  g.comps = 1; g.R = n; g.O = m; g.J = k; g.scale = scale;
}

}  // namespace fc

extern "C" int64_t fc_linear_wgrad_workspace(const fc_linear_desc* d, int64_t n, float* const* grad_w) {
  const int st = check_linear(d);
  if (st != FC_OK) return -st;
  if (n < 0) return -FC_ERR_SHAPE;
  // only which entries are non-NULL matters here (NULL array: every rank)
  float* all[FC_MAX_RANKS];
  for (int l = 0; l < FC_MAX_RANKS; ++l) all[l] = reinterpret_cast<float*>(16);
  WgradBatch wb;
  linear_wgrad_batch(d, n, nullptr, nullptr, 1.f, grad_w ? grad_w : all, wb);
  int TO, TJ;
  return plan_wgrad(wb, &TO, &TJ);
}

extern "C" int fc_linear_wgrad(const fc_linear_desc* d, int64_t n, const float* go, const float* x, float alpha,
                               float* const* grad_w, float* workspace, int64_t workspace_floats, void* stream) {
  int st = check_linear(d);
  if (st != FC_OK) return st;
  if (n < 0) return FC_ERR_SHAPE;
  if (!grad_w) return FC_ERR_NULL;
  if (n * (2 * FC_MAX_RANKS - 1) > 0x7fffffff) return FC_ERR_SHAPE;
  const int common = d->in_l_max < d->out_l_max ? d->in_l_max : d->out_l_max;
  if (n == 0) {  // no rows: zero gradients (a fill kernel, so the call can be graph-captured)
    for (int l = 0; l <= common; ++l)
      if (grad_w[l]) {
        const int64_t sz = (int64_t)d->out_features * d->in_features * d->in_paths[l];
        st = fill_columns(1, sz, 0, sz, nullptr, grad_w[l], (hipStream_t)stream);
        if (st != FC_OK) return st;
      }
    return FC_OK;
  }
  if (!go || !x) return FC_ERR_NULL;
  WgradBatch wb;
  linear_wgrad_batch(d, n, go, x, alpha, grad_w, wb);
  if (wb.n == 0) return FC_OK;
  return launch_wgrad(wb, workspace, workspace_floats, (hipStream_t)stream);
}

extern "C" int64_t fc_dense_wgrad_workspace(int64_t n, int32_t k, int32_t m, int32_t with_bias) {
  if (n < 0 || k < 1 || m < 1) return -FC_ERR_BAD_DESC;
  WgradBatch wb;
  dense_wgrad_batch(n, k, m, nullptr, nullptr, 0, nullptr, 1.f, reinterpret_cast<float*>(16),
                    with_bias ? reinterpret_cast<float*>(16) : nullptr, wb);
  int TO, TJ;
  return plan_wgrad(wb, &TO, &TJ);
}

extern "C" int fc_dense_wgrad(int64_t n, int32_t k, int32_t m, const float* go, const float* pre_act, int32_t act,
                              const float* x, float scale, float* gw, float* gb, float* workspace,
                              int64_t workspace_floats, void* stream) {
  if (n < 0 || k < 1 || m < 1 || act < 0 || act > 1) return FC_ERR_BAD_DESC;
  if (!gw) return FC_ERR_NULL;
  if (n == 0) {  // no rows: zero gradients (a fill kernel, so the call can be graph-captured)
    const int st = fill_columns(1, (int64_t)k * m, 0, (int64_t)k * m, nullptr, gw, (hipStream_t)stream);
    if (st != FC_OK || !gb) return st;
    return fill_columns(1, m, 0, m, nullptr, gb, (hipStream_t)stream);
  }
  if (!go || !x || (act == 1 && !pre_act)) return FC_ERR_NULL;
  if (n > 0x7fffffff - 256) return FC_ERR_SHAPE;  // row indices are 32-bit in the kernel
  WgradBatch wb;
  dense_wgrad_batch(n, k, m, go, pre_act, act, x, scale, gw, gb, wb);
  return launch_wgrad(wb, workspace, workspace_floats, (hipStream_t)stream);
}
