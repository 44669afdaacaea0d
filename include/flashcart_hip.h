/*
 * flashcart_hip.h -- C ABI of the MI355X (gfx950) FlashCart hot path.
 *
 * Every entry point takes plain device pointers, sizes and a HIP stream
 * (hipStream_t passed as void*; NULL is the default stream). The library never
 * allocates, frees or retains caller memory: outputs and workspaces are owned by
 * the caller (in the Python layer, the PyTorch caching allocator). Kernels write
 * every output element unless stated otherwise. All calls are asynchronous on the
 * given stream and return an fc_status code; nothing throws across the ABI.
 *
 * Feature layout (the reference's layout contract): a tensor of maximal rank L
 * with F channels is a row of (L+1)^2 * F floats, rank blocks in increasing l,
 * each block (2l+1, F) component-major. Stored components follow
 * src/flashcart/o3/_codegen_common.py:37-73 of the reference.
 */
#ifndef FLASHCART_HIP_H
#define FLASHCART_HIP_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Rank slots of the descriptors (ranks 0..4). A library compiled for ranks <= 3 (the default,
 * as the reference's FLASHCART_KERNEL_L_MAX) rejects rank 4 with FC_ERR_UNSUPPORTED_L; callers
 * fill the slots above their ranks with zeros / NULL. */
#define FC_MAX_RANKS 5

typedef enum fc_status {
  FC_OK = 0,
  FC_ERR_BAD_DESC = 1,       /* inconsistent descriptor (feature counts, flags) */
  FC_ERR_UNSUPPORTED_L = 2,  /* a rank above fc_kernel_l_max() (3; 4 for a FLASHCART_KERNEL_L_MAX=4 build) */
  FC_ERR_LAUNCH = 3,         /* hipGetLastError() reported a launch failure */
  FC_ERR_SHAPE = 4,          /* sizes the kernels do not support (e.g. > 1024 channels) */
  FC_ERR_NULL = 5,           /* a required pointer is NULL */
  FC_ERR_WORKSPACE = 6,      /* workspace missing or too small */
  FC_ERR_SCRATCH_LIMIT = 7   /* input larger than an allocation-free entry point's fixed scratch */
} fc_status;

/* Library version (major*10000 + minor*100 + patch) and the maximal supported rank. */
int fc_version(void);
int fc_kernel_l_max(void);
/* Human-readable message for a status code (static storage). */
const char* fc_status_string(int status);

/* ------------------------------------------------------------------------- */
/* Eq. (1) expansion of unit vectors: replaces torch.ops.flashcart.irreps_fwd  */
/* and irreps_bwd (reference src/flashcart/o3/_irreps.py:84-104, :117-150;    */
/* generated kernels src/flashcart/o3/_codegen_irreps.py:426-505).             */
/* x: (n, 3) unit vectors; out: (n, (l_max+1)^2); grad_x: (n, 3).             */
/* ------------------------------------------------------------------------- */
int fc_irreps_fwd(int64_t n, int32_t l_max, const float* x, float* out, void* stream);
int fc_irreps_bwd(int64_t n, int32_t l_max, const float* grad_out, const float* x, float* grad_x,
                  void* stream);
/* Backward of fc_irreps_bwd along a cotangent v (n, 3) of grad_x: replaces
 * torch.ops.flashcart.irreps_dbwd (reference src/flashcart/o3/_irreps.py:146-199; kernel
 * _codegen_irreps.py irreps_dbwd). d_grad_out (n, (l_max+1)^2) = J(x) v, d_x (n, 3) =
 * sum_a grad_out_a H_a(x) v; either output may be NULL. */
int fc_irreps_dbwd(int64_t n, int32_t l_max, const float* grad_out, const float* x, const float* v,
                   float* d_grad_out, float* d_x, void* stream);

/* ------------------------------------------------------------------------- */
/* Radial basis and cutoff envelope: replaces ChebyshevBasis.forward,          */
/* BesselBasis.forward and PolynomialCutoff.calculate_envelope (reference      */
/* src/flashcart/nn/radial.py:44-54, :98-121, :181-242) and their autograd.     */
/* ------------------------------------------------------------------------- */
typedef enum fc_basis_kind {
  FC_BASIS_CHEBYSHEV_AFFINE = 0,
  FC_BASIS_CHEBYSHEV_COSINE = 1,
  FC_BASIS_BESSEL = 2,
  FC_BASIS_NONE = 3 /* no radial basis (envelope / expansion only) */
} fc_basis_kind;

typedef struct fc_radial_desc {
  int32_t basis;      /* fc_basis_kind */
  int32_t n_radial;   /* basis functions (1..32) */
  float r_min;        /* Chebyshev mapping interval [r_min, r_max] */
  float r_max;        /* basis / cutoff radius */
  int32_t poly_order; /* cutoff polynomial order p >= 2; 0 disables the envelope */
} fc_radial_desc;

/* d: (n,) -> feats (n, n_radial) (may be NULL), env (n,) (may be NULL). */
int fc_radial_fwd(const fc_radial_desc* desc, int64_t n, const float* d, float* feats, float* env,
                  void* stream);
/* grad_d (n,) = sum_k g_feats[:,k] dfeat_k/dd + g_env denv/dd (either gradient may be NULL). */
int fc_radial_bwd(const fc_radial_desc* desc, int64_t n, const float* d, const float* g_feats,
                  const float* g_env, float* grad_d, void* stream);

/* ------------------------------------------------------------------------- */
/* Fused edge geometry: edge vectors (reference src/flashcart/utils/geometry.py */
/* :25-53), lengths and directions with the 1e-4 clamp (src/flashcart/model/    */
/* flashcart.py:22,280-281), the Eq. (1) expansion of the directions, the       */
/* radial basis and the cutoff envelope (src/flashcart/model/flashcart.py       */
/* :280-284) in one pass over the edges.                                       */
/*   positions mode: vec = pos[idx_j] - pos[idx_i] + shift_vec[e]              */
/*   vectors mode (pos == NULL): vec = vectors[e] (LAMMPS ML-IAP rij)           */
/* ------------------------------------------------------------------------- */
typedef struct fc_edge_desc {
  int32_t l_max;             /* expansion rank (0..3) */
  fc_radial_desc radial;     /* basis and cutoff */
} fc_edge_desc;

/* Periodic translation of every edge (reference src/flashcart/utils/geometry.py:52,
 * shifts @ cell[batch[idx_i]]): out[e, k] = (S0 cell[b][0][k] + S1 cell[b][1][k]) + S2 cell[b][2][k],
 * b = 0 for one cell, else batch[idx_i[e]]; each product and sum rounded on its own, so the
 * translation of -S is exactly the negation of that of S. shifts (n_edges, 3) int64, cell
 * (n_cells, 3, 3) row-major, out (n_edges, 3). idx_i (n_edges) and batch (n_nodes) are read only
 * when n_cells > 1; an index out of range gives a NaN row. */
int fc_shift_vectors(int64_t n_edges, int32_t n_cells, const int64_t* shifts, const float* cell,
                     const int32_t* idx_i, const int32_t* batch, int64_t n_nodes, float* out, void* stream);

int fc_edge_geometry_fwd(const fc_edge_desc* desc, int64_t n_edges, const float* pos,
                         const float* shift_vec, const int32_t* idx_i, const int32_t* idx_j,
                         const float* vectors, float* attrs, float* feats, float* env,
                         void* stream);
/* grad_vec (n_edges, 3) = dL/dvec given dL/dattrs, dL/dfeats, dL/denv (each may be NULL). */
int fc_edge_geometry_bwd(const fc_edge_desc* desc, int64_t n_edges, const float* pos,
                         const float* shift_vec, const int32_t* idx_i, const int32_t* idx_j,
                         const float* vectors, const float* g_attrs, const float* g_feats,
                         const float* g_env, float* grad_vec, void* stream);
/* Second derivative (force-loss training; the reference differentiates its torch edge
 * geometry and irreps_dbwd, src/flashcart/o3/_irreps.py:146-199): for the cotangent cot_vec
 * (n_edges, 3) of grad_vec, d_vec = the derivative of grad_vec along cot_vec (Hessian-vector
 * product of g . geometry) and d_g_* = the derivative of the geometry along cot_vec (the
 * gradients with respect to g_attrs / g_feats / g_env). Any input gradient and any output
 * may be NULL. */
int fc_edge_geometry_dbwd(const fc_edge_desc* desc, int64_t n_edges, const float* pos,
                          const float* shift_vec, const int32_t* idx_i, const int32_t* idx_j,
                          const float* vectors, const float* g_attrs, const float* g_feats,
                          const float* g_env, const float* cot_vec, float* d_g_attrs, float* d_g_feats,
                          float* d_g_env, float* d_vec, void* stream);

/* ------------------------------------------------------------------------- */
/* Receiver-sorted graph, computed once per neighbour list.                   */
/* ------------------------------------------------------------------------- */
typedef struct fc_csr {
  int64_t n_nodes;             /* receiver rows (output rows of the convolution) */
  int64_t n_edges;
  const int32_t* idx_j;        /* sender of each edge */
  const int32_t* rowptr;       /* receiver CSR over edges sorted by receiver (n_nodes+1) */
  const int32_t* sender_perm;  /* edge ids ordered by sender (stable), n_edges */
  const int32_t* sender_ptr;   /* sender CSR into sender_perm (n_sender_rows+1) */
  int64_t n_sender_rows;       /* rows of in1 (senders may include ghost atoms) */
  const int32_t* pair_slot;    /* optional (NULL: edge e uses weight row e). Per-edge weights shared
                                  by the two edges of a pair (fc_edge_pairs): edge e reads weight row
                                  pair_slot[e] / 2; its weight gradient stays at row e. Must come
                                  from a complete pairing (fc_edge_pairs with counts[0] == 0 and
                                  counts[1] == n_edges / 2): an edge with a negative slot has no
                                  weight row and contributes nothing (weights read as zero, its
                                  density and h-gradient terms skipped). No counterpart
                                  in the reference, which forms the weights of every edge
                                  (nn/layers.py:357-364). */
  const int32_t* idx_i;        /* optional: receiver of each edge. With it, fc_tp_bwd computes the three
                                  gradients of a 64-channel interaction-layer convolution (at most 40
                                  unreduced output rows) in sender order (no per-edge messages); NULL
                                  keeps receiver order. No counterpart in the reference. */
} fc_csr;

/* Edge pairs of a full neighbour list (no counterpart in the reference): the reverse of
 * edge (i <- j, S) is the edge (j <- i, -S) of receiver j, found by bisection; each receiver's
 * edges must be sorted by strictly increasing (sender, shift) (fc_neighbor_list and
 * fc_neighbor_list_device emit them so), an edge out of that order counts as unpaired. shifts
 * (n_edges, 3) may be NULL (no periodic shifts). Writes pair_slot[e] = 2p for the lower edge of pair p and 2p + 1
 * for its reverse (-1: no unique mutual reverse), pair_edge[p] = the lower edge (pairs
 * numbered in its order, at most max_pairs written), pair_upper[p] = its reverse and
 * reverse[e] = the reverse of every edge (-1: none; each may be NULL), counts[0] = edges
 * without a reverse, counts[1] = pairs. With every edge paired, reverse[rowptr[n] ..
 * rowptr[n+1]) lists the edges whose sender is n: a sender order with sender_ptr = rowptr.
 * Index work only; workspace of fc_edge_pairs_workspace(n_edges) int32. */
int64_t fc_edge_pairs_workspace(int64_t n_edges);
int fc_edge_pairs(const fc_csr* graph, const int32_t* idx_i, const int32_t* shifts, int32_t* pair_slot,
                  int32_t* pair_edge, int32_t* pair_upper, int32_t* reverse, int64_t max_pairs,
                  int32_t* counts, int32_t* workspace, int64_t workspace_ints, void* stream);

/* Radial-MLP inputs of edge pairs (no counterpart in the reference, which forms
 * edge_feats * envelope for every edge, src/flashcart/nn/layers.py:350-356):
 *   x[p, k] = feats[pair_edge[p], k] * env[pair_edge[p]]                 (n_pairs, width)
 * and its backward for all n_edges edges: the lower edge of each pair (even pair_slot) gets
 *   g_feats[e, k] = gx[p, k] * env[e],  g_env[e] = sum_k gx[p, k] feats[e, k],
 * the other edge zeros. Either backward output may be NULL. */
int fc_pair_inputs_fwd(int64_t n_pairs, int32_t width, const int32_t* pair_edge, const float* feats,
                       const float* env, float* x, void* stream);
int fc_pair_inputs_bwd(int64_t n_edges, int32_t width, const int32_t* pair_slot, const float* feats,
                       const float* env, const float* gx, float* g_feats, float* g_env, void* stream);

/* First interaction layer as a species density. Replaces the radial output layer and the
 * 0 x L -> L convolution of the first InteractionLayer (reference src/flashcart/nn/layers.py
 * :351-369) when its sender features depend on the species alone: with h (n_pairs, 64) the last
 * hidden activation of the radial MLP per edge pair (graph->pair_slot required),
 * y (n_edges, (y_l_max+1)^2) the edge attributes and edge_species[e] the species of the sender,
 *   dens[i, (l, m), Z, k] = sum_{e -> i, species Z} h[pair(e), k] y[e, (l, m)],  l <= l_max,
 * rows of (l_max+1)^2 x n_species x 64 floats (n_species <= 8), receiver-segmented, no atomics.
 * The layer output is then fc_linear_fwd over dens (in_features 64, in_paths n_species). */
int fc_species_density_fwd(const fc_csr* graph, int32_t l_max, int32_t y_l_max, int32_t n_species,
                           const int32_t* edge_species, const float* h, const float* y, float* dens,
                           void* stream);
/* Its backward from g_dens = dL/d dens: g_h (n_edges, 64) per edge at row pair_slot[e] (the two
 * rows of a pair sum to the gradient of its h row) and g_y (n_edges, (y_l_max+1)^2) (zero above
 * l_max). */
int fc_species_density_bwd(const fc_csr* graph, int32_t l_max, int32_t y_l_max, int32_t n_species,
                           const int32_t* edge_species, const float* h, const float* y, const float* g_dens,
                           float* g_h, float* g_y, void* stream);
/* The matrices of that layer map, one launch for all ranks l < n_ranks (no counterpart in the
 * reference; they fold the first layer's linear_first, radial output layer and linear_second,
 * reference nn/layers.py:351-369, into one matrix per rank):
 *   x[Z, c] = s_first / *alpha_div * sum_j table[Z, j] w_first[c, j]
 *   maps[l][o, Z * n_hidden + k] = sum_c w_second[l][o, c] x[Z, c] w_radial[(l * c_mid + c) * n_hidden + k]
 * table (n_species, c_in) the species' sender features, w_first (c_mid, c_in), w_second[l] (c_out, c_mid),
 * w_radial (n_ranks * c_mid, n_hidden) the radial output layer's rows of paths (0, l, l), maps[l]
 * (c_out, n_species * n_hidden); alpha_div a device scalar (the layer's sqrt_avg_neighbors).
 * Limits: n_species <= 8, c_in and c_mid <= 1024, n_hidden <= 64, n_ranks <= FC_MAX_RANKS. */
int fc_species_maps(int32_t n_species, int32_t c_in, int32_t c_mid, int32_t c_out, int32_t n_hidden,
                    int32_t n_ranks, const float* table, const float* w_first, float s_first,
                    const float* alpha_div, const float* const* w_second, const float* w_radial,
                    float* const* maps, void* stream);

/* rowptr[n] = first edge with idx_sorted[e] >= n, for n in [0, n_nodes]. */
int fc_csr_from_sorted(int64_t n_edges, const int32_t* idx_sorted, int64_t n_nodes,
                       int32_t* rowptr, void* stream);

/* Position gradient from edge-vector gradients, as a segmented reduction
 * (replaces the autograd index_select -> index_add backward of get_edge_vectors):
 *   grad_pos[n] = sum_{e: idx_j[e]=n} grad_vec[e] - sum_{e: idx_i[e]=n} grad_vec[e]. */
int fc_edge_grad_to_nodes(const fc_csr* graph, const float* grad_vec, float* grad_pos,
                          void* stream);

/* ------------------------------------------------------------------------- */
/* Irreducible Cartesian tensor product: replaces torch.ops.flashcart.tp_fwd  */
/* and tp_bwd (reference src/flashcart/o3/_tensor_product.py:332-479,         */
/* :550-787; kernels src/flashcart/o3/_codegen_tensor_product.py:2062-2140,    */
/* :2274-2421, :2447-2603, :3245-3311).                                        */
/* ------------------------------------------------------------------------- */
typedef struct fc_tp_desc {
  int32_t in1_l_max, in2_l_max, out_l_max; /* each 0..3 */
  int32_t in1_features, in2_features;      /* equal, or one of them 1 (broadcast) */
  int32_t symmetric_product;               /* canonical pairs only (in1 == in2) */
  int32_t shared_weights;                  /* weights (n_paths*C,) instead of (items, n_paths*C) */
  int32_t reduce_paths;                    /* sum paths within each output rank */
  const float* alpha_div;                  /* optional device scalar s (NULL: 1): the output (and the
                                              gradient's transpose) is scaled by alpha / s, read on the
                                              device at launch, so a divisor held in a device buffer
                                              (the interaction layers' sqrt_avg_neighbors, reference
                                              nn/layers.py:368) needs no host copy */
} fc_tp_desc;

/* Path count (the weight layout) of a configuration, or a negative fc_status. */
int fc_tp_num_paths(const fc_tp_desc* desc);
/* Output width in floats per row, or a negative fc_status. */
int64_t fc_tp_out_dim(const fc_tp_desc* desc);

/* graph == NULL: independent rows (in1, in2, weights and out all have n_rows rows).
 * graph != NULL: convolution; in1 has graph->n_sender_rows rows, in2 and weights have
 * n_edges rows, out has graph->n_nodes rows (receiver-sorted segmented sum).
 * out = alpha / *desc->alpha_div * TP(...) (alpha * TP(...) when alpha_div is NULL). */
int fc_tp_fwd(const fc_tp_desc* desc, const fc_csr* graph, int64_t n_rows, const float* in1,
              const float* in2, const float* weights, float alpha, float* out, void* stream);

/* Floats of workspace fc_tp_bwd needs for the requested gradients. */
int64_t fc_tp_bwd_workspace(const fc_tp_desc* desc, const fc_csr* graph, int64_t n_rows,
                            int need_in1, int need_weights);

/* Vector-Jacobian product of fc_tp_fwd (with the same alpha). NULL gradient pointers
 * are not computed. In convolution mode the in1 gradient is gathered to the senders
 * through graph->sender_perm / sender_ptr (segmented sum, no atomics), or, with
 * graph->idx_i for a 64-channel interaction layer, summed per sender in one pass over
 * each sender's edges (then the workspace goes unused). */
int fc_tp_bwd(const fc_tp_desc* desc, const fc_csr* graph, int64_t n_rows, const float* grad_out,
              const float* in1, const float* in2, const float* weights, float alpha,
              float* grad_in1, float* grad_in2, float* grad_weights, float* workspace,
              int64_t workspace_floats, void* stream);

/* Input gradients of a node-wise product (graph == NULL mode of fc_tp_bwd) added to
 * gradients that other consumers of the operands already produced:
 *   grad_in1 = pad(res1) + dL/d in1,   grad_in2 = pad(res2) + dL/d in2
 * res1 / res2 hold the first res1_comps / res2_comps rank components of each row (row
 * width comps * C, the leading rank blocks of the operand's layout), zero above; NULL
 * adds nothing, and a residual may be the very gradient buffer it is added to. Needs
 * in1_features == in2_features and per-path outputs (reduce_paths == 0); NULL gradient
 * pointers are not computed. No counterpart in the reference, where autograd adds the
 * gradients of an operand used by several products; its caller is the fused backward
 * of the product block (inference with frozen parameters). */
int fc_tp_bwd_rows_acc(const fc_tp_desc* desc, int64_t n_rows, const float* grad_out, const float* in1,
                       const float* in2, const float* weights, float alpha, const float* res1,
                       int32_t res1_comps, const float* res2, int32_t res2_comps, float* grad_in1,
                       float* grad_in2, void* stream);

/* ------------------------------------------------------------------------- */
/* Equivariant linear map on MFMA: replaces torch.ops.flashcart.linear_fwd and  */
/* the input-gradient branch of linear_bwd (reference src/flashcart/o3/         */
/* _linear.py:64-110, :328-385, :457-538; kernels _codegen_linear.py:161-221).  */
/*   out_l[n, m, :] = alpha * scale_l * x_l[n, m, :] @ W_l^T   for l <= min(in,out) */
/* with x_l viewed as (n, 2l+1, in_features*in_paths[l]); output ranks above     */
/* min(in_l_max, out_l_max) are zero.                                          */
/* ------------------------------------------------------------------------- */
typedef struct fc_linear_desc {
  int32_t in_l_max, out_l_max;
  int32_t in_features, out_features;
  int32_t in_paths[FC_MAX_RANKS];     /* paths per input rank (1 for plain features) */
  const float* weight[FC_MAX_RANKS];  /* W_l, row-major (out_features, in_features*in_paths[l]) */
  float scale[FC_MAX_RANKS];          /* s_l */
} fc_linear_desc;

/* residual (may be NULL, may equal out / grad_x): a tensor of the output's layout added to
 * the result, e.g. a skip connection or a gradient accumulated by another consumer. */
int fc_linear_fwd(const fc_linear_desc* desc, int64_t n_rows, const float* x, float alpha,
                  const float* residual, float* out, void* stream);
int fc_linear_dgrad(const fc_linear_desc* desc, int64_t n_rows, const float* grad_out,
                    float alpha, const float* residual, float* grad_x, void* stream);

/* Plain dense map out = act(x @ W^T * scale + bias), x (n, k), W (m, k) row-major:
 * the radial and readout MLP layers (reference src/flashcart/nn/layers.py:84-145,
 * :12-39). act: 0 none, 1 rescaled SiLU (1.6765324703310907 * silu). pre_act (n, m)
 * receives the value before the activation when non-NULL. */
int fc_dense_fwd(int64_t n, int32_t k, int32_t m, const float* x, const float* w, float scale,
                 const float* bias, int32_t act, float* pre_act, float* out, void* stream);
/* out (n, m) = scale * (x_lo[p] + x_hi[p]) @ W^T, W (m, k), m <= 64, k a multiple of 32, x and W
 * 16-byte aligned: a dense layer applied to the sum of two rows without forming it. rows_lo and
 * rows_hi NULL: x is (n, 2k) and the halves are x[p, 0:k] and x[p, k:2k]; else x has rows of k
 * floats and the halves are rows rows_lo[p] and rows_hi[p]. No counterpart in the reference;
 * the radial output layer's input gradient over edge pairs (the two edges' weight gradients). */
int fc_dense_fwd_pairsum(int64_t n, int32_t k, int32_t m, const float* x, const int32_t* rows_lo,
                         const int32_t* rows_hi, const float* w, float scale, float* out, void* stream);
/* grad_x (n, k) = (grad_out * act'(pre_act)) @ W * scale. */
int fc_dense_dgrad(int64_t n, int32_t k, int32_t m, const float* grad_out, const float* pre_act,
                   const float* w, float scale, int32_t act, float* grad_x, void* stream);

/* The radial MLP of an interaction layer with two hidden layers of 64 (reference
 * InteractionLayer.radial_mlp, src/flashcart/nn/layers.py:258-267 and :357-363, i.e. three
 * fc_dense_fwd calls): out (n, m) = s2 silu(s1 silu(s0 x W0^T) W1^T) W2^T with x (n, n_in),
 * n_in <= 64, W0 (64, n_in), W1 (64, 64), W2 (m, 64) row-major (W2 16-byte aligned), silu the
 * rescaled SiLU. The hidden activations stay on chip; nothing but out is written. */
int fc_radial_mlp_fwd(int64_t n, int32_t n_in, const float* x, const float* w0, float s0, const float* w1,
                      float s1, int32_t m, const float* w2, float s2, float* out, void* stream);
/* Its hidden part alone: h2 (n, 64) = silu(s1 silu(s0 x W0^T) W1^T), the input of the output
 * layer (no counterpart in the reference; the first layer's species density reads it). */
int fc_radial_mlp_hidden_fwd(int64_t n, int32_t n_in, const float* x, const float* w0, float s0,
                             const float* w1, float s1, float* h2, void* stream);
/* Input gradient of its hidden part: grad_x (n, n_in) from grad_h2 = dL/dh2 (n, 64), the
 * hidden layers recomputed from x (replaces the two hidden fc_dense_dgrad calls). */
int fc_radial_mlp_bwd(int64_t n, int32_t n_in, const float* x, const float* w0, float s0, const float* w1,
                      float s1, const float* grad_h2, float* grad_x, void* stream);
/* The same with dL/dh2 given as two rows per input row (grad_h2 (2n, 64); row p takes rows 2p and
 * 2p + 1 summed): the rows of an edge pair's two edges, no counterpart in the reference. */
int fc_radial_mlp_bwd_pairsum(int64_t n, int32_t n_in, const float* x, const float* w0, float s0,
                              const float* w1, float s1, const float* grad_h2, float* grad_x, void* stream);

/* Weight gradients (training). Replaces the weight-gradient part of the reference's
 * linear_bwd and its linear_wgrad kernel (src/flashcart/o3/_linear.py:457-570), and the
 * autograd weight gradient of the torch dense layers (src/flashcart/nn/layers.py:84-145).
 * grad_w[l] (out_features, in_features*in_paths[l]) = alpha * scale_l *
 * sum over rows (node, component) of grad_out_l^T x_l, for every rank l <= min(in_l_max,
 * out_l_max) whose pointer is non-NULL. The row reduction is split over workgroups; the
 * partial sums need fc_linear_wgrad_workspace() floats of workspace (0: none; pass the
 * same grad_w array, whose non-NULL entries select the ranks, or NULL for all ranks) and
 * are added in a fixed order, so results are deterministic. */
int64_t fc_linear_wgrad_workspace(const fc_linear_desc* desc, int64_t n_rows, float* const* grad_w);
int fc_linear_wgrad(const fc_linear_desc* desc, int64_t n_rows, const float* grad_out, const float* x,
                    float alpha, float* const* grad_w, float* workspace, int64_t workspace_floats,
                    void* stream);
/* Float64 equivariant linear map: replaces the reference's linear_fwd / linear_bwd called with
 * float64 tensors (use_fp64 = True, float64 accumulation: src/flashcart/o3/_linear.py:328-343,
 * :382, :457-538, selected by dtype in src/flashcart/o3/utils.py:36-50). Same layout, residual
 * and zero-fill rules as the float32 entry points above, with float64 weights, scales and
 * data. fc_linear_wgrad_f64 splits the row reduction over workgroups when
 * fc_linear_wgrad_f64_workspace() > 0 doubles (partial sums added in a fixed order). */
typedef struct fc_linear_desc_f64 {
  int32_t in_l_max, out_l_max;
  int32_t in_features, out_features;
  int32_t in_paths[FC_MAX_RANKS];
  const double* weight[FC_MAX_RANKS];  /* W_l, row-major (out_features, in_features*in_paths[l]) */
  double scale[FC_MAX_RANKS];
} fc_linear_desc_f64;

int fc_linear_fwd_f64(const fc_linear_desc_f64* desc, int64_t n_rows, const double* x, double alpha,
                      const double* residual, double* out, void* stream);
int fc_linear_dgrad_f64(const fc_linear_desc_f64* desc, int64_t n_rows, const double* grad_out, double alpha,
                        const double* residual, double* grad_x, void* stream);
int64_t fc_linear_wgrad_f64_workspace(const fc_linear_desc_f64* desc, int64_t n_rows, double* const* grad_w);
int fc_linear_wgrad_f64(const fc_linear_desc_f64* desc, int64_t n_rows, const double* grad_out, const double* x,
                        double alpha, double* const* grad_w, double* workspace, int64_t workspace_doubles,
                        void* stream);

/* grad_w (m, k) = scale * g^T x and grad_b (m, may be NULL) = column sums of g, with
 * g = grad_out * act'(pre_act) (act 1) or grad_out (act 0). */
int64_t fc_dense_wgrad_workspace(int64_t n, int32_t k, int32_t m, int32_t with_bias);
int fc_dense_wgrad(int64_t n, int32_t k, int32_t m, const float* grad_out, const float* pre_act, int32_t act,
                   const float* x, float scale, float* grad_w, float* grad_b, float* workspace,
                   int64_t workspace_floats, void* stream);

/* Elementwise products with the derivatives of the rescaled SiLU f(x) = 1.6765 x sigmoid(x)
 * (RescaledSiLULayer, reference src/flashcart/nn/layers.py:12-45), for the second-order
 * backward of the dense layers that the reference leaves to PyTorch autograd over that layer:
 *   out1 = a * f'(pre) + add   (add may be NULL),   out2 = a * b * f''(pre),
 * each formed when its pointer is non-NULL; n elements of each operand. */
int fc_silu_grad_mix(int64_t n, const float* a, const float* b, const float* pre, const float* add,
                     float* out1, float* out2, void* stream);

/* ------------------------------------------------------------------------- */
/* Invariant RMS normalisation: replaces RMSLayerNorm.forward (reference        */
/* src/flashcart/nn/layers.py:494-528; no centering) and its autograd in one    */
/* pass each. x, out, grad_x: (n, (l_max+1)^2 * C) feature rows; weight:        */
/* (l_max+1, C) per-rank gains g_l; scale: (n,) receives (m + eps)^-1/2 in the  */
/* forward (may be NULL) and is read by the backward, where                     */
/* m = mean_c sum_l TP_sym(x_l, x_l)_0 / ((2l+1)(l_max+1)).                     */
/* ------------------------------------------------------------------------- */
int fc_rms_norm_fwd(int64_t n, int32_t l_max, int32_t C, const float* x, const float* weight, float eps,
                    float* out, float* scale, void* stream);
/* grad_x = d<grad_out, out>/dx for fixed weight (the gain gradient is not formed). */
int fc_rms_norm_bwd(int64_t n, int32_t l_max, int32_t C, const float* grad_out, const float* x,
                    const float* weight, const float* scale, float* grad_x, void* stream);
/* Second derivative (no counterpart in the reference, which differentiates its torch norm
 * with autograd): the gradients of <cot, grad_x> with respect to grad_out, x and the gain.
 * d_weight_part (n, l_max+1, C) receives each node's share of the gain gradient (sum it
 * over nodes). Any output may be NULL. */
int fc_rms_norm_dbwd(int64_t n, int32_t l_max, int32_t C, const float* grad_out, const float* x,
                     const float* weight, const float* scale, const float* cot, float* d_grad_out,
                     float* d_x, float* d_weight_part, void* stream);

/* ------------------------------------------------------------------------- */
/* Rank-wise gating: replaces the gate activation, index_select and product of  */
/* EquivariantGatedLayer.forward (reference src/flashcart/nn/layers.py:609-635). */
/* values, out, grad_values: (n, (l_max+1)^2 * C); pre, grad_pre: (n, l_max+1, C) */
/* gate logits. act: 0 identity (gate already activated), 1 rescaled sigmoid     */
/* (1.8462285453386054 * sigmoid). out[n,(l,a),c] = values * act(pre[n,l,c]).     */
/* ------------------------------------------------------------------------- */
int fc_gate_fwd(int64_t n, int32_t l_max, int32_t C, const float* values, const float* pre, int32_t act,
                float* out, void* stream);
/* grad_values = grad_out * act(pre); grad_pre = act'(pre) * sum_a grad_out * values (either may be NULL). */
int fc_gate_bwd(int64_t n, int32_t l_max, int32_t C, const float* grad_out, const float* values,
                const float* pre, int32_t act, float* grad_values, float* grad_pre, void* stream);
/* Second derivative (no counterpart in the reference, which differentiates its torch gate
 * with autograd): gradients of <cot_values, grad_values> + <cot_pre, grad_pre> with respect
 * to grad_out, values and pre. Cotangents and outputs may be NULL. */
int fc_gate_dbwd(int64_t n, int32_t l_max, int32_t C, const float* grad_out, const float* values,
                 const float* pre, int32_t act, const float* cot_values, const float* cot_pre,
                 float* d_grad_out, float* d_values, float* d_pre, void* stream);

/* ------------------------------------------------------------------------- */
/* Segment reductions: replace scatter_sum (reference src/flashcart/utils/     */
/* scatter.py:33-68) for sorted segments, e.g. per-graph energies              */
/* (src/flashcart/model/atomistic.py:288).                                     */
/*   dst[s, :] = sum_{k in [ptr[s], ptr[s+1])} src[perm ? perm[k] : k, :]      */
/* ------------------------------------------------------------------------- */
int fc_segment_sum(int64_t n_seg, int64_t width, const float* src, const int32_t* perm,
                   const int32_t* ptr, float* dst, void* stream);

/* ------------------------------------------------------------------------- */
/* Host neighbour list (cell list over periodic images): replaces            */
/* NeighborList.build / _matscipy_neighbors (reference src/flashcart/data/      */
/* neighbors.py:56-77, :120-143). Pairs (i, j, S) with                         */
/* |pos[j] - pos[i] + S.cell| < cutoff, self pairs with S = 0 removed, sorted   */
/* lexicographically by (i, j, Sx, Sy, Sz). pos (n,3) and cell (3x3, rows are  */
/* lattice vectors) in float64; pbc[3] flags. Returns the pair count and fills */
/* the outputs only when it fits in `capacity`; -1 singular cell, -2 bad args. */
/* Host memory only; no GPU is touched.                                        */
/* ------------------------------------------------------------------------- */
int64_t fc_neighbor_list(int64_t n, const double* pos, const double* cell, const int32_t* pbc,
                         double cutoff, int64_t capacity, int64_t* out_i, int64_t* out_j,
                         int32_t* out_shift);

/* The same list built on the GPU from device positions (also replaces NeighborList.build,
 * reference src/flashcart/data/neighbors.py:56-77,120-143): identical pairs in identical
 * order (float64 arithmetic of the host list, no fused multiply-adds). pos (n,3) float64
 * and the outputs are device memory; cell[9] and pbc[3] host memory. workspace: device
 * memory of fc_neighbor_list_device_workspace(n) bytes. Synchronises `stream` (the pair
 * count is read back). Returns the pair count (outputs written only when it fits in
 * `capacity`), or -fc_status: FC_ERR_BAD_DESC (singular cell, bad cutoff),
 * FC_ERR_SHAPE (more than 1024 pairs for one atom, or a shift component >= 512). */
int64_t fc_neighbor_list_device_workspace(int64_t n);
int64_t fc_neighbor_list_device(int64_t n, const double* pos, const double* cell, const int32_t* pbc,
                                double cutoff, int64_t capacity, int64_t* out_i, int64_t* out_j,
                                int32_t* out_shift, void* workspace, int64_t workspace_bytes,
                                void* stream);

/* Allocation-free variant of fc_neighbor_list_device. No counterpart in the reference: it is
 * for callers that cannot allocate device memory (tight MD / serving loops, harnesses that
 * forbid hipMalloc). The same pairs in the same order, with the working arrays in a fixed
 * 64 MiB array of device memory that the library holds on each device it runs on until the
 * process ends, instead of a caller workspace. Inputs and outputs as fc_neighbor_list_device;
 * allocates and frees nothing. n above fc_neighbor_list_device_noalloc_max_atoms() (about
 * 640k atoms) returns -FC_ERR_SCRATCH_LIMIT. Every call on a device shares that device's
 * array, so calls that overlap on one device (other streams, other host threads) race. */
int64_t fc_neighbor_list_device_noalloc_max_atoms(void);
int64_t fc_neighbor_list_device_noalloc(int64_t n, const double* pos, const double* cell, const int32_t* pbc,
                                        double cutoff, int64_t capacity, int64_t* out_i, int64_t* out_j,
                                        int32_t* out_shift, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* FLASHCART_HIP_H */
