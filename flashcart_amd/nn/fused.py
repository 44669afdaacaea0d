"""Fused inference backward of the product and gating blocks.

With frozen parameters (energy + forces evaluation), the input gradient is all that the
backward of a block has to produce. Autograd over the per-module ops then spends a large
share of its time on glue: the block input feeds every product step, the skip projection
and the gate, so its gradient is summed by separate elementwise kernels, and the rank
selections (``x[:, :stop]``) come back as zero-padded copies. The Functions below run the
same forward ops and a backward written out by hand in which every such sum happens inside
a kernel: the linear input gradients take the running gradient as their GEMM-epilogue
residual, and the node-wise product backward adds into its operands' gradients
(``fc_tp_bwd_rows_acc``).

They are used only when the block input needs a gradient, no parameter of the block does,
no second derivative is wanted and no graph is being traced; otherwise the modules run op
by op with autograd (training, parameter gradients, create_graph, torch.compile). The
hand-written backward is first-order only (``once_differentiable``: differentiating it
again raises). Reference behaviour: ``nn/layers.py:538-652`` (gated update) and
``nn/layers.py:769-1016`` (product layer) — the outputs are those of the op-by-op path;
only the order of floating-point additions in the backward differs.
"""

import collections
import contextlib
import threading
from typing import List, Optional

import torch
from torch import Tensor
from torch.autograd.function import once_differentiable

from flashcart_amd.o3 import _ops

_state = threading.local()

# How often each fused path's forward ran (keys "paired", "species", "entry_maps", "product",
# "gated"), for tests and diagnostics that must know which path an evaluation took; clear()
# resets it. Under graph capture the count grows while capturing, not per replay.
path_counts: "collections.Counter[str]" = collections.Counter()


@contextlib.contextmanager
def disabled():
    """Run every block op by op inside the context (used when the backward will be
    differentiated again, e.g. ``predict(create_graph=True)``)."""
    prev = getattr(_state, "off", False)
    _state.off = True
    try:
        yield
    finally:
        _state.off = prev


def applies(module: torch.nn.Module, x: Tensor) -> bool:
    """True when ``module`` may run as one fused Function on input ``x``."""
    if getattr(_state, "off", False):
        return False
    if not (torch.is_grad_enabled() and x.requires_grad and x.is_cuda):
        return False
    if torch.compiler.is_compiling():
        return False
    return not any(p.requires_grad for p in module.parameters())


class _ProductBlock(torch.autograd.Function):
    """ProductLayer without path reduction and with shared path weights, up to and
    including the skip projection (the RMS norm stays a separate op).

    Forward, with t_0 = x and sel() the leading rank blocks up to out_l_max:
        p_k = L_k(t_k),  t_{k+1} = TP_k(p_k, x, w_{k+1}),  out = sum_{k<K-1} sel(p_k) + L_{K-1}(t_{K-1})
        out += Skip(x)
    Backward, given g = dL/d out:
        gx  = Skip^T g
        gt  = L_{K-1}^T g
        for k = K-1 .. 1:  (gp, gx) = TP_{k-1}^T gt + (sel^T g, gx)      one kernel
                           gt = L_{k-1}^T gp                               (k > 1)
        gx  = L_0^T gp + gx                                                residual epilogue
    """

    @staticmethod
    def forward(ctx, x: Tensor, layer) -> Tensor:
        path_counts["product"] += 1
        K = layer.correlation
        out: Optional[Tensor] = None
        p = x
        saved = []
        for k in range(K):
            if k == 0:
                t = x
            else:
                w = layer.path_weights[k](None)
                saved += [p, w]
                t = layer.tensor_products[k - 1](p, x, w)
            if k == K - 1 and out is not None:
                p = layer.product_linears[k](t, residual=out)
                out = None
            else:
                p = layer.product_linears[k](t)
            sel = layer.irreps_selectors[k](p)
            out = sel if out is None else out + sel
        if layer.skip_projection is not None:
            out = layer.skip_projection(x, residual=out)
        ctx.layer = layer
        ctx.save_for_backward(x, *saved)
        return out

    @staticmethod
    @once_differentiable
    def backward(ctx, g: Tensor):
        layer = ctx.layer
        x, *saved = ctx.saved_tensors
        g = g.contiguous()
        K = layer.correlation
        gx = layer.skip_projection.input_grad(g) if layer.skip_projection is not None else None
        gt = layer.product_linears[K - 1].input_grad(g)
        for k in range(K - 1, 0, -1):
            p, w = saved[2 * (k - 1)], saved[2 * (k - 1) + 1]
            tp = layer.tensor_products[k - 1]
            gp, gx = _ops.tp_bwd_rows_acc(gt, p, x, w, tp.in1_l_max, tp.in2_l_max, tp.out_l_max, tp.in1_features,
                                          tp.shared_weights, res1=g, res2=gx, inplace2=True)
            if k > 1:
                gt = layer.product_linears[k - 1].input_grad(gp)
            else:
                gx = layer.product_linears[0].input_grad(gp, residual=gx)
        return gx, None


def product_applies(layer, x: Tensor, atom_types: Optional[Tensor]) -> bool:
    return (not layer.path_reduced and layer.step0_weight_index is None and
            all(tp.shared_weights and tp.in1_features == tp.in2_features and not tp.symmetric_product
                for tp in layer.tensor_products) and applies(layer, x))


def product_block(layer, x: Tensor) -> Tensor:
    return _ProductBlock.apply(x, layer)


class _GatedBlock(torch.autograd.Function):
    """EquivariantGatedLayer: out = L_out(gate(L_val(x), act(L_gate(x_0)))) + x.

    Backward, given g: g_gated = L_out^T g; (g_val, g_pre) = gate^T; gx = L_val^T g_val + g
    (residual epilogue); gx_0 += L_gate^T g_pre (the scalar block only).
    """

    @staticmethod
    def forward(ctx, x: Tensor, layer) -> Tensor:
        path_counts["gated"] += 1
        values = layer.value_linear(x)
        gl = layer.gate_linear
        act_gemm = 1 if layer.gate_activation_name == "silu" else 0
        pre, pre_act = _ops.dense_fwd(x[:, : layer.in_features], gl.weight, gl.bias, gl._scale, act_gemm)
        act = 0 if act_gemm else 1
        gated = _ops.gate(values, pre, layer.l_max, act)
        out = layer.output_linear(gated, residual=x)
        ctx.layer = layer
        ctx.acts = (act, act_gemm)
        ctx.save_for_backward(values, pre, pre_act)
        return out

    @staticmethod
    @once_differentiable
    def backward(ctx, g: Tensor):
        layer = ctx.layer
        values, pre, pre_act = ctx.saved_tensors
        act, act_gemm = ctx.acts
        g = g.contiguous()
        g_gated = layer.output_linear.input_grad(g)
        g_values, g_pre = _ops.gate_bwd(g_gated, values, pre, layer.l_max, act, True, True)
        gx = layer.value_linear.input_grad(g_values, residual=g)
        gl = layer.gate_linear
        # add_ on the column view: `gx[:, :k] += y` would also copy the view onto itself (a second kernel)
        gx[:, : layer.in_features].add_(_ops.dense_bwd(g_pre, pre_act, gl.weight, gl._scale, act_gemm))
        return gx, None


def gated_block(layer, x: Tensor) -> Tensor:
    return _GatedBlock.apply(x, layer)


class _RadialMLP(torch.autograd.Function):
    """The interaction layer's radial MLP, Linear(n_in, 64) -> SiLU -> Linear(64, 64) -> SiLU
    -> Linear(64, m) (reference ``nn/layers.py:258-267``, applied at ``:357-363``), as one
    forward kernel whose hidden activations never leave the chip. Backward (input gradient
    only): dh2 = s2 g W2 (the wide dgrad GEMM), then one kernel that recomputes the hidden
    layers from x and applies both hidden-layer input gradients."""

    @staticmethod
    def forward(ctx, x: Tensor, mlp) -> Tensor:
        l0, l1, l2 = mlp[0], mlp[2], mlp[4]
        out = _ops.radial_mlp_fwd(x, l0.weight, l0._scale, l1.weight, l1._scale, l2.weight, l2._scale)
        ctx.save_for_backward(x)
        ctx.mlp = mlp
        return out

    @staticmethod
    @once_differentiable
    def backward(ctx, g: Tensor):
        (x,) = ctx.saved_tensors
        l0, l1, l2 = ctx.mlp[0], ctx.mlp[2], ctx.mlp[4]
        gh2 = _ops.dense_bwd(g, g.new_empty(0), l2.weight, l2._scale, 0)
        return _ops.radial_mlp_bwd(gh2, x, l0.weight, l0._scale, l1.weight, l1._scale), None


def radial_mlp_applies(mlp: torch.nn.Sequential, x: Tensor) -> bool:
    """True for the default radial MLP shape (two hidden layers of 64 with rescaled SiLU,
    no biases, at most 64 inputs) under the conditions of ``applies``."""
    from flashcart_amd.nn.layers import SILU_SCALE, LinearLayer, RescaledSiLULayer
    mods = list(mlp)
    if len(mods) != 5 or not all(isinstance(mods[i], LinearLayer) for i in (0, 2, 4)):
        return False
    if not all(isinstance(mods[i], RescaledSiLULayer) and mods[i]._scale == SILU_SCALE for i in (1, 3)):
        return False
    l0, l1, l2 = mods[0], mods[2], mods[4]
    if any(m.bias is not None for m in (l0, l1, l2)):
        return False
    if l0.weight.shape[0] != 64 or tuple(l1.weight.shape) != (64, 64) or l2.weight.shape[1] != 64:
        return False
    if not 1 <= l0.weight.shape[1] <= 64 or x.shape[-1] != l0.weight.shape[1]:
        return False
    return applies(mlp, x)


def radial_mlp(mlp: torch.nn.Sequential, x: Tensor) -> Tensor:
    return _RadialMLP.apply(x, mlp)


class _PairedConv(torch.autograd.Function):
    """Radial MLP + convolution tensor product of an interaction layer over edge pairs.

    The radial MLP input of an edge depends only on its length, which both edges of a pair
    (i <- j, S) / (j <- i, -S) share bitwise, so the weights are formed once per pair
    (``x``: the MLP inputs of the pairs' lower edges) and both edges read them
    (``tp_fwd(..., pair_slot)``): half the MLP work and half the weight stream written. The
    forward output equals the per-edge path's. Backward: the convolution's weight gradient
    comes out pair-major and the output layer's input gradient sums each pair inside its
    GEMM (``dense_bwd_pairs``); the hidden layers' backward then runs over the pairs.
    Reference: ``nn/layers.py:351-369`` (the MLP of every edge, then the convolution).
    """

    @staticmethod
    def forward(ctx, in1: Tensor, in2: Tensor, x: Tensor, layer, graph, pairs, alpha_div: Tensor) -> Tensor:
        path_counts["paired"] += 1
        slot = pairs.slot
        l0, l1, l2 = layer.radial_mlp[0], layer.radial_mlp[2], layer.radial_mlp[4]
        w = _ops.radial_mlp_fwd(x, l0.weight, l0._scale, l1.weight, l1._scale, l2.weight, l2._scale)
        tp = layer.tp
        out = _ops.tp_fwd(in1, in2, w, graph.idx_i, graph.idx_j, tp.in1_l_max, tp.in2_l_max, tp.out_l_max,
                          tp.in1_features, tp.in2_features, tp.symmetric_product, tp.shared_weights, *tp.op_meta,
                          tp.reduce_paths, graph.rowptr, graph.sender_perm, graph.sender_ptr, 1.0, slot, alpha_div)
        ctx.save_for_backward(in1, in2, x, w, slot, pairs.edge, pairs.upper, alpha_div)
        ctx.layer, ctx.graph = layer, graph
        return out

    @staticmethod
    @once_differentiable
    def backward(ctx, g: Tensor):
        in1, in2, x, w, slot, pairs_lo, pairs_hi, alpha_div = ctx.saved_tensors
        layer, graph = ctx.layer, ctx.graph
        n1, n2, nx = ctx.needs_input_grad[0], ctx.needs_input_grad[1], ctx.needs_input_grad[2]
        tp = layer.tp
        g1, g2, gw = _ops.tp_bwd(g.contiguous(), in1, in2, w, graph.idx_i, graph.idx_j, tp.in1_l_max, tp.in2_l_max,
                                 tp.out_l_max, tp.in1_features, tp.in2_features, tp.symmetric_product,
                                 tp.shared_weights, *tp.op_meta, tp.reduce_paths, bool(n1), bool(n2), bool(nx),
                                 graph.rowptr, graph.sender_perm, graph.sender_ptr, 1.0, slot, alpha_div)
        gx = None
        if nx:
            l0, l1, l2 = layer.radial_mlp[0], layer.radial_mlp[2], layer.radial_mlp[4]
            gh2 = _ops.dense_bwd_pairs(gw, l2.weight, l2._scale, pairs_lo, pairs_hi)
            del gw
            gx = _ops.radial_mlp_bwd(gh2, x, l0.weight, l0._scale, l1.weight, l1._scale)
        return (g1 if n1 else None), (g2 if n2 else None), gx, None, None, None, None


def paired_conv_applies(layer, node_feats: Tensor) -> bool:
    """True when an interaction layer may form its radial weights once per edge pair: the
    MLP input is the edge length alone (no element embeddings), the radial MLP has the fused
    kernel's shape, the convolution takes per-edge weights, no parameter of the MLP needs a
    gradient and no second derivative is wanted."""
    if getattr(_state, "off", False) or torch.compiler.is_compiling():
        return False
    if layer.emb_i is not None or layer.tp.shared_weights or not node_feats.is_cuda:
        return False
    mlp = layer.radial_mlp
    if any(p.requires_grad for p in mlp.parameters()):
        return False
    from flashcart_amd.nn.layers import SILU_SCALE, LinearLayer, RescaledSiLULayer
    mods = list(mlp)
    if len(mods) != 5 or not all(isinstance(mods[i], LinearLayer) for i in (0, 2, 4)):
        return False
    if not all(isinstance(mods[i], RescaledSiLULayer) and mods[i]._scale == SILU_SCALE for i in (1, 3)):
        return False
    l0, l1, l2 = mods[0], mods[2], mods[4]
    if any(m.bias is not None for m in (l0, l1, l2)):
        return False
    return (l0.weight.shape[0] == 64 and tuple(l1.weight.shape) == (64, 64) and l2.weight.shape[1] == 64
            and 1 <= l0.weight.shape[1] <= 64)


class _EntryMaps(torch.autograd.Function):
    """The two equivariant maps an interaction layer applies to its input rows (``linear_first``
    and the skip projection) and the leading ``n_read`` columns the energy readout takes from the
    same rows, as one Function: the skip projection's input gradient takes ``linear_first``'s as
    its GEMM-epilogue residual and the readout's gradient is added into its columns in place,
    instead of three full-width gradients summed by autograd (reference: the separate calls of
    ``nn/layers.py:351-379`` and ``model/flashcart.py:298-311``)."""

    @staticmethod
    def forward(ctx, x: Tensor, layer, n_read: int):
        path_counts["entry_maps"] += 1
        h = layer.linear_first(x)
        r = layer.skip_projection(x)
        s = x[:, :n_read].contiguous()
        ctx.layer, ctx.n_read = layer, n_read
        return h, r, s

    @staticmethod
    @once_differentiable
    def backward(ctx, gh: Tensor, gr: Tensor, gs: Tensor):
        layer = ctx.layer
        g = layer.linear_first.input_grad(gh.contiguous()) if gh is not None else None
        if gr is not None:
            g = layer.skip_projection.input_grad(gr.contiguous(), residual=g)
        if g is None and gs is not None:
            g = gs.new_zeros(gs.shape[0], layer.linear_first.in_dim)
        if g is not None and gs is not None:
            g[:, : ctx.n_read].add_(gs)
        return g, None, None


def entry_maps_apply(layer, x: Tensor, n_read: int) -> bool:
    """True when the interaction layer's input maps may run as ``entry_maps``: the paired
    convolution applies, the skip projection is an equivariant map feeding ``linear_second``'s
    epilogue, both maps are frozen, and the readout columns lie inside the rows."""
    from flashcart_amd.o3.linear import LinearLayer as O3Linear
    if not paired_conv_applies(layer, x) or not isinstance(layer.linear_first, O3Linear):
        return False
    sp = layer.skip_projection
    if sp is None or layer.in1_l_max == 0 or not isinstance(sp, O3Linear):
        return False
    if any(p.requires_grad for p in layer.linear_first.parameters()) or any(p.requires_grad for p in sp.parameters()):
        return False
    return x.dim() == 2 and 0 < n_read <= x.shape[1]


def entry_maps(layer, x: Tensor, n_read: int):
    """(linear_first(x), skip_projection(x), x[:, :n_read]) with one input gradient."""
    return _EntryMaps.apply(x, layer, n_read)


def paired_conv(layer, in1: Tensor, in2: Tensor, x_pairs: Tensor, graph, pairs, alpha_div: Tensor) -> Tensor:
    """``alpha_div``: the one-element device tensor the convolution output is divided by (the
    layer's ``sqrt_avg_neighbors``)."""
    return _PairedConv.apply(in1, in2, x_pairs, layer, graph, pairs, alpha_div)


def species_maps(layer, table: Tensor, alpha_div: Tensor):
    """Matrices and scales of the first interaction layer's species density, with its
    ``linear_second`` folded in: per rank l, with x_table = linear_first(table) / s (the sender
    features of each species, divided by the device scalar s = ``alpha_div``),
        M_l[o, Z * 64 + k] = sum_c Wsec_l[o, c] x_table[Z, c] W2[l C + c, k],
        scale_l = s2 s_l,
    so that linear_second(TP(...) / s)_l = scale_l dens_l @ M_l^T (the path (0, l, l) takes block l
    of the radial output layer W2). Formed on the device at every call (one launch of
    ``fc_species_maps``, no host synchronisation) from the parameters as they are at that moment, so
    weights written in place by any route (``param.data.copy_`` included, which no version counter
    records) are always seen; under graph capture the launch is recorded and replayed."""
    tp, lin, first = layer.tp, layer.linear_second, layer.linear_first
    lm = min(tp.in2_l_max, tp.out_l_max)
    common = min(lm, lin.out_l_max)
    n_sp = table.shape[0]
    mats = _ops.species_maps(table.detach(), first.weight[0].detach(), first._scale_list[0], alpha_div,
                             [lin.weight[l].detach() for l in range(common + 1)],
                             layer.radial_mlp[4].weight.detach())
    s2 = layer.radial_mlp[4]._scale
    cfg = (lm, lin.out_l_max, 64, lin.out_features, [n_sp] * (lm + 1),
           [s2 * lin._scale_list[l] for l in range(common + 1)])
    return mats, cfg


class _SpeciesConv(torch.autograd.Function):
    """Radial MLP + 0 x L -> L convolution + ``linear_second`` of the first interaction layer,
    whose sender features x_table[Z_j] depend on the sender's species alone, as a species
    density (``csrc/fc_species.hip``): the radial MLP up to its last hidden activation h (per edge
    pair), the receiver density dens[i, (l, m), Z, k] = sum_{e -> i, Z_j = Z} h_e[k] y_e[(l, m)],
    and one equivariant linear map per rank with the matrices of ``species_maps``. Same function
    as the per-edge path followed by ``linear_second``, with sums in another order; the
    E x paths x C weights and the convolution output are never formed. Reference
    ``nn/layers.py:351-369``.
    """

    @staticmethod
    def forward(ctx, y: Tensor, x_pairs: Tensor, layer, graph, pairs, edge_species: Tensor,
                table: Tensor, alpha_div: Tensor, maps=None) -> Tensor:
        path_counts["species"] += 1
        from flashcart_amd import _lib
        tp = layer.tp
        l0, l1 = layer.radial_mlp[0], layer.radial_mlp[2]
        n_sp = table.shape[0]
        lm = min(tp.in2_l_max, tp.out_l_max)
        h = _ops.radial_mlp_hidden_fwd(x_pairs, l0.weight, l0._scale, l1.weight, l1._scale)
        csr = _lib.csr_struct(graph.n_nodes, graph.n_edges, graph.idx_j, graph.rowptr, pair_slot=pairs.slot)
        dens = _ops.species_density_fwd(csr, lm, tp.in2_l_max, n_sp, edge_species, h, y, graph.n_nodes)
        mats, cfg = maps if maps is not None else species_maps(layer, table, alpha_div)
        out = _ops.linear_fwd(dens, mats, *cfg)
        ctx.save_for_backward(y, x_pairs, h, edge_species, pairs.slot, *mats)
        ctx.layer, ctx.graph, ctx.cfg, ctx.n_sp = layer, graph, cfg, n_sp
        return out

    @staticmethod
    @once_differentiable
    def backward(ctx, g: Tensor):
        from flashcart_amd import _lib
        y, x_pairs, h, edge_species, slot, *mats = ctx.saved_tensors
        layer, graph, cfg = ctx.layer, ctx.graph, ctx.cfg
        if not (ctx.needs_input_grad[0] or ctx.needs_input_grad[1]):
            return (None,) * 9
        g_dens = _ops.linear_bwd(g.contiguous(), mats, *cfg)
        csr = _lib.csr_struct(graph.n_nodes, graph.n_edges, graph.idx_j, graph.rowptr, pair_slot=slot)
        g_h, g_y = _ops.species_density_bwd(csr, cfg[0], layer.tp.in2_l_max, ctx.n_sp, edge_species, h, y, g_dens)
        del g_dens
        gx = None
        if ctx.needs_input_grad[1]:
            l0, l1 = layer.radial_mlp[0], layer.radial_mlp[2]
            # both edges of a pair read its h row: rows 2p and 2p + 1 of g_h summed in the kernel
            gx = _ops.radial_mlp_bwd_pairsum(g_h, x_pairs, l0.weight, l0._scale, l1.weight, l1._scale)
        return (g_y if ctx.needs_input_grad[0] else None), gx, None, None, None, None, None, None, None


MAX_DENSITY_SPECIES = 8


def species_conv_applies(layer, node_feats: Tensor, n_species: int) -> bool:
    """True when the first interaction layer may run as a species density: the conditions of
    ``paired_conv_applies``, rank-0 sender features of one channel block through a frozen
    ``linear_first``, single-channel edge attributes, unreduced paths, at most
    ``MAX_DENSITY_SPECIES`` species."""
    tp, lin = layer.tp, layer.linear_second
    if layer.in1_l_max != 0 or tp.in1_l_max != 0 or tp.in2_features != 1 or tp.reduce_paths or tp.symmetric_product:
        return False
    lm = min(tp.in2_l_max, tp.out_l_max)
    if lin.in_l_max != lm or lin.in_paths != [1] * (lm + 1) or lin.in_features != tp.in1_features:
        return False
    if not 1 <= n_species <= MAX_DENSITY_SPECIES:
        return False
    if any(p.requires_grad for p in layer.linear_first.parameters()) or any(p.requires_grad for p in lin.parameters()):
        return False
    return paired_conv_applies(layer, node_feats)


def species_conv(layer, edge_attrs: Tensor, x_pairs: Tensor, graph, pairs, edge_species: Tensor,
                 table: Tensor, alpha_div: Tensor, maps=None) -> Tensor:
    """``table``: the embedding rows of the species (the layer's sender features are
    linear_first(table)[species]); ``alpha_div``: the layer's ``sqrt_avg_neighbors``; ``maps``:
    ``species_maps(layer, table, alpha_div)`` when the caller formed them already."""
    return _SpeciesConv.apply(edge_attrs, x_pairs, layer, graph, pairs, edge_species, table, alpha_div, maps)
