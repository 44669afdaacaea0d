"""Model layers of the FlashCart potential (reference src/flashcart/nn/layers.py).

Each class keeps the reference's constructor, parameter/buffer names, shapes and
construction (initialisation) order, so reference checkpoints load unchanged and a
given seed draws the same initial weights. The heavy operations run on the HIP
library: the equivariant linear maps (MFMA), the tensor products, and the radial /
readout MLP layers with their fused rescaled-SiLU epilogue. Element-wise glue
(gates, norm scaling, residual sums) uses PyTorch tensor ops on the same device.
"""

from typing import Iterator, List, Optional, Tuple

import torch
import torch.nn as nn
import torch.nn.functional as F

from flashcart_amd import o3
from flashcart_amd.o3 import _ops
from flashcart_amd.o3._graph import EdgePairs, GraphCSR
from flashcart_amd.nn import fused

SILU_SCALE = 1.6765324703310907      # reference nn/layers.py:23
SIGMOID_SCALE = 1.8462285453386054   # reference nn/layers.py:59


class RescaledSiLULayer(nn.Module):
    """scale * silu(x), scale = 1/sqrt(E[silu(x)^2]) for x ~ N(0,1) (reference ``nn/layers.py:12-45``)."""

    def __init__(self, scale: Optional[float] = None):
        super().__init__()
        self.register_buffer("scale", torch.tensor(SILU_SCALE if scale is None else scale,
                                                   dtype=torch.get_default_dtype()), persistent=False)
        self._scale = float(SILU_SCALE if scale is None else scale)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        return self.scale * F.silu(x)


class RescaledSigmoidLayer(nn.Module):
    """scale * sigmoid(x) (reference ``nn/layers.py:48-81``)."""

    def __init__(self, scale: Optional[float] = None):
        super().__init__()
        self.register_buffer("scale", torch.tensor(SIGMOID_SCALE if scale is None else scale,
                                                   dtype=torch.get_default_dtype()), persistent=False)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        return self.scale * torch.sigmoid(x)


class LinearLayer(nn.Module):
    """F.linear(x, W * in_features^-1/2, bias) (reference ``nn/layers.py:84-145``), on the MFMA GEMM."""

    def __init__(self, in_features: int, out_features: int, bias: bool = False,
                 weight_scale: Optional[float] = None):
        super().__init__()
        self.in_features = in_features
        self.out_features = out_features
        scale = float(in_features) ** -0.5 if weight_scale is None else float(weight_scale)
        self._scale = scale
        self.register_buffer("scale", torch.tensor(scale, dtype=torch.get_default_dtype()), persistent=False)
        self.weight = nn.Parameter(torch.randn(out_features, in_features))
        if bias:
            self.bias = nn.Parameter(torch.zeros(out_features))
        else:
            self.register_parameter("bias", None)

    def forward(self, x: torch.Tensor, act: int = 0) -> torch.Tensor:
        """``act=1`` fuses the following RescaledSiLULayer into the GEMM epilogue."""
        out, _ = _ops.dense_fwd(x, _ops.param_alias(self.weight), _ops.param_alias(self.bias), self._scale, act)
        return out

    def __repr__(self) -> str:
        return (f"{self.__class__.__name__}(in_features={self.in_features}, out_features={self.out_features}, "
                f"bias={self.bias is not None}, scale={self._scale:.6g})")


def run_mlp(seq: nn.Sequential, x: torch.Tensor) -> torch.Tensor:
    """Evaluate a Sequential of LinearLayer / RescaledSiLULayer with fused activations."""
    mods = list(seq)
    i = 0
    while i < len(mods):
        m = mods[i]
        if isinstance(m, LinearLayer):
            fuse = i + 1 < len(mods) and isinstance(mods[i + 1], RescaledSiLULayer) and \
                mods[i + 1]._scale == SILU_SCALE
            x = m(x, act=1 if fuse else 0)
            i += 2 if fuse else 1
        else:
            x = m(x)
            i += 1
    return x


class _AddLeading(torch.autograd.Function):
    """out[:, :k] += r in place on a fresh GEMM output, k = r.shape[-1] (the rank-0 skip
    connection). Same values as ``cat([out[:, :k] + r, out[:, k:]])``; the backward passes the
    gradient through (for r its leading columns) instead of zero-filling, copying and adding
    two slice gradients."""

    @staticmethod
    def forward(ctx, out: torch.Tensor, r: torch.Tensor) -> torch.Tensor:
        ctx.k = r.shape[-1]
        out[:, : ctx.k].add_(r)
        ctx.mark_dirty(out)
        return out

    @staticmethod
    def backward(ctx, g: torch.Tensor):
        return g, g[:, : ctx.k]


class InteractionLayer(nn.Module):
    """Equivariant convolution with radial-MLP tensor-product weights (reference ``nn/layers.py:185-418``).

    Forward: linear_first -> radial MLP (on radial features times envelope) ->
    receiver-sorted TP convolution with the 1/sqrt(avg_neighbors) factor folded into
    the kernel output -> linear_second -> skip projection -> RMS norm.
    """

    def __init__(self, in1_l_max: int, in2_l_max: int, out_l_max: int, in1_features: int, out_features: int,
                 n_radial: int, hidden_radial: Optional[List[int]] = None, n_elements: Optional[int] = None,
                 element_features: Optional[int] = None, avg_neighbors: float = 1.0, use_sc: bool = False,
                 use_layer_norm: bool = False, use_triton: bool = False, recompute_radial: bool = False):
        super().__init__()
        self.in1_l_max = in1_l_max
        self.in2_l_max = in2_l_max
        self.out_l_max = out_l_max
        self.in1_features = in1_features
        self.out_features = out_features
        self.n_radial = n_radial
        self.hidden_radial = [64, 64] if hidden_radial is None else list(hidden_radial)
        self.use_sc = use_sc
        self.use_layer_norm = use_layer_norm
        self.recompute_radial = recompute_radial
        if avg_neighbors <= 0.0:
            raise ValueError(f"avg_neighbors must be positive. Provided: {avg_neighbors}.")
        self.register_buffer("sqrt_avg_neighbors",
                             torch.tensor(float(avg_neighbors) ** 0.5, dtype=torch.get_default_dtype()))
        self.out_dim = sum((2 * l + 1) * out_features for l in range(out_l_max + 1))
        out_paths, n_total_paths = o3.utils.count_output_paths(in1_l_max, in2_l_max, out_l_max)
        if n_elements is not None and element_features is None:
            raise ValueError("element_features must be provided when n_elements is set.")
        self.element_features = element_features
        radial_in = n_radial + 2 * self.element_features if n_elements is not None else n_radial
        layers = []
        for a, b in zip([radial_in] + self.hidden_radial, self.hidden_radial + [n_total_paths * in1_features]):
            layers.append(LinearLayer(a, b))
            layers.append(RescaledSiLULayer())
        self.radial_mlp = nn.Sequential(*layers[:-1])
        self.tp = o3.TensorProduct(in1_l_max=in1_l_max, in2_l_max=in2_l_max, out_l_max=out_l_max,
                                   in1_features=in1_features, in2_features=1, use_triton=use_triton,
                                   reduce_paths=False)
        self.linear_first = o3.LinearLayer(in1_l_max, in1_l_max, in1_features, in1_features, use_triton=use_triton)
        self.linear_second = o3.LinearLayer(out_l_max, out_l_max, in1_features, out_features, in_paths=out_paths,
                                            use_triton=use_triton)
        if self.use_sc:
            self.skip_projection = (LinearLayer(in1_features, out_features) if in1_l_max == 0 else
                                    o3.LinearLayer(in1_l_max, out_l_max, in1_features, out_features,
                                                   use_triton=use_triton))
        else:
            self.skip_projection = None
        self.layer_norm = (RMSLayerNorm(out_l_max, out_features, eps=1.0e-6, use_triton=use_triton)
                           if self.use_layer_norm else None)
        if n_elements is not None:
            self.emb_i = nn.Embedding(n_elements, self.element_features)
            self.emb_j = nn.Embedding(n_elements, self.element_features)
            nn.init.uniform_(self.emb_i.weight, a=-0.001, b=0.001)
            nn.init.uniform_(self.emb_j.weight, a=-0.001, b=0.001)
        else:
            self.emb_i = None
            self.emb_j = None

    def forward(self, node_feats: torch.Tensor, edge_attrs: torch.Tensor, edge_feats: torch.Tensor,
                edge_index: torch.Tensor, envelope: torch.Tensor, atom_types: Optional[torch.Tensor] = None,
                out_nodes: Optional[int] = None, graph: Optional[GraphCSR] = None,
                edge_pairs: Optional[EdgePairs] = None,
                species: Optional[Tuple[torch.Tensor, torch.Tensor]] = None,
                shared: Optional[dict] = None,
                entry: Optional[Tuple[torch.Tensor, torch.Tensor]] = None) -> torch.Tensor:
        """``edge_pairs`` (with ``graph``): the reverse-edge pairing of a full neighbour list whose
        edge lengths agree bitwise within each pair; the radial weights are then formed once per
        pair where ``fused.paired_conv_applies`` (same outputs, half the radial MLP work).
        ``shared``: a dict the caller passes to every interaction layer of one evaluation; the
        radial-MLP inputs per pair (the same for every layer without element embeddings) are
        formed by the first layer that needs them and reused by the others.
        ``entry = (linear_first(node_feats), skip_projection(node_feats))`` from
        ``fused.entry_maps``, used on the paired path instead of evaluating both maps here.
        ``species = (edge_species, table)`` or ``(edge_species, table, maps)``: ``node_feats`` is
        ``table[atom_types]`` and ``edge_species[e]`` the sender's row of ``table``; with pairs the
        layer then runs as a species density where ``fused.species_conv_applies`` (``maps``: its
        ``fused.species_maps``, formed by the caller)."""
        idx_i, idx_j = edge_index[0], edge_index[1]
        residual_feats = node_feats if out_nodes is None else node_feats[:out_nodes]
        if edge_pairs is not None and graph is not None and fused.paired_conv_applies(self, node_feats):
            key = ("pair_inputs", id(edge_feats), id(envelope), id(edge_pairs))
            mlp_pairs = shared.get(key) if shared is not None else None
            if mlp_pairs is None:
                mlp_pairs = _ops.pair_inputs(edge_feats, envelope, edge_pairs.edge, edge_pairs.slot)
                if shared is not None:
                    shared[key] = mlp_pairs
            if species is not None and out_nodes is None and \
                    fused.species_conv_applies(self, node_feats, species[1].shape[0]):
                mapped = fused.species_conv(self, edge_attrs, mlp_pairs, graph, edge_pairs, species[0],
                                            species[1], self.sqrt_avg_neighbors,
                                            species[2] if len(species) > 2 else None)
                return self._finish(mapped, residual_feats, out_nodes, mapped=True)
            else:
                in1 = entry[0] if entry is not None else self.linear_first(node_feats)
                aggregated = fused.paired_conv(self, in1, edge_attrs, mlp_pairs, graph, edge_pairs,
                                               self.sqrt_avg_neighbors)
            return self._finish(aggregated, residual_feats, out_nodes, skip=entry[1] if entry is not None else None)
        if self.emb_i is not None:
            if atom_types is None:
                raise ValueError(f"atom_types required when n_elements is set. Provided: {atom_types}.")
            emb_i, emb_j = self.emb_i(atom_types)[idx_i], self.emb_j(atom_types)[idx_j]
            mlp_input = torch.cat([edge_feats, emb_i, emb_j], dim=-1) * envelope.unsqueeze(-1)
        else:
            mlp_input = edge_feats * envelope.unsqueeze(-1)
        node_feats = self.linear_first(node_feats)
        if fused.radial_mlp_applies(self.radial_mlp, mlp_input):
            weights = fused.radial_mlp(self.radial_mlp, mlp_input)
        else:
            weights = run_mlp(self.radial_mlp, mlp_input)
        aggregated = self.tp(node_feats, edge_attrs, weights, idx_i, idx_j, graph=graph,
                             alpha_div=self.sqrt_avg_neighbors)
        return self._finish(aggregated, residual_feats, out_nodes)

    def _finish(self, aggregated: torch.Tensor, residual_feats: torch.Tensor,
                out_nodes: Optional[int], mapped: bool = False,
                skip: Optional[torch.Tensor] = None) -> torch.Tensor:
        """linear_second, skip connection and norm; ``mapped``: ``aggregated`` is already the
        output of linear_second (the species density folds it in); ``skip``: the skip projection
        of ``residual_feats``, already formed."""
        if out_nodes is not None:
            aggregated = aggregated[:out_nodes]
        if self.skip_projection is not None and self.in1_l_max > 0 and not mapped:
            # the skip projection enters linear_second's GEMM epilogue as its residual
            if skip is None:
                skip = self.skip_projection(residual_feats)
            out = self.linear_second(aggregated, residual=skip)
        elif mapped and self.skip_projection is not None and self.in1_l_max > 0:
            out = aggregated + self.skip_projection(residual_feats)
        else:
            out = aggregated if mapped else self.linear_second(aggregated)
            if self.skip_projection is not None:
                skip = self.skip_projection(residual_feats)
                out = _AddLeading.apply(out, skip) if torch.is_grad_enabled() else \
                    torch.cat([out[:, : self.out_features] + skip, out[:, self.out_features:]], dim=-1)
        if self.layer_norm is not None:
            out = self.layer_norm(out)
        return out

    def set_avg_neighbors(self, avg_neighbors: float) -> None:
        if avg_neighbors <= 0.0:
            raise ValueError(f"avg_neighbors must be positive. Provided: {avg_neighbors}.")
        self.sqrt_avg_neighbors.fill_(float(avg_neighbors) ** 0.5)


class RMSLayerNorm(nn.Module):
    """Invariant RMS normalisation of Cartesian features (reference ``nn/layers.py:420-535``).

    inv_l = symmetric TP(x_l, x_l) -> rank 0 (unit path weights); mean_sq averages
    inv_l / ((2l+1)(L+1)) over ranks and channels; out = x * (mean_sq + eps)^-1/2 * g_l.
    """

    def __init__(self, l_max: int, n_features: int, eps: float = 1.0e-12, affine: bool = True,
                 centering: bool = False, use_triton: bool = False):
        super().__init__()
        self.l_max = l_max
        self.n_features = n_features
        self.eps = eps
        self.affine = affine
        self.centering = centering
        self.slices = o3.utils.get_irreps_slices(l_max, n_features)
        self.shapes = o3.utils.get_irreps_shapes(l_max, n_features)
        self.block_dims = [s[0] * s[1] for s in self.shapes]
        self.dim = sum(self.block_dims)
        self.tp = o3.TensorProduct(in1_l_max=l_max, in2_l_max=l_max, out_l_max=0, in1_features=n_features,
                                   in2_features=n_features, use_triton=use_triton, symmetric_product=True,
                                   shared_weights=True, reduce_paths=False)
        _, n_paths = o3.utils.count_output_paths(l_max, l_max, 0, symmetric_product=True)
        assert n_paths == l_max + 1
        self.register_buffer("dummy_tp_weights", torch.ones(n_paths * n_features), persistent=False)
        self.register_buffer("l_weights", torch.tensor([1.0 / ((2 * l + 1) * (l_max + 1)) for l in range(l_max + 1)],
                                                       dtype=torch.float64), persistent=False)
        if affine:
            self.weights = nn.ParameterList([nn.Parameter(torch.ones(n_features)) for _ in range(l_max + 1)])
            self.register_buffer("l_expand_index", torch.arange(l_max + 1).repeat_interleave(
                torch.tensor([2 * l + 1 for l in range(l_max + 1)])), persistent=False)
            if centering:
                self.bias = nn.Parameter(torch.zeros(n_features))
            else:
                self.register_parameter("bias", None)
        else:
            self.weights = nn.ParameterList()
            self.register_parameter("bias", None)

    def forward(self, node_feats: torch.Tensor) -> torch.Tensor:
        if node_feats.shape[-1] != self.dim:
            raise RuntimeError(f"Incorrect last dimension for node_feats. Expected {self.dim}, "
                               f"got {node_feats.shape[-1]}.")
        n = node_feats.shape[0]
        if self.affine and not self.centering and self.n_features <= 256:
            # one fused kernel per direction (same formula as below)
            out, _ = _ops.rms_norm(node_feats, torch.stack(tuple(self.weights)), self.l_max, float(self.eps))
            return out
        feats = node_feats
        if self.centering:
            l0 = node_feats[:, : self.n_features]
            feats = torch.cat([l0 - l0.mean(dim=-1, keepdim=True), node_feats[:, self.n_features:]], dim=-1)
        inv = self.tp(feats, feats, self.dummy_tp_weights).view(n, self.l_max + 1, self.n_features)
        mean_sq = (inv * self.l_weights.to(inv.dtype).view(1, -1, 1)).sum(dim=1).mean(dim=-1, keepdim=True)
        scaled = feats * torch.pow(mean_sq + self.eps, -0.5)
        if not self.affine:
            return scaled
        w_full = torch.stack(tuple(self.weights)).index_select(0, self.l_expand_index).view(1, -1)
        out = scaled * w_full
        if self.bias is not None:
            out = torch.cat([out[:, : self.n_features] + self.bias, out[:, self.n_features:]], dim=-1)
        return out


class EquivariantGatedLayer(nn.Module):
    """Gated residual update, identity at initialisation (reference ``nn/layers.py:538-652``)."""

    def __init__(self, l_max: int, in_features: int, hidden_features: Optional[int] = None,
                 gate_activation: str = "silu", gate_bias: bool = True, use_triton: bool = False):
        super().__init__()
        if gate_activation not in ("silu", "sigmoid"):
            raise ValueError(f"gate_activation must be 'silu' or 'sigmoid'. Provided: {gate_activation!r}.")
        self.l_max = l_max
        self.in_features = in_features
        self.gate_activation_name = gate_activation
        self.gate_bias = gate_bias
        self.hidden_features = in_features if hidden_features is None else hidden_features
        if self.hidden_features <= 0:
            raise ValueError(f"hidden_features must be positive. Provided: {self.hidden_features}.")
        self.in_dim = sum((2 * l + 1) * in_features for l in range(l_max + 1))
        self.hidden_dim = sum((2 * l + 1) * self.hidden_features for l in range(l_max + 1))
        self.hidden_slices = o3.utils.get_irreps_slices(l_max, self.hidden_features)
        self.value_linear = o3.LinearLayer(l_max, l_max, in_features, self.hidden_features, use_triton=use_triton)
        self.gate_linear = LinearLayer(in_features, (l_max + 1) * self.hidden_features, bias=gate_bias)
        self.gate_activation = RescaledSiLULayer() if gate_activation == "silu" else RescaledSigmoidLayer()
        self.output_linear = o3.LinearLayer(l_max, l_max, self.hidden_features, in_features, use_triton=use_triton)
        for weight in self.output_linear.weight:
            nn.init.zeros_(weight)
        self.register_buffer("comp_rank", torch.arange(l_max + 1).repeat_interleave(
            torch.tensor([2 * l + 1 for l in range(l_max + 1)])), persistent=False)

    def forward(self, node_feats: torch.Tensor) -> torch.Tensor:
        if node_feats.shape[-1] != self.in_dim:
            raise RuntimeError(f"Incorrect last dimension for node_feats. Expected {self.in_dim}, "
                               f"got {node_feats.shape[-1]}.")
        if fused.applies(self, node_feats):
            # frozen parameters: one Function whose backward sums gradients inside kernels
            return fused.gated_block(self, node_feats)
        values = self.value_linear(node_feats)
        if self.gate_activation_name == "silu":  # activation fused into the gate GEMM
            pre, act = self.gate_linear(node_feats[:, : self.in_features], act=1), 0
        else:  # rescaled sigmoid applied inside the gating kernel
            pre, act = self.gate_linear(node_feats[:, : self.in_features]), 1
        gated = _ops.gate(values, pre, self.l_max, act)
        return self.output_linear(gated, residual=node_feats)


class IrrepsSelector(nn.Module):
    """Leading rank blocks up to out_l_max (reference ``nn/layers.py:655-700``)."""

    def __init__(self, in_l_max: int, out_l_max: int, in_features: int, in_paths: Optional[List[int]] = None):
        super().__init__()
        if out_l_max > in_l_max:
            raise ValueError("out_l_max must be less than or equal to in_l_max. "
                             f"Provided: out_l_max={out_l_max}, in_l_max={in_l_max}.")
        in_paths = [1] * (in_l_max + 1) if in_paths is None else list(in_paths)
        self.stop = o3.utils.get_irreps_slices(in_l_max, in_features, in_paths)[out_l_max][1]
        self.in_dim = sum((2 * l + 1) * in_features * in_paths[l] for l in range(in_l_max + 1))

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        if x.shape[-1] != self.in_dim:
            raise RuntimeError(f"Incorrect last dimension for x. Expected {self.in_dim}, got {x.shape[-1]}.")
        return x[:, : self.stop]


class ProductPathWeights(nn.Module):
    """Multiplicative path weights 1 + delta, delta zero-initialised (reference ``nn/layers.py:703-766``)."""

    def __init__(self, n_weights: int, n_elements: Optional[int] = None, learnable: bool = False):
        super().__init__()
        if n_elements is not None and not learnable:
            raise ValueError("Element-dependent path weights must be learnable. "
                             "Provided: learnable=False with n_elements set.")
        self.learnable = learnable
        self.element_dependent = False
        if not learnable:
            self.register_buffer("delta", torch.zeros(n_weights), persistent=False)
        elif n_elements is None:
            self.delta = nn.Parameter(torch.zeros(n_weights))
        else:
            self.element_dependent = True
            self.delta = nn.Embedding(n_elements, n_weights)
            nn.init.zeros_(self.delta.weight)

    def forward(self, atom_types: Optional[torch.Tensor] = None) -> torch.Tensor:
        if self.element_dependent:
            if atom_types is None:
                raise ValueError("atom_types required when n_elements is set.")
            return 1.0 + self.delta(atom_types)
        return 1.0 + self.delta


class ProductLayer(nn.Module):
    """Recurrent node-wise products B_k = TP(B_{k-1}, x) (reference ``nn/layers.py:769-1016``)."""

    def __init__(self, in_l_max: int, out_l_max: int, in_features: int, n_elements: Optional[int] = None,
                 correlation: int = 2, path_reduced: bool = False, use_sc: bool = False,
                 use_layer_norm: bool = False, use_triton: bool = False):
        super().__init__()
        if correlation < 2:
            raise ValueError("ProductLayer requires correlation >= 2. "
                             "Use FlashCartPotential(correlation=1) for an interaction-only model.")
        self.in_l_max = in_l_max
        self.out_l_max = out_l_max
        self.in_features = in_features
        self.correlation = correlation
        self.path_reduced = path_reduced
        self.learnable_path_weights = path_reduced or n_elements is not None
        self.use_sc = use_sc
        self.use_layer_norm = use_layer_norm
        self.in_dim = sum((2 * l + 1) * in_features for l in range(in_l_max + 1))
        self.out_dim = sum((2 * l + 1) * in_features for l in range(out_l_max + 1))
        self.skip_projection = (o3.LinearLayer(in_l_max, out_l_max, in_features, in_features, use_triton=use_triton)
                                if self.use_sc else None)
        self.layer_norm = (RMSLayerNorm(out_l_max, in_features, eps=1.0e-6, use_triton=use_triton)
                           if self.use_layer_norm else None)
        if self.path_reduced:
            self.final_linear = o3.LinearLayer(out_l_max, out_l_max, in_features, in_features, use_triton=use_triton)
        self.tensor_products = nn.ModuleList()
        self.path_weights = nn.ModuleList()
        self.irreps_selectors = nn.ModuleList()
        self.product_linears = nn.ModuleList()
        self.path_norm_names: List[Optional[str]] = []
        for k in range(self.correlation):
            p_out = out_l_max if k == self.correlation - 1 else in_l_max
            if k == 0:
                l1, l2, f2 = in_l_max, 0, 1
            else:
                l1, l2, f2 = in_l_max, in_l_max, in_features
            out_paths, n_total = o3.utils.count_output_paths(l1, l2, p_out, symmetric_product=False)
            self.path_weights.append(ProductPathWeights(n_total * in_features, n_elements=n_elements,
                                                        learnable=self.learnable_path_weights))
            if path_reduced:
                norm = torch.cat([torch.full(((2 * l + 1) * in_features,), out_paths[l] ** -0.5)
                                  for l in range(p_out + 1)])
                if torch.all(norm == 1.0):
                    self.path_norm_names.append(None)
                else:
                    name = f"path_norm_{k}"
                    self.register_buffer(name, norm)
                    self.path_norm_names.append(name)
            else:
                self.product_linears.append(o3.LinearLayer(p_out, p_out if k < self.correlation - 1 else out_l_max,
                                                           in_features, in_features, in_paths=out_paths,
                                                           use_triton=use_triton))
            self.irreps_selectors.append(nn.Identity() if p_out == out_l_max else
                                         IrrepsSelector(p_out, out_l_max, in_features))
            if k > 0:
                self.tensor_products.append(o3.TensorProduct(in1_l_max=l1, in2_l_max=l2, out_l_max=p_out,
                                                             in1_features=in_features, in2_features=f2,
                                                             use_triton=use_triton, reduce_paths=path_reduced,
                                                             symmetric_product=False,
                                                             shared_weights=n_elements is None))
        if self.learnable_path_weights:
            self.register_buffer("step0_weight_index", torch.cat([
                torch.arange(l * in_features, (l + 1) * in_features).repeat(2 * l + 1) for l in range(in_l_max + 1)
            ]), persistent=False)
        else:
            self.step0_weight_index = None

    def forward(self, node_feats: torch.Tensor, atom_types: Optional[torch.Tensor] = None) -> torch.Tensor:
        if fused.product_applies(self, node_feats, atom_types):
            # frozen parameters: one Function whose backward sums gradients inside kernels
            output = fused.product_block(self, node_feats)
            return self.layer_norm(output) if self.layer_norm is not None else output
        output = None
        product_feats = node_feats
        for k in range(self.correlation):
            if k == 0:
                if self.step0_weight_index is not None:
                    w = self.path_weights[0](atom_types)
                    product_feats = node_feats * w[..., self.step0_weight_index]
                else:
                    product_feats = node_feats
            else:
                w = self.path_weights[k](atom_types)
                product_feats = self.tensor_products[k - 1](product_feats, node_feats, w)
            if self.path_reduced:
                name = self.path_norm_names[k]
                if name is not None:
                    product_feats = product_feats * getattr(self, name)
            elif k == self.correlation - 1 and output is not None:
                # last step (output ranks only): the running sum enters the GEMM epilogue
                product_feats = self.product_linears[k](product_feats, residual=output)
                output = None
            else:
                product_feats = self.product_linears[k](product_feats)
            sel = self.irreps_selectors[k](product_feats)
            output = sel if output is None else output + sel
        if self.path_reduced:
            output = self.final_linear(output)
        if self.skip_projection is not None:
            output = self.skip_projection(node_feats, residual=output)
        if self.layer_norm is not None:
            output = self.layer_norm(output)
        return output


class EnergyReadoutLayer(nn.Module):
    """MLP on the concatenated scalar channels of every layer (reference ``nn/layers.py:1019-1078``)."""

    def __init__(self, in_features: int, n_layers: int, hidden_readout: Optional[List[int]] = None):
        super().__init__()
        self.in_features = in_features
        self.n_layers = n_layers
        self.hidden_readout = [64, 64] if hidden_readout is None else list(hidden_readout)
        layers = []
        for a, b in zip([in_features * n_layers] + self.hidden_readout, self.hidden_readout + [1]):
            layers.append(LinearLayer(a, b))
            layers.append(RescaledSiLULayer())
        self.readout_mlp = nn.Sequential(*layers[:-1])

    def forward(self, node_feats: List[torch.Tensor]) -> torch.Tensor:
        scalars = torch.cat([nf[:, : self.in_features] for nf in node_feats], dim=1)
        if scalars.shape[-1] != self.in_features * self.n_layers:
            raise RuntimeError("Incorrect last dimension for scalars. "
                               f"Expected: {self.in_features * self.n_layers}. Provided: {scalars.shape[-1]}.")
        return run_mlp(self.readout_mlp, scalars).squeeze(-1)


class ScaleShiftEnergyLayer(nn.Module):
    """Per-element energy scale; shifts stored for calculators (reference ``nn/layers.py:1081-1138``)."""

    def __init__(self, n_elements: int):
        super().__init__()
        self.n_elements = n_elements
        self.register_buffer("shifts", torch.zeros(n_elements))
        self.register_buffer("scales", torch.ones(n_elements))

    def forward(self, node_output: torch.Tensor, atom_types: torch.Tensor) -> torch.Tensor:
        return self.scales[atom_types] * node_output
