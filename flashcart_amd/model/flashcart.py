"""The FlashCart potential (reference src/flashcart/model/flashcart.py).

Constructor arguments, module tree, parameter names and initialisation order follow
the reference (``model/flashcart.py:92-221``), so reference checkpoints
(``model.pt`` + ``model_config.yaml``) load unchanged. The forward evaluates the
edge geometry (vectors, expansion, radial basis, envelope) in one fused HIP op and
shares one receiver-sorted graph (CSR + sender order) across all layers.
"""

from __future__ import annotations

from collections.abc import Mapping
from typing import Any, Dict, List, Literal, Optional

import torch
import torch.nn as nn

from flashcart_amd import _lib
from flashcart_amd import o3
from flashcart_amd.model.atomistic import AtomisticModel
from flashcart_amd.nn.layers import (
    EnergyReadoutLayer,
    EquivariantGatedLayer,
    InteractionLayer,
    ProductLayer,
    ScaleShiftEnergyLayer,
)
from flashcart_amd.nn import fused
from flashcart_amd.nn.radial import ChebyshevBasis, PolynomialCutoff
from flashcart_amd.o3 import _ops
from flashcart_amd.o3._graph import GraphCSR, build_graph
from flashcart_amd.utils.geometry import shift_vectors, uses_periodic_shifts
from flashcart_amd.utils.lammps import lammps_exchange_features

MIN_EDGE_LENGTH = 1.0e-4


class FlashCartPotential(AtomisticModel):
    """Equivariant potential predicting site energies (reference ``model/flashcart.py:25-317``)."""

    def __init__(self, elements: List[str], r_max: float, r_min: float = 0.0, n_hidden_feats: int = 32,
                 l_max_hidden_feats: int = 1, l_max_edge_attrs: int = 3, n_radial: int = 8, n_interactions: int = 2,
                 correlation: int = 3, path_reduced_product: bool = True, element_agnostic_interaction: bool = True,
                 element_agnostic_product: bool = True, n_element_interaction_features: int = 16,
                 nonlinearity: bool = False, gate_activation: str = "silu", gate_bias: bool = True,
                 layer_norm: bool = False, hidden_radial: Optional[List[int]] = None,
                 hidden_readout: Optional[List[int]] = None, radial_mapping: Literal["cosine", "affine"] = "affine",
                 cutoff_poly_order: int = 6, avg_neighbors: Optional[float] = None,
                 atomic_shifts: Optional[List[float]] = None, fit_atomic_shifts: bool = True,
                 recompute_radial: bool = False, use_triton: bool = False):
        super().__init__()
        self.elements = list(elements)
        self.r_min = r_min
        self.r_max = float(r_max)
        self.n_hidden_feats = n_hidden_feats
        self.l_max_hidden_feats = l_max_hidden_feats
        self.l_max_edge_attrs = l_max_edge_attrs
        self.n_radial = n_radial
        self.n_interactions = n_interactions
        self.correlation = correlation
        self.path_reduced_product = path_reduced_product
        self.hidden_radial = [64, 64] if hidden_radial is None else list(hidden_radial)
        self.hidden_readout = [64, 64] if hidden_readout is None else list(hidden_readout)
        self.radial_mapping = radial_mapping
        self.cutoff_poly_order = cutoff_poly_order
        self.atomic_shifts = None if atomic_shifts is None else list(atomic_shifts)
        self.fit_atomic_shifts = bool(fit_atomic_shifts)
        self.avg_neighbors = 1.0 if avg_neighbors is None else float(avg_neighbors)
        self.auto_avg_neighbors = avg_neighbors is None
        self.nonlinearity = nonlinearity
        self.gate_activation = gate_activation
        self.gate_bias = gate_bias
        self.layer_norm = layer_norm
        self.element_agnostic_interaction = element_agnostic_interaction
        self.element_agnostic_product = element_agnostic_product
        self.n_element_interaction_features = n_element_interaction_features
        self.recompute_radial = recompute_radial
        self.use_triton = use_triton
        self.node_dim = sum((2 * l + 1) * n_hidden_feats for l in range(l_max_hidden_feats + 1))

        self.embedding = nn.Embedding(len(elements), n_hidden_feats)
        self.radial_basis = ChebyshevBasis(n_radial, r_max=r_max, r_min=r_min, mapping=radial_mapping)
        self.cutoff_fn = PolynomialCutoff(r_max, poly_order=cutoff_poly_order)
        self.irreps = o3.Irreps(l_max_edge_attrs, use_triton=use_triton)
        product_out = [l_max_hidden_feats if k < n_interactions - 1 else 0 for k in range(n_interactions)]
        inter_in = [0 if k == 0 else l_max_hidden_feats for k in range(n_interactions)]
        self.use_products = correlation > 1
        inter_out = [l_max_edge_attrs] * n_interactions if self.use_products else product_out
        self.interactions = nn.ModuleList([
            InteractionLayer(in1_l_max=a, in2_l_max=l_max_edge_attrs, out_l_max=b, in1_features=n_hidden_feats,
                             out_features=n_hidden_feats, n_radial=n_radial, hidden_radial=self.hidden_radial,
                             n_elements=None if element_agnostic_interaction else len(elements),
                             element_features=n_element_interaction_features, avg_neighbors=self.avg_neighbors,
                             use_sc=True, use_layer_norm=layer_norm, use_triton=use_triton,
                             recompute_radial=recompute_radial)
            for a, b in zip(inter_in, inter_out)
        ])
        self.products = nn.ModuleList([
            ProductLayer(in_l_max=l_max_edge_attrs, out_l_max=p, in_features=n_hidden_feats,
                         n_elements=None if element_agnostic_product else len(elements), correlation=correlation,
                         path_reduced=path_reduced_product, use_sc=True, use_layer_norm=layer_norm,
                         use_triton=use_triton)
            for p in product_out
        ] if self.use_products else [])
        if self.nonlinearity:
            self.nonlinearities = nn.ModuleList([
                EquivariantGatedLayer(l_max=b, in_features=n_hidden_feats, hidden_features=n_hidden_feats,
                                      gate_activation=gate_activation, gate_bias=gate_bias, use_triton=use_triton)
                for b in inter_out
            ])
        self.readout = EnergyReadoutLayer(n_hidden_feats, n_interactions, hidden_readout=self.hidden_readout)
        self.scale_shift = ScaleShiftEnergyLayer(len(elements))

    def graph_csr(self, graph: Dict[str, Any]) -> GraphCSR:
        """Receiver CSR + sender order of the graph, cached on the source graph object."""
        src = graph.get("_source")
        csr = graph.get("csr") or (getattr(src, "csr", None) if src is not None else None)
        n_rows = graph["atom_types"].shape[0]
        if csr is None or csr.n_nodes != n_rows or csr.idx_i.device != graph["edge_index"].device:
            csr = build_graph(graph["edge_index"], n_rows)
            if src is not None:
                src.csr = csr
        return csr

    def wants_edge_pairs(self, positions: torch.Tensor) -> bool:
        """True when an interaction layer would form its radial weights once per edge pair
        (``fused.paired_conv_applies``); the edge list is then paired with its reverse edges."""
        return any(fused.paired_conv_applies(m, positions) for m in self.interactions)

    def edge_pair_shifts(self, graph: Dict[str, Any]):
        """(True, the shifts the edge list is paired by, or None) when ``forward`` would pair the
        edges of this graph dict, else (False, None)."""
        if graph.get("vectors") is not None or bool(graph.get("lammps_exchange", False)):
            return False, None
        if not self.wants_edge_pairs(graph["positions"]):
            return False, None
        use_shifts = graph.get("use_shifts", True)
        if not isinstance(use_shifts, bool):
            use_shifts = uses_periodic_shifts(use_shifts)
        return True, (graph["shifts"] if use_shifts else None)

    def forward(self, graph: Dict[str, Any]) -> torch.Tensor:
        if not isinstance(graph, Mapping):
            raise TypeError(f"{self.__class__.__name__}.forward expects a tensor dictionary. Use predict() for graphs.")
        edge_index = graph["edge_index"]
        batch = graph["batch"]
        atom_types = graph["atom_types"]
        is_lammps = bool(graph.get("lammps_exchange", False))
        if is_lammps:
            nlocal, ntotal = batch.shape[0], atom_types.shape[0]
            local_types = atom_types[:nlocal]
        else:
            nlocal = ntotal = None
            local_types = atom_types
        csr = self.graph_csr(graph)
        basis = self.radial_basis.basis_kind
        geo = (self.l_max_edge_attrs, basis, self.n_radial, float(self.r_min), self.r_max, self.cutoff_poly_order)
        vectors = graph.get("vectors")
        pairs = None
        if vectors is None:
            positions = graph["positions"]
            use_shifts = graph.get("use_shifts", True)
            if not isinstance(use_shifts, bool):
                use_shifts = uses_periodic_shifts(use_shifts)
            want_pairs = not is_lammps and self.wants_edge_pairs(positions)
            pair_shifts = graph["shifts"] if use_shifts else None
            # The pairing is launched first and its counters are read only after the edge geometry
            # and the embedding are queued. Until then the geometry takes the sender order a
            # complete pairing gives (the reverse edges, which its backward alone reads); an
            # incomplete pairing re-runs it with the sorted sender order.
            speculative = want_pairs and csr.request_edge_pairs(pair_shifts)
            sv = shift_vectors(graph["cell"], graph["shifts"], edge_index[0], batch,
                               antisymmetric=want_pairs) if use_shifts else None
            senders = speculative if speculative else (csr.sender_perm, csr.sender_ptr)
            edge_attrs, edge_feats, envelope = _ops.edge_geometry(
                positions, sv, csr.idx_i, csr.idx_j, None, csr.rowptr, *senders, *geo)
        else:
            edge_attrs, edge_feats, envelope = _ops.edge_geometry(
                None, None, csr.idx_i, csr.idx_j, vectors, csr.rowptr, csr.sender_perm, csr.sender_ptr, *geo)
        node_feats = self.embedding(atom_types)
        species = None
        if vectors is None and want_pairs and not self.embedding.weight.requires_grad and self.interactions and \
                fused.species_conv_applies(self.interactions[0], node_feats, self.embedding.weight.shape[0]):
            # the first layer's sender features are embedding rows: species density (fused.species_conv).
            # Its sender species and maps are queued before the pairing counters are read, so the GPU
            # has them at hand when that read returns
            first = self.interactions[0]
            species = (torch.index_select(atom_types.to(torch.int32), 0, csr.idx_j), self.embedding.weight,
                       fused.species_maps(first, self.embedding.weight, first.sqrt_avg_neighbors))
        if vectors is None and want_pairs:
            pairs = csr.edge_pairs(pair_shifts)
            if pairs is None and speculative:
                edge_attrs, edge_feats, envelope = _ops.edge_geometry(
                    positions, sv, csr.idx_i, csr.idx_j, None, csr.rowptr, csr.sender_perm, csr.sender_ptr, *geo)
        if pairs is None:
            species = None
        outputs = []
        shared = {}  # per-evaluation values the interaction layers share (their pair radial inputs)
        entry = None
        n_layers = len(self.interactions)
        for k, interaction in enumerate(self.interactions):
            msg = node_feats
            if is_lammps and k > 0:
                # owned features (nlocal, C) -> (ntotal, C) with ghost rows from their owners
                msg = lammps_exchange_features(node_feats, nlocal, ntotal)
            feats = interaction(msg, edge_attrs, edge_feats, edge_index, envelope,
                                atom_types=atom_types if not self.element_agnostic_interaction else None,
                                out_nodes=nlocal, graph=csr, edge_pairs=pairs, species=species if k == 0 else None,
                                shared=shared, entry=entry)
            entry = None
            if self.nonlinearity:
                feats = self.nonlinearities[k](feats)
            if self.use_products:
                node_feats = self.products[k](feats, None if self.element_agnostic_product else local_types)
            else:
                node_feats = feats
            nxt = self.interactions[k + 1] if k + 1 < n_layers else None
            if nxt is not None and pairs is not None and not is_lammps and \
                    fused.entry_maps_apply(nxt, node_feats, self.n_hidden_feats):
                # the next layer's input maps and this layer's readout columns with one input gradient
                h, r, readout = fused.entry_maps(nxt, node_feats, self.n_hidden_feats)
                entry = (h, r)
                outputs.append(readout)
            else:
                outputs.append(node_feats[:, : self.n_hidden_feats])
        return self.scale_shift(self.readout(outputs), local_types)

    def to_model_config(self) -> Dict[str, Any]:
        return {
            "elements": list(self.elements), "r_max": self.r_max, "r_min": self.r_min,
            "n_hidden_feats": self.n_hidden_feats, "l_max_hidden_feats": self.l_max_hidden_feats,
            "l_max_edge_attrs": self.l_max_edge_attrs, "n_radial": self.n_radial,
            "n_interactions": self.n_interactions, "correlation": self.correlation,
            "path_reduced_product": self.path_reduced_product,
            "element_agnostic_interaction": self.element_agnostic_interaction,
            "element_agnostic_product": self.element_agnostic_product,
            "n_element_interaction_features": self.n_element_interaction_features,
            "nonlinearity": self.nonlinearity, "gate_activation": self.gate_activation, "gate_bias": self.gate_bias,
            "layer_norm": self.layer_norm, "hidden_radial": list(self.hidden_radial),
            "hidden_readout": list(self.hidden_readout), "radial_mapping": self.radial_mapping,
            "cutoff_poly_order": self.cutoff_poly_order, "atomic_shifts": self.atomic_shifts,
            "fit_atomic_shifts": self.fit_atomic_shifts, "avg_neighbors": float(self.avg_neighbors),
            "use_triton": self.use_triton,
        }

    @classmethod
    def from_config(cls, cfg: Dict[str, Any]) -> "FlashCartPotential":
        return cls(
            elements=cfg["elements"], r_max=cfg["r_max"], r_min=cfg.get("r_min", 0.0),
            n_hidden_feats=cfg.get("n_hidden_feats", 32), l_max_hidden_feats=cfg.get("l_max_hidden_feats", 1),
            l_max_edge_attrs=cfg.get("l_max_edge_attrs", 3), n_radial=cfg.get("n_radial", 8),
            n_interactions=cfg.get("n_interactions", 2), correlation=cfg.get("correlation", 3),
            path_reduced_product=cfg.get("path_reduced_product", True),
            element_agnostic_interaction=cfg.get("element_agnostic_interaction", True),
            element_agnostic_product=cfg.get("element_agnostic_product", True),
            n_element_interaction_features=cfg.get("n_element_interaction_features", 16),
            nonlinearity=cfg.get("nonlinearity", False), gate_activation=cfg.get("gate_activation", "silu"),
            gate_bias=cfg.get("gate_bias", True), layer_norm=cfg.get("layer_norm", False),
            hidden_radial=cfg.get("hidden_radial", [64, 64]), hidden_readout=cfg.get("hidden_readout", [64, 64]),
            radial_mapping=cfg.get("radial_mapping", "affine"), cutoff_poly_order=cfg.get("cutoff_poly_order", 6),
            atomic_shifts=cfg.get("atomic_shifts"), fit_atomic_shifts=cfg.get("fit_atomic_shifts", True),
            avg_neighbors=cfg.get("avg_neighbors"), use_triton=cfg.get("use_triton", False),
            recompute_radial=cfg.get("recompute_radial", False),
        )
