"""Energy/force driver (reference src/flashcart/model/atomistic.py).

``predict`` sums site energies per structure with the HIP segment sum and obtains
forces (-dE/dR), stress/virials (symmetric virtual strain) and edge forces (dE/d rij)
with autograd, whose backward runs through the registered HIP ops.
"""

from __future__ import annotations

from pathlib import Path
from typing import Any, Dict, Optional, Union

import torch
import torch.nn as nn
import yaml

from flashcart_amd.o3 import _ops
from flashcart_amd.utils.geometry import to_voigt6, uses_periodic_shifts


def save_inference_metadata(ckpt_dir: Path, model_config: Dict[str, Any], meta: Optional[Dict[str, Any]] = None):
    ckpt_dir = Path(ckpt_dir)
    ckpt_dir.mkdir(parents=True, exist_ok=True)
    with open(ckpt_dir / "model_config.yaml", "w") as fh:
        yaml.safe_dump(model_config, fh)
    if meta is not None:
        with open(ckpt_dir / "meta.yaml", "w") as fh:
            yaml.safe_dump(meta, fh)


def load_model_config(ckpt_dir: Path) -> Dict[str, Any]:
    path = Path(ckpt_dir) / "model_config.yaml"
    if not path.exists():
        raise FileNotFoundError(f"No model_config.yaml in {ckpt_dir}.")
    with open(path) as fh:
        return yaml.safe_load(fh)


def _graph_dict(graph) -> Dict[str, Any]:
    if isinstance(graph, dict):
        return dict(graph)
    d = graph.to_dict()
    d["_source"] = graph
    return d


class _PredictReplay:
    """HIP graphs of ``_predict_impl`` for fixed input shapes.

    The graph's tensors are copied into private input buffers that the captured work
    reads. The receiver CSR of the edge list and its edge pairing are a graph of their own,
    replayed only when the edge list or the periodic shifts (which the pairing reads) are a
    different tensor or were modified in place since the last call (the previous tensors are
    kept referenced, so their identity is meaningful); an MD step with a fixed neighbour
    list copies the positions and replays the prediction only. Outputs are cloned out of the
    graph's buffers, which the next replay overwrites.
    """

    def __init__(self, model, gd, tensors, flags):
        self.inputs = {k: v.detach().clone() for k, v in tensors.items()}
        base = {k: v for k, v in gd.items() if k not in ("_source", "csr")}
        base.update(self.inputs)
        self.flags = flags
        self.topology = None
        self._src_edges = None
        self.pair_counts = None  # device counters of the edge pairing replayed with the topology
        self.paired = False
        side = torch.cuda.Stream()  # default priority
        side.wait_stream(torch.cuda.current_stream())
        if not gd.get("lammps_exchange", False):
            from flashcart_amd.o3._graph import build_graph, launch_edge_pairs, pairable, pairs_complete
            n_rows = int(self.inputs["atom_types"].shape[0])
            want_pairs, pair_shifts = (model.edge_pair_shifts(model._prepare_predict_graph(base, *flags))
                                       if hasattr(model, "edge_pair_shifts") else (False, None))
            with torch.cuda.stream(side):
                warm = build_graph(self.inputs["edge_index"], n_rows)  # warm-up outside the capture
                want_pairs = want_pairs and pairable(warm, pair_shifts)
                if want_pairs:
                    launch_edge_pairs(warm, pair_shifts)
            torch.cuda.current_stream().wait_stream(side)
            self.topology = torch.cuda.CUDAGraph()
            with torch.cuda.graph(self.topology):
                csr = build_graph(self.inputs["edge_index"], n_rows)
                pend = launch_edge_pairs(csr, pair_shifts) if want_pairs else None
                sorted_senders = csr.sort_senders()  # the sender order without a pairing
                base["csr"] = csr
            self.topology.replay()  # capturing records the work without running it
            if pend is not None:
                # the captured prediction takes the pairing whenever this first edge list pairs up;
                # a later edge list whose pairing state differs is evaluated eagerly (__call__)
                self.pair_counts = pend[1]
                self.paired = pairs_complete(pend[1], csr.n_edges)
                csr.set_edge_pairs(pair_shifts, pend[0] if self.paired else None)
            # both sender orders are refreshed by every topology replay
            if self.paired:
                csr.set_senders(pend[0].reverse, csr.rowptr)
            else:
                csr.set_senders(*sorted_senders)
            self._src_edges = self._topology_sources(tensors)

        def run():
            g = model._prepare_predict_graph(base, *flags)
            return model._predict_impl(g, *flags)

        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            for _ in range(2):  # allocator and library warm-up outside the capture
                run()
        torch.cuda.current_stream().wait_stream(side)
        self.graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(self.graph):
            self.outputs = run()

    @staticmethod
    def _topology_sources(tensors):
        """The tensors the topology graph depends on (edge list, periodic shifts) with their
        in-place version counters."""
        return tuple((tensors[k], tensors[k]._version) for k in ("edge_index", "shifts") if k in tensors)

    def _same_topology(self, tensors) -> bool:
        src = self._src_edges
        now = self._topology_sources(tensors)
        return (src is not None and len(src) == len(now)
                and all(a[0] is b[0] and a[1] == b[1] for a, b in zip(src, now)))

    def __call__(self, tensors):
        edges = tensors["edge_index"]
        same_edges = self.topology is not None and self._same_topology(tensors)
        for k, buf in self.inputs.items():
            if not (same_edges and k == "edge_index"):
                buf.copy_(tensors[k])
        if self.topology is not None and not same_edges:
            self.topology.replay()
            self._src_edges = self._topology_sources(tensors)
            if self.pair_counts is not None:
                from flashcart_amd.o3._graph import pairs_complete
                if pairs_complete(self.pair_counts, int(edges.shape[1])) != self.paired:
                    self._src_edges = None  # replay the topology again next time
                    return None
        self.graph.replay()
        return {k: v.clone() for k, v in self.outputs.items()}


class AtomisticModel(nn.Module):
    """Base class: site energies -> per-structure energies and their derivatives."""

    def forward(self, graph: Dict[str, torch.Tensor]) -> torch.Tensor:  # pragma: no cover - abstract
        raise NotImplementedError()

    def predict(self, graph, compute_forces: bool = False, compute_stress: bool = False,
                compute_edge_forces: bool = False, create_graph: bool = False, use_compile: bool = False,
                compile_mode: str = "reduce-overhead", fullgraph: bool = True,
                dynamic: bool = False) -> Dict[str, torch.Tensor]:
        """Energies and requested derivatives (reference ``model/atomistic.py:75-156``).

        ``create_graph`` keeps the derivatives differentiable (force-loss training): the
        returned energies and forces carry autograd graphs whose backward runs the second
        derivatives of the ops. Every block then runs op by op (no fused first-order
        backward) and ``use_compile`` is ignored (graph replay serves inference only).

        ``use_compile`` takes the place of the reference's ``torch.compile`` (default mode
        "reduce-overhead", i.e. graph replay): the whole prediction, forward and backward,
        is captured once per set of input shapes as a HIP graph and replayed, with the
        graph's tensors copied into the captured input buffers on every call. Like the
        reference's cached compiled functions, a new shape (atom or edge count) captures
        a new graph. ``compile_mode``, ``fullgraph`` and ``dynamic`` are accepted for API
        compatibility; shapes are always static.

        Per-structure energies are segment sums over ``batch``, which must be sorted (atoms of
        a structure contiguous, as ``batch_graphs`` and the reference's ``Batch.from_data_list``
        build it); a plain dict graph is checked for that here.
        """
        if isinstance(graph, dict):
            self._check_batch_sorted(graph["batch"])
        if create_graph:
            from flashcart_amd.nn import fused
            with fused.disabled():
                gd = self._prepare_predict_graph(graph, compute_forces, compute_stress, compute_edge_forces)
                return self._predict_impl(gd, compute_forces, compute_stress, compute_edge_forces, True)
        if use_compile:
            return self._replay_predict(_graph_dict(graph), compute_forces, compute_stress, compute_edge_forces)
        gd = self._prepare_predict_graph(graph, compute_forces, compute_stress, compute_edge_forces)
        return self._predict_impl(gd, compute_forces, compute_stress, compute_edge_forces)

    def _check_batch_sorted(self, b: torch.Tensor) -> None:
        """Raise unless ``b`` is sorted. The answer is remembered for the tensor object and its
        in-place version (the tensor is kept referenced, so its identity is meaningful), so an MD
        loop passing the same batch vector reads it from the device once, not at every call."""
        if b.numel() <= 1:
            return
        seen = self.__dict__.get("_sorted_batch")
        if seen is not None and seen[0] is b and seen[1] == b._version:
            return
        if not bool((b[1:] >= b[:-1]).all()):
            raise ValueError("graph['batch'] must be sorted: the atoms of each structure contiguous.")
        self.__dict__["_sorted_batch"] = (b, b._version)

    def _replay_predict(self, gd, compute_forces, compute_stress, compute_edge_forces):
        flags = (bool(compute_forces), bool(compute_stress), bool(compute_edge_forces))
        tensors = {k: v for k, v in gd.items() if torch.is_tensor(v)}
        if not all(v.is_cuda for v in tensors.values()):
            raise RuntimeError("use_compile replays a HIP graph: move the graph to the model's ROCm device first.")
        plain = tuple(sorted((k, v) for k, v in gd.items()
                             if not torch.is_tensor(v) and k not in ("_source", "csr")
                             and isinstance(v, (bool, int, float, str))))
        key = flags + plain + tuple(sorted((k, tuple(v.shape), v.dtype, str(v.device)) for k, v in tensors.items()))
        # Captured kernels read parameters and buffers in place (each interaction's
        # sqrt_avg_neighbors included: the kernels divide by it on the device), so values written
        # in place by any route are seen by the next replay; a re-capture when any of them was
        # reallocated.
        key += tuple(t.data_ptr() for t in self.parameters()) + tuple(t.data_ptr() for t in self.buffers())
        cache = self.__dict__.setdefault("_replay_cache", {})
        entry = cache.get(key)
        if entry is None:
            entry = _PredictReplay(self, gd, tensors, flags)
            cache[key] = entry
        out = entry(tensors)
        if out is None:  # the captured edge pairing does not hold for this edge list
            gd = self._prepare_predict_graph(gd, compute_forces, compute_stress, compute_edge_forces)
            return self._predict_impl(gd, compute_forces, compute_stress, compute_edge_forces)
        return out

    def _prepare_predict_graph(self, graph, compute_forces, compute_stress, compute_edge_forces):
        gd = _graph_dict(graph)
        gd["use_shifts"] = uses_periodic_shifts(gd.get("use_shifts", gd.get("pbc")))
        if not (compute_forces or compute_stress or compute_edge_forces):
            gd["positions"] = gd["positions"].detach()
            return gd
        positions = gd["positions"].detach()
        cell = gd["cell"].detach() if torch.is_tensor(gd.get("cell")) else None
        if compute_stress:
            if cell is None:
                raise ValueError("Cannot compute stress without cell information.")
            disp = torch.zeros_like(cell).requires_grad_(True)
            sym = 0.5 * (disp + disp.transpose(-1, -2))
            scaling = torch.eye(3, device=cell.device, dtype=cell.dtype).unsqueeze(0) + sym
            positions = (positions.unsqueeze(-2) @ scaling[gd["batch"]]).squeeze(-2)
            cell = cell @ scaling
            gd["displacement"] = disp
        if compute_forces:
            positions.requires_grad_(True)
        gd["positions"] = positions
        gd["cell"] = cell
        if compute_edge_forces:
            v = gd.get("vectors")
            if v is None:
                raise ValueError("Cannot compute edge forces without graph.vectors.")
            gd["vectors"] = v.detach().requires_grad_(True)
        return gd

    def _predict_impl(self, gd, compute_forces, compute_stress, compute_edge_forces, create_graph=False):
        node_energies = self(gd)
        out = {"node_energies": node_energies}
        n_atoms = gd["n_atoms"]
        if node_energies.shape[0] == gd["batch"].shape[0]:
            # Segment bounds from `batch` itself (the vector the forces' backward follows), so
            # energies and forces always agree; the segmented sum needs `batch` sorted, as every
            # graph builder here (and the reference's Batch.from_data_list) makes it.
            batch = gd["batch"]
            ptr = torch.searchsorted(batch, torch.arange(n_atoms.shape[0] + 1, device=batch.device,
                                                         dtype=batch.dtype))
            out["energy"] = _ops.segment_sum(node_energies, ptr, batch)
        else:
            out["energy"] = node_energies.sum().reshape(1)
        inputs, names = [], []
        if compute_forces:
            inputs.append(gd["positions"]); names.append("forces")
        if compute_stress:
            inputs.append(gd["displacement"]); names.append("stress")
        if compute_edge_forces:
            inputs.append(gd["vectors"]); names.append("edge_forces")
        if inputs:
            grads = torch.autograd.grad(out["energy"].sum(), inputs, allow_unused=True, create_graph=create_graph)
            for name, g, x in zip(names, grads, inputs):
                g = torch.zeros_like(x) if g is None else g
                if name == "forces":
                    out["forces"] = -g
                elif name == "stress":
                    vol = torch.det(gd["cell"])
                    out["stress"] = to_voigt6(g / vol.view(-1, 1, 1))
                    out["virials"] = -out["stress"] * vol.unsqueeze(-1)
                else:
                    out["edge_forces"] = g
            if not create_graph:
                out["node_energies"] = out["node_energies"].detach()
                out["energy"] = out["energy"].detach()
        return out

    # -- checkpoints (reference model/atomistic.py:441-527) -------------------------------
    def to_model_config(self) -> Dict[str, Any]:  # pragma: no cover - abstract
        raise NotImplementedError()

    @classmethod
    def from_config(cls, cfg: Dict[str, Any]) -> "AtomisticModel":  # pragma: no cover - abstract
        raise NotImplementedError()

    def save_weights(self, path: Union[str, Path], filename: str = "model.pt") -> None:
        path = Path(path)
        path.mkdir(parents=True, exist_ok=True)
        torch.save(self.state_dict(), path / filename)

    def load_weights(self, path: Union[str, Path], filename: str = "model.pt", map_location="cpu") -> None:
        self.load_state_dict(torch.load(Path(path) / filename, weights_only=True, map_location=map_location))

    def save_inference_checkpoint(self, path: Union[str, Path], meta: Optional[Dict[str, Any]] = None) -> None:
        self.save_weights(path)
        save_inference_metadata(Path(path), self.to_model_config(), meta=meta)

    @classmethod
    def from_checkpoint(cls, ckpt_dir: Union[str, Path], device=None, map_location="cpu") -> "AtomisticModel":
        model = cls.from_config(load_model_config(Path(ckpt_dir)))
        model.load_weights(ckpt_dir, map_location=map_location)
        if device is not None:
            model = model.to(device)
        model.eval()
        return model
