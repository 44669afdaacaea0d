"""LAMMPS ML-IAP interface (reference src/flashcart/calculators/lammps_mliap.py:122-803).

``FlashCartLAMMPSUnified.compute_forces(data)`` reads the per-step wire format of the
ML-IAP "unified" interface — ``nlocal``, ``ntotal``, ``npairs``, ``pair_i`` (owned
receivers), ``pair_j`` (owned or ghost senders), ``rij`` (pair vectors) and ``elems``
(element index per atom) — evaluates the owned atoms' site energies, differentiates
the energy with respect to ``rij`` (edge forces), and hands them to
``data.update_pair_forces`` (or accumulates them into ``data.f``). Models with more
than one interaction layer refresh ghost-atom features between layers through the
data object's ``forward_exchange`` / ``reverse_exchange`` hooks
(:mod:`flashcart_amd.utils.lammps`).

Arrays that LAMMPS exposes on the device (``__cuda_array_interface__``, which ROCm
builds of PyTorch read for HIP memory) are used in place; host arrays are copied to
the model's device. Evaluation always uses the HIP kernels, so ``compile_mode`` is
accepted for configuration compatibility and evaluation is eager.
"""

from __future__ import annotations

import os
import sys
from pathlib import Path
from typing import Dict, List, NoReturn, Optional, Union

import numpy as np
import torch

from flashcart_amd.data.graph import atomic_number
from flashcart_amd.model.flashcart import FlashCartPotential
from flashcart_amd.utils.lammps import lammps_data_slot

COMPILE_MODES = ("default", "max-autotune-no-cudagraphs")

try:  # pragma: no cover - depends on the environment
    from lammps.mliap.mliap_unified_abc import MLIAPUnified
except ImportError:

    class MLIAPUnified:  # type: ignore[no-redef]
        def __init__(self, *args, **kwargs):
            pass


def _on_device(v) -> bool:
    return (torch.is_tensor(v) and v.is_cuda) or (not torch.is_tensor(v) and hasattr(v, "__cuda_array_interface__"))


def _array_device(values, requested: Optional[torch.device]) -> torch.device:
    """Device for the step's tensors: the ROCm device the arrays live on, else the
    requested device (host arrays are copied there; the kernels run on the GPU only)."""
    if any(_on_device(v) for v in values):
        if requested is not None and torch.device(requested).type == "cuda":
            return torch.device(requested)
        if not torch.cuda.is_available():
            raise RuntimeError("LAMMPS provides device ML-IAP arrays, but no ROCm device is visible to this process.")
        return torch.device("cuda")
    if requested is None:
        if not torch.cuda.is_available():
            raise RuntimeError("FlashCart's HIP kernels need a visible ROCm device.")
        return torch.device("cuda")
    return torch.device(requested)


def _check_range(name: str, idx: torch.Tensor, size: int) -> None:
    if idx.numel() and (int(idx.min()) < 0 or int(idx.max()) >= size):
        raise ValueError(f"LAMMPS {name} holds indices outside [0, {size}).")


def graph_dict_from_mliap(data, element_types: List[str], device: Optional[torch.device] = None,
                          dtype: Optional[torch.dtype] = None, validate: bool = False) -> Dict[str, object]:
    """Graph dictionary (edge vectors instead of positions) of one ML-IAP call
    (reference calculators/lammps_mliap.py:122-173)."""
    ntotal, nlocal, npairs = int(data.ntotal), int(data.nlocal), int(data.npairs)
    if npairs <= 0 or ntotal <= 0:
        raise ValueError(f"Empty ML-IAP layout: ntotal={ntotal}, npairs={npairs}.")
    dtype = torch.get_default_dtype() if dtype is None else dtype
    arrays = (data.pair_i, data.pair_j, data.rij, data.elems)
    device = _array_device(arrays, device)
    pair_i = torch.as_tensor(data.pair_i, device=device)[:npairs].to(torch.long)
    pair_j = torch.as_tensor(data.pair_j, device=device)[:npairs].to(torch.long)
    vectors = torch.as_tensor(data.rij, device=device)[:npairs].to(dtype)
    atom_types = torch.as_tensor(data.elems, device=device)[:ntotal].to(torch.long)
    if vectors.ndim != 2 or vectors.shape[-1] != 3:
        raise ValueError(f"LAMMPS rij must have shape (npairs, 3), got {tuple(vectors.shape)}.")
    if validate:
        _check_range("pair_i", pair_i, nlocal)
        _check_range("pair_j", pair_j, ntotal)
        _check_range("elems", atom_types, len(element_types))
    z_table = torch.tensor([atomic_number(s) for s in element_types], dtype=torch.long, device=device)
    return {
        "n_atoms": torch.tensor([nlocal], dtype=torch.long, device=device),
        "edge_index": torch.stack([pair_i, pair_j], dim=0),
        "atomic_numbers": z_table[atom_types],
        "atom_types": atom_types,
        "vectors": vectors,
        "batch": torch.zeros(nlocal, dtype=torch.long, device=device),
        "use_shifts": False,
        "lammps_exchange": True,
    }


class _IdentityExchange:
    """Exchange for a rank without ghost atoms and without LAMMPS communication hooks."""

    def forward_exchange(self, feats, out, vec_len: int) -> None:
        out.copy_(feats)

    def reverse_exchange(self, grads, out, vec_len: int) -> None:
        out.copy_(grads)


def _exchange_object(data, nlocal: int, ntotal: int):
    if hasattr(data, "forward_exchange") and hasattr(data, "reverse_exchange"):
        return data
    if ntotal == nlocal:
        return _IdentityExchange()
    raise RuntimeError("Ghost atoms require the ML-IAP communication hooks (KOKKOS ML-IAP build), "
                       "or use a model with one interaction layer.")


def _has_attr(data, name: str) -> bool:
    return hasattr(type(data), name) or name in getattr(data, "__dict__", {})


class FlashCartLAMMPSUnified(MLIAPUnified):
    """FlashCart potential behind the LAMMPS ML-IAP unified interface."""

    def __init__(self, model: FlashCartPotential, add_atomic_offsets: bool = False,
                 compile_mode: Optional[str] = None, compile_fullgraph: bool = True):
        super().__init__()
        if compile_mode is not None and compile_mode not in COMPILE_MODES:
            raise ValueError(f"compile_mode must be one of {COMPILE_MODES} or None, got {compile_mode!r}.")
        self.model = model
        self.element_types = list(model.elements)
        self.r_max = float(model.r_max)
        self.rcutfac = 0.5 * self.r_max
        self.ndescriptors = 1
        self.nparams = 1
        self.dtype = next(model.parameters()).dtype
        self.add_atomic_offsets = bool(add_atomic_offsets)
        self.compile_mode = compile_mode
        self.compile_fullgraph = bool(compile_fullgraph)
        self._atomic_shifts = model.scale_shift.shifts.detach().to(torch.float64)
        # The model stays where it is until the first step picks the arrays' device.
        self.device = next(model.parameters()).device
        self.model = self.model.eval()
        self._checked = False
        for p in self.model.parameters():
            p.requires_grad_(False)

    def compute_descriptors(self, data) -> None:
        pass

    def compute_gradients(self, data) -> None:
        pass

    def _fail(self, message: str) -> NoReturn:
        # An exception inside a LAMMPS callback would leave the other ranks waiting in
        # the next exchange: end an attached process instead.
        if getattr(self, "interface", None) is not None:
            try:
                print(f"FlashCart LAMMPS: {message}", file=sys.stderr, flush=True)
            finally:
                os._exit(1)
        raise RuntimeError(message)

    def compute_forces(self, data) -> None:
        """Site energies and edge forces of one step (reference lammps_mliap.py:635-744)."""
        nlocal, ntotal, npairs = int(data.nlocal), int(data.ntotal), int(data.npairs)
        if nlocal == 0 or npairs <= 0:
            self._fail(f"This rank owns {nlocal} atoms with {npairs} neighbor pairs. Every rank must own atoms "
                       "with neighbor pairs.")
        validate = not self._checked or os.environ.get("FLASHCART_LAMMPS_VALIDATE", "0") not in ("", "0")
        graph = graph_dict_from_mliap(data, self.element_types,
                                      device=self.device if self.device.type == "cuda" else None, dtype=self.dtype,
                                      validate=validate)
        self._checked = True
        if graph["vectors"].device != self.device:
            self.device = graph["vectors"].device
            self.model = self.model.to(self.device)
        graph["vectors"] = graph["vectors"].detach().requires_grad_(True)
        exchange_data = data
        if self.model.n_interactions > 1:
            try:
                exchange_data = _exchange_object(data, nlocal, ntotal)
            except RuntimeError as exc:
                self._fail(str(exc))
        with lammps_data_slot(exchange_data):
            out = self.model._predict_impl(graph, compute_forces=False, compute_stress=False,
                                           compute_edge_forces=True)
        pair_forces = out["edge_forces"].detach().to(torch.float64)

        if bool(getattr(data, "eflag", True)):
            e_local = out["node_energies"].detach().to(torch.float64)[:nlocal]
            if self.add_atomic_offsets:
                e_local = e_local + self._atomic_shifts.to(e_local.device)[graph["atom_types"][:nlocal]]
            if _has_attr(data, "eatoms"):
                buf = getattr(data, "eatoms", None)
                if buf is None:
                    data.eatoms = e_local.cpu().numpy()
                else:
                    t = torch.as_tensor(buf)
                    t[:nlocal].copy_(e_local.to(dtype=t.dtype, device=t.device))
            data.energy = float(e_local.sum().cpu())

        if hasattr(data, "update_pair_forces"):
            data.update_pair_forces(pair_forces if pair_forces.is_cuda else pair_forces.numpy())
            return
        f_view = data.f
        if f_view is None:
            raise RuntimeError("ML-IAP data.f is NULL: Cannot write forces.")
        # dE/d r_ij with r_ij = x_j - x_i: +g on the receiver i, -g on the sender j.
        pair_i, pair_j = graph["edge_index"]
        forces = torch.zeros(ntotal, 3, dtype=pair_forces.dtype, device=pair_forces.device)
        forces.index_add_(0, pair_i, pair_forces)
        forces.index_add_(0, pair_j, -pair_forces)
        if torch.is_tensor(f_view):
            f_view[:ntotal].copy_(forces.to(dtype=f_view.dtype, device=f_view.device))
        else:
            np.asarray(f_view)[:ntotal, :] = forces.cpu().numpy()


def build_lammps_unified(checkpoint: Union[str, Path], compile_mode: Optional[str] = None) -> FlashCartLAMMPSUnified:
    """Load an inference checkpoint on the host and wrap it for LAMMPS."""
    model = FlashCartPotential.from_checkpoint(checkpoint, device=torch.device("cpu"), map_location="cpu")
    return FlashCartLAMMPSUnified(model, compile_mode=compile_mode)


class SingleRankMLIAPData:
    """A periodic structure in the layout a single-rank LAMMPS run hands to ML-IAP: owned
    atoms, one ghost atom per periodic image that a pair reaches, pair indices into
    owned + ghost atoms and the pair vectors r_ij = x_j - x_i on the device. The exchange
    hooks copy owner features to their ghosts and add ghost gradients back to the owners,
    as LAMMPS's forward / reverse communication does on one rank.

    Drives ``FlashCartLAMMPSUnified.compute_forces`` without LAMMPS (tests, benchmarks);
    pair forces are kept as a device tensor (``pair_forces``) through
    ``update_pair_forces``, and ``atom_forces()`` folds them onto the owned atoms."""

    def __init__(self, graph, device=None):
        ei = graph.edge_index.cpu().numpy()
        shifts = graph.shifts.cpu().numpy().astype(np.int64)
        n_local = int(graph.positions.shape[0])
        ghost = np.any(shifts != 0, axis=1)
        keys, inv = np.unique(np.concatenate([ei[1][ghost, None], shifts[ghost]], axis=1), axis=0,
                              return_inverse=True)
        pair_j = ei[1].copy()
        pair_j[ghost] = n_local + inv.reshape(-1)
        device = torch.device(device) if device is not None else graph.positions.device
        self.nlocal = n_local
        self.ntotal = n_local + keys.shape[0]
        self.npairs = ei.shape[1]
        self.owner = torch.as_tensor(keys[:, 0], device=device)
        pos = graph.positions.double().cpu().numpy()
        cell = graph.cell[0].double().cpu().numpy()
        self.pair_i = torch.as_tensor(ei[0].astype(np.int32), device=device)
        self.pair_j = torch.as_tensor(pair_j.astype(np.int32), device=device)
        self.rij = torch.as_tensor(pos[ei[1]] + shifts @ cell - pos[ei[0]], dtype=torch.float32, device=device)
        types = graph.atom_types.cpu().numpy()
        self.elems = torch.as_tensor(np.concatenate([types, types[keys[:, 0]]]).astype(np.int32), device=device)
        self.eflag = True
        self.eatoms = None
        self.energy = None
        self.pair_forces = None

    def forward_exchange(self, src, dst, width) -> None:
        dst[: self.nlocal] = src[: self.nlocal]
        dst[self.nlocal:] = src[self.owner]

    def reverse_exchange(self, src, dst, width) -> None:
        dst.copy_(src)
        dst[self.nlocal:] = 0
        dst.index_add_(0, self.owner, src[self.nlocal:])

    def update_pair_forces(self, pair_forces) -> None:
        self.pair_forces = pair_forces

    def atom_forces(self) -> torch.Tensor:
        """Forces on the owned atoms: -dE/dx from the pair forces dE/dr_ij, ghost forces folded
        onto their owners."""
        pf = torch.as_tensor(self.pair_forces)
        f = torch.zeros(self.ntotal, 3, dtype=pf.dtype, device=pf.device)
        f.index_add_(0, self.pair_i.to(pf.device, torch.long), pf)
        f.index_add_(0, self.pair_j.to(pf.device, torch.long), -pf)
        out = f[: self.nlocal].clone()
        out.index_add_(0, self.owner.to(pf.device), f[self.nlocal:])
        return out


def save_lammps_unified(unified: FlashCartLAMMPSUnified, path: Union[str, Path]) -> Path:
    """Write the interface for the LAMMPS ``pair_style mliap unified <file>`` command
    (``torch.save`` of the object, as the reference does)."""
    path = Path(path)
    path.parent.mkdir(parents=True, exist_ok=True)
    torch.save(unified, path)
    return path
