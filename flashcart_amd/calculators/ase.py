"""ASE calculator front-end (reference src/flashcart/calculators/ase.py:14-230).

``FlashCartCalculator`` keeps the reference's constructor, ``implemented_properties``,
result conventions (energy as a float, forces (N,3), stress as 6 Voigt components
``xx, yy, zz, yz, xz, xy``) and neighbour-list reuse rule (a positive ``skin``, only
positions/cell changed, every displacement and the cell change below ``skin / 2``).

When ``ase`` is installed the class derives from ``ase.calculators.calculator.Calculator``.
Without it, a small base class provides the same ``calculate`` / ``get_property`` /
``results`` contract for any object with ``get_positions()``, ``get_atomic_numbers()``,
``get_cell()``, ``get_pbc()`` and ``copy()``.

Evaluation always runs the HIP kernels eagerly: they accept any atom and edge count,
so the reference's ``torch.compile`` shape padding (``compile_mode``, ``pad_*``) has no
role here; those arguments are accepted and reported as ignored.
"""

from __future__ import annotations

import warnings
from pathlib import Path
from typing import List, Optional, Union

import numpy as np
import torch

from flashcart_amd.data.graph import AtomicGraph, update_graph_positions
from flashcart_amd.model.flashcart import FlashCartPotential

_ALL_CHANGES = ["positions", "numbers", "cell", "pbc", "initial_charges", "initial_magmoms"]

try:  # pragma: no cover - depends on the environment
    from ase.calculators.calculator import Calculator as _CalculatorBase
    from ase.calculators.calculator import all_changes

    HAVE_ASE = True
except ImportError:
    HAVE_ASE = False
    all_changes = list(_ALL_CHANGES)

    class _CalculatorBase:
        """Subset of ``ase.calculators.calculator.Calculator`` used by the calculator."""

        implemented_properties: List[str] = []

        def __init__(self, **kwargs):
            self.parameters = dict(kwargs)
            self.atoms = None
            self.results = {}

        def check_state(self, atoms) -> List[str]:
            if self.atoms is None:
                return list(_ALL_CHANGES)
            changes = []
            if not np.array_equal(atoms.get_positions(), self.atoms.get_positions()):
                changes.append("positions")
            if not np.array_equal(atoms.get_atomic_numbers(), self.atoms.get_atomic_numbers()):
                changes.append("numbers")
            if not np.array_equal(np.asarray(atoms.get_cell()), np.asarray(self.atoms.get_cell())):
                changes.append("cell")
            if not np.array_equal(atoms.get_pbc(), self.atoms.get_pbc()):
                changes.append("pbc")
            return changes

        def calculate(self, atoms=None, properties=None, system_changes=all_changes):
            if atoms is not None:
                self.atoms = atoms.copy()

        def get_property(self, name: str, atoms=None, allow_calculation: bool = True):
            if name not in self.implemented_properties:
                raise NotImplementedError(f"{name} property not implemented")
            if atoms is None:
                atoms = self.atoms
                changes = []
            else:
                changes = self.check_state(atoms)
                if changes:
                    self.results = {}
            if name not in self.results:
                if not allow_calculation:
                    return None
                self.calculate(atoms, [name], changes)
            return self.results[name]

        def get_potential_energy(self, atoms=None, force_consistent: bool = False) -> float:
            return self.get_property("energy", atoms)

        def get_forces(self, atoms=None) -> np.ndarray:
            return self.get_property("forces", atoms)

        def get_stress(self, atoms=None) -> np.ndarray:
            return self.get_property("stress", atoms)


class FlashCartCalculator(_CalculatorBase):
    """Energies, forces and stress of a :class:`FlashCartPotential` for ASE structures."""

    implemented_properties = ["energy", "forces", "stress"]

    def __init__(self, checkpoint: Optional[Union[str, Path]] = None, model: Optional[FlashCartPotential] = None,
                 device: Optional[Union[str, torch.device]] = None, skin: float = 0.0,
                 compile_mode: Optional[str] = None, compile_fullgraph: bool = True, pad_n_atoms: int = 0,
                 pad_n_edges: int = 0, pad_extra_atoms: Optional[int] = None, pad_atom_multiple: int = 1,
                 pad_edge_headroom: float = 1.1, pad_edge_multiple: int = 128, add_atomic_offsets: bool = False,
                 **kwargs):
        super().__init__(**kwargs)
        if model is None:
            if checkpoint is None:
                raise ValueError("Provide either checkpoint or model.")
            model = FlashCartPotential.from_checkpoint(checkpoint, device=device)
            # the calculator's own copy only evaluates: frozen parameters select the fused
            # inference backward of the gated and product blocks
            model.requires_grad_(False)
        elif device is not None:
            model = model.to(device)
        if compile_mode is not None or pad_n_atoms > 0 or pad_n_edges > 0:
            warnings.warn("compile_mode and pad_* are ignored: the HIP kernels take any atom and edge count, "
                          "so the model is evaluated eagerly without padding.", UserWarning, stacklevel=2)
        self.model = model
        self._device = next(model.parameters()).device
        self.add_atomic_offsets = bool(add_atomic_offsets)
        self._atomic_shifts = model.scale_shift.shifts.detach().to(self._device)
        self.skin = float(skin)
        self.compile_mode = compile_mode
        self.compile_fullgraph = bool(compile_fullgraph)
        self._cached_graph: Optional[AtomicGraph] = None
        self._cached_positions: Optional[np.ndarray] = None
        self._cached_cell: Optional[np.ndarray] = None

    @classmethod
    def from_checkpoint(cls, checkpoint: Union[str, Path], device: Optional[Union[str, torch.device]] = None,
                        skin: float = 0.0, **kwargs) -> "FlashCartCalculator":
        return cls(checkpoint=checkpoint, device=device, skin=skin, **kwargs)

    def calculate(self, atoms=None, properties: Optional[List[str]] = None, system_changes=all_changes):
        """Evaluate ``properties`` (default energy and forces) into ``self.results``."""
        if properties is None:
            properties = ["energy", "forces"]
        super().calculate(atoms, properties, system_changes)
        if self.atoms is None:
            raise ValueError("No structure to evaluate.")
        graph = self._get_graph(system_changes)
        out = self.model.predict(graph, compute_forces="forces" in properties,
                                 compute_stress="stress" in properties)
        self.results = {}
        if "energy" in properties:
            energy = float(out["energy"].detach().double().cpu().reshape(-1)[0])
            if self.add_atomic_offsets:
                energy += float(self._atomic_shifts[graph.atom_types].double().sum().cpu())
            self.results["energy"] = energy
        if "forces" in properties:
            self.results["forces"] = out["forces"].detach().cpu().numpy()
        if "stress" in properties:
            self.results["stress"] = out["stress"].detach().cpu().numpy().reshape(-1)

    def _get_graph(self, system_changes: List[str]) -> AtomicGraph:
        """Reuse the cached connectivity when the reference's skin criterion allows it
        (reference calculators/ase.py:191-230), otherwise rebuild the neighbour list."""
        atoms = self.atoms
        positions = np.asarray(atoms.get_positions(), dtype=np.float64)
        cell = np.asarray(atoms.get_cell(), dtype=np.float64).reshape(3, 3)
        reuse = (self.skin > 0.0 and self._cached_graph is not None and set(system_changes) <= {"positions", "cell"})
        if reuse:
            disp = np.linalg.norm(positions - self._cached_positions, axis=-1)
            cell_disp = np.linalg.norm(cell - self._cached_cell)
            if np.all(disp < self.skin / 2) and cell_disp < self.skin / 2:
                return update_graph_positions(self._cached_graph, positions, cell)
        dtype = next(self.model.parameters()).dtype
        graph = AtomicGraph.from_arrays(atoms.get_atomic_numbers(), positions, self.model.elements,
                                        self.model.r_max, cell=cell, pbc=atoms.get_pbc(), skin=self.skin,
                                        dtype=dtype).to(self._device)
        self._cached_graph = graph
        self._cached_positions = positions.copy()
        self._cached_cell = cell.copy()
        return graph
