"""Atomic graphs and batching (reference src/flashcart/data/data.py:185-323, data/graph.py,
utils/torch_geometric/batch.py:42-137).

``AtomicGraph`` carries the same fields as the reference's ``AtomicData``
(positions, cell (G,3,3), pbc (G,3), shifts (E,3) integer cell translations,
edge_index (2,E) with row 0 = receivers sorted, atom_types, n_atoms (G,), batch)
and ``batch_graphs`` concatenates graphs with the node offsets added to edge_index,
so receiver order stays globally sorted.
"""

from __future__ import annotations

from typing import Dict, List, Optional, Sequence, Union

import numpy as np
import torch

from flashcart_amd.data.neighbors import NeighborList

_ATOMIC_NUMBERS = {
    "H": 1, "He": 2, "Li": 3, "Be": 4, "B": 5, "C": 6, "N": 7, "O": 8, "F": 9, "Ne": 10, "Na": 11, "Mg": 12,
    "Al": 13, "Si": 14, "P": 15, "S": 16, "Cl": 17, "Ar": 18, "K": 19, "Ca": 20, "Sc": 21, "Ti": 22, "V": 23,
    "Cr": 24, "Mn": 25, "Fe": 26, "Co": 27, "Ni": 28, "Cu": 29, "Zn": 30, "Ga": 31, "Ge": 32, "As": 33,
    "Se": 34, "Br": 35, "Kr": 36,
}


def atomic_number(symbol: Union[str, int]) -> int:
    return int(symbol) if not isinstance(symbol, str) else _ATOMIC_NUMBERS[symbol]


def numbers_to_types(numbers: Sequence[int], elements: Sequence[Union[str, int]]) -> np.ndarray:
    """Zero-based element indices in ``elements`` order (reference data/utils.py numbers_to_types)."""
    lut = {atomic_number(e): k for k, e in enumerate(elements)}
    try:
        return np.asarray([lut[int(z)] for z in numbers], dtype=np.int64)
    except KeyError as exc:
        raise ValueError(f"atomic number {exc.args[0]} is not in elements {list(elements)}") from None


class AtomicGraph:
    """Tensor graph of one or more structures."""

    TENSOR_FIELDS = ("positions", "cell", "pbc", "shifts", "edge_index", "atom_types", "atomic_numbers", "n_atoms",
                     "batch", "ptr", "vectors", "energy", "forces")

    def __init__(self, **fields):
        for k, v in fields.items():
            setattr(self, k, v)
        if getattr(self, "batch", None) is None and getattr(self, "positions", None) is not None:
            n = self.positions.shape[0]
            self.batch = torch.zeros(n, dtype=torch.long, device=self.positions.device)
        if getattr(self, "ptr", None) is None and getattr(self, "n_atoms", None) is not None:
            self.ptr = torch.cat([torch.zeros(1, dtype=torch.long, device=self.n_atoms.device),
                                  torch.cumsum(self.n_atoms, 0)])
        self.csr = None  # GraphCSR cached per device by the model

    @property
    def num_nodes(self) -> int:
        return int(self.positions.shape[0])

    @property
    def num_graphs(self) -> int:
        return int(self.n_atoms.shape[0])

    def to(self, device) -> "AtomicGraph":
        out = AtomicGraph.__new__(AtomicGraph)
        for k, v in self.__dict__.items():
            setattr(out, k, v.to(device) if torch.is_tensor(v) else v)
        out.csr = None
        return out

    def to_dict(self) -> Dict[str, object]:
        d = {k: v for k, v in self.__dict__.items() if v is not None}
        if "use_shifts" not in d:  # (a device pbc tensor costs a synchronisation)
            d["use_shifts"] = bool(torch.any(self.pbc).item()) if torch.is_tensor(getattr(self, "pbc", None)) \
                else True
        return d

    @classmethod
    def from_arrays(cls, numbers: Sequence[int], positions: np.ndarray, elements: Sequence[Union[str, int]],
                    r_max: float, cell: Optional[np.ndarray] = None, pbc=False, skin: float = 0.0,
                    neighbors: Optional[NeighborList] = None, dtype: Optional[torch.dtype] = None) -> "AtomicGraph":
        """Build the graph of one structure (positions in Angstrom, cell rows = lattice vectors)."""
        dtype = dtype or torch.get_default_dtype()
        pos = np.asarray(positions, dtype=np.float64).reshape(-1, 3)
        cell = np.zeros((3, 3)) if cell is None else np.asarray(cell, dtype=np.float64).reshape(3, 3)
        pbc_arr = np.broadcast_to(np.asarray(pbc, dtype=bool), (3,)).copy()
        nl = neighbors if neighbors is not None else NeighborList(r_max, skin).build(pos, cell, pbc_arr)
        n = pos.shape[0]
        types = numbers_to_types(numbers, elements)
        g = cls(
            positions=torch.as_tensor(pos, dtype=dtype),
            cell=torch.as_tensor(cell, dtype=dtype).unsqueeze(0),
            pbc=torch.as_tensor(pbc_arr).unsqueeze(0),
            shifts=torch.as_tensor(nl.unit_shifts, dtype=torch.long),
            edge_index=torch.as_tensor(nl.edge_index, dtype=torch.long),
            atom_types=torch.as_tensor(types, dtype=torch.long),
            atomic_numbers=torch.as_tensor(np.asarray(numbers), dtype=torch.long),
            n_atoms=torch.tensor([n], dtype=torch.long),
            use_shifts=bool(pbc_arr.any()),
        )
        g.neighbors = nl
        return g


def batch_graphs(graphs: List[AtomicGraph]) -> AtomicGraph:
    """Concatenate graphs; edge_index is offset by the running node count."""
    offs, ei, batch = 0, [], []
    for k, g in enumerate(graphs):
        ei.append(g.edge_index + offs)
        batch.append(torch.full((g.num_nodes,), k, dtype=torch.long, device=g.positions.device))
        offs += g.num_nodes
    cat = lambda name: torch.cat([getattr(g, name) for g in graphs], dim=0)
    return AtomicGraph(
        positions=cat("positions"), cell=cat("cell"), pbc=cat("pbc"), shifts=cat("shifts"),
        edge_index=torch.cat(ei, dim=1), atom_types=cat("atom_types"), atomic_numbers=cat("atomic_numbers"),
        n_atoms=cat("n_atoms"), batch=torch.cat(batch), use_shifts=any(bool(getattr(g, "use_shifts", True))
                                                                        for g in graphs),
    )


def update_graph_positions(graph: AtomicGraph, positions: np.ndarray, cell: Optional[np.ndarray] = None):
    """Reuse connectivity with new positions (and cell) (reference data/graph.py:70-92)."""
    out = graph.to(graph.positions.device)
    out.positions = torch.as_tensor(np.asarray(positions), dtype=graph.positions.dtype,
                                    device=graph.positions.device)
    if cell is not None:
        out.cell = torch.as_tensor(np.asarray(cell), dtype=graph.cell.dtype, device=graph.cell.device).reshape(1, 3, 3)
    out.csr = graph.csr
    return out
