"""Neighbour lists (reference src/flashcart/data/neighbors.py).

``NeighborList`` keeps the reference's interface (``r_max``, ``skin``, ``build``,
``from_arrays``, ``edge_index`` / ``unit_shifts`` arrays). The pairs come from the
host cell list of libflashcart_hip.so (``fc_neighbor_list``) in the canonical order
(i, j, Sx, Sy, Sz); the reference delegates to matscipy, whose order inside a
receiver block is not documented, so only the edge set and the receiver sort are
shared with it.
"""

from __future__ import annotations

import ctypes
from typing import Optional, Union

import numpy as np

from flashcart_amd import _lib


def neighbor_pairs(positions: np.ndarray, cell: np.ndarray, pbc, cutoff: float, eps: float = 1e-7):
    """(edge_index (2, E) int64 [i; j], unit_shifts (E, 3) int32) for one structure.

    A near-singular cell is replaced by a bounding box padded by 2 * cutoff, as the
    reference does before calling its backend (reference ``neighbors.py:131-135``).
    """
    pos = np.ascontiguousarray(positions, dtype=np.float64).reshape(-1, 3)
    cell = np.ascontiguousarray(cell, dtype=np.float64).reshape(3, 3)
    pbc = np.broadcast_to(np.asarray(pbc, dtype=bool), (3,))
    if abs(np.linalg.det(cell)) < eps:
        span = np.ptp(pos, axis=0) if len(pos) else np.zeros(3)
        cell = np.diag(np.maximum(span, 1e-3) + 2.0 * cutoff)
        pbc = np.zeros(3, dtype=bool)
    n = pos.shape[0]
    flags = np.ascontiguousarray(pbc.astype(np.int32))
    lib = _lib.load()
    cap = max(64, int(n * 64))
    while True:
        ei = np.empty(cap, dtype=np.int64)
        ej = np.empty(cap, dtype=np.int64)
        sh = np.empty((cap, 3), dtype=np.int32)
        cnt = lib.fc_neighbor_list(n, pos.ctypes.data, cell.ctypes.data, flags.ctypes.data, float(cutoff), cap,
                                   ei.ctypes.data, ej.ctypes.data, sh.ctypes.data)
        if cnt < 0:
            raise ValueError(f"fc_neighbor_list failed with status {cnt}.")
        if cnt <= cap:
            return np.stack([ei[:cnt], ej[:cnt]]), sh[:cnt].copy()
        cap = int(cnt)


class NeighborList:
    """Pairs within ``r_max + skin`` (reference ``neighbors.py:10-117``)."""

    def __init__(self, r_max: float, skin: float = 0.0, backend: str = "native"):
        self.r_max = r_max
        self.skin = skin
        self.backend = backend
        self.edge_index: Optional[np.ndarray] = None
        self.unit_shifts: Optional[np.ndarray] = None

    @property
    def is_built(self) -> bool:
        return self.edge_index is not None

    def copy(self) -> "NeighborList":
        nl = NeighborList(self.r_max, self.skin, self.backend)
        nl.edge_index = None if self.edge_index is None else self.edge_index.copy()
        nl.unit_shifts = None if self.unit_shifts is None else self.unit_shifts.copy()
        return nl

    def build(self, positions: np.ndarray, cell: np.ndarray, pbc: Union[bool, list]) -> "NeighborList":
        ei, sh = neighbor_pairs(positions, cell, pbc, self.r_max + self.skin)
        self.edge_index = np.asarray(ei, dtype=np.int64)
        self.unit_shifts = np.asarray(sh, dtype=np.int32)
        return self

    @classmethod
    def from_arrays(cls, edge_index, unit_shifts, r_max: float = float("nan"), skin: float = 0.0,
                    backend: str = "native") -> "NeighborList":
        nl = cls(r_max, skin, backend)
        nl.edge_index = np.asarray(edge_index, dtype=np.int64)
        nl.unit_shifts = np.asarray(unit_shifts, dtype=np.int32)
        return nl
