"""Neighbour lists (reference src/flashcart/data/neighbors.py).

``NeighborList`` keeps the reference's interface (``r_max``, ``skin``, ``build``,
``from_arrays``, ``edge_index`` / ``unit_shifts`` arrays). The pairs come from the
host cell list of libflashcart_hip.so (``fc_neighbor_list``) in the canonical order
(i, j, Sx, Sy, Sz), or from its GPU twin (``fc_neighbor_list_device``, same pairs and
order) for positions already in HBM; the reference delegates to matscipy, whose order
inside a receiver block is not documented, so only the edge set and the receiver sort
are shared with it.
"""

from __future__ import annotations

import ctypes
from typing import Optional, Union

import numpy as np
import torch

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


_last_device_count = {}  # atom count -> pairs of the last device build (output size hint)


_FC_ERR_SHAPE = 4  # fc_status, include/flashcart_hip.h


def host_fallback_needed(status: int) -> bool:
    """Whether fc_neighbor_list_device's return value asks for the host list: -FC_ERR_SHAPE
    means an atom with more than 1,024 pairs or a shift component of 512 or more (sizes the
    device kernels do not hold); every other negative value is an error of its own."""
    return status == -_FC_ERR_SHAPE


def neighbor_pairs_device(positions: torch.Tensor, cell, pbc, cutoff: float, eps: float = 1e-7):
    """The pairs of ``neighbor_pairs`` built on the GPU from positions in HBM
    (``fc_neighbor_list_device``): (edge_index (2, E) int64, unit_shifts (E, 3) int32) on
    the positions' device, identical to the host list (same float64 tests, same order)."""
    if not positions.is_cuda:
        raise RuntimeError(f"neighbor_pairs_device needs positions on a ROCm device, got {positions.device}.")
    pos = positions.detach().to(torch.float64).reshape(-1, 3).contiguous()
    cell_np = np.ascontiguousarray(
        cell.detach().cpu().numpy() if torch.is_tensor(cell) else np.asarray(cell), dtype=np.float64).reshape(3, 3)
    pbc = np.broadcast_to(np.asarray(pbc.cpu() if torch.is_tensor(pbc) else pbc, dtype=bool).reshape(-1), (3,))
    n = pos.shape[0]
    if abs(np.linalg.det(cell_np)) < eps:  # open boundaries: a padded bounding box, as the host list
        span = (pos.amax(0) - pos.amin(0)).cpu().numpy() if n else np.zeros(3)
        cell_np = np.diag(np.maximum(span, 1e-3) + 2.0 * cutoff)
        pbc = np.zeros(3, dtype=bool)
    flags = np.ascontiguousarray(pbc.astype(np.int32))
    lib = _lib.load()
    ws_bytes = int(lib.fc_neighbor_list_device_workspace(n))
    if ws_bytes < 0:
        _lib.check(-ws_bytes, "fc_neighbor_list_device_workspace")
    ws = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=pos.device)
    # an undersized output costs a second search: start from the last count for this size
    cap = max(64, int(n * 64), _last_device_count.get(n, 0) * 9 // 8)
    while True:
        ei = torch.empty(2, cap, dtype=torch.int64, device=pos.device)
        sh = torch.empty(cap, 3, dtype=torch.int32, device=pos.device)
        cnt = lib.fc_neighbor_list_device(n, pos.data_ptr(), cell_np.ctypes.data, flags.ctypes.data, float(cutoff),
                                          cap, ei[0].data_ptr(), ei[1].data_ptr(), sh.data_ptr(), ws.data_ptr(),
                                          ws_bytes, _lib.stream_of(pos))
        if host_fallback_needed(cnt):
            # more pairs for one atom than the device list holds in LDS (1024), or a periodic
            # shift component >= 512: the host cell list builds the same pairs in the same order
            ei_h, sh_h = neighbor_pairs(pos.cpu().numpy(), cell_np, pbc, cutoff)
            return (torch.as_tensor(ei_h, device=pos.device),
                    torch.as_tensor(np.ascontiguousarray(sh_h), dtype=torch.int32, device=pos.device))
        if cnt < 0:
            _lib.check(-cnt, "fc_neighbor_list_device")
        _last_device_count[n] = int(cnt)
        if cnt <= cap:
            return ei[:, :cnt].contiguous(), sh[:cnt]
        cap = int(cnt) * 9 // 8


class NeighborList:
    """Pairs within ``r_max + skin`` (reference ``neighbors.py:10-117``).

    ``backend="device"`` builds the list on the GPU (``neighbor_pairs_device``) from
    positions given as a ROCm tensor and keeps ``edge_index`` / ``unit_shifts`` as device
    tensors; the pairs are those of the host backend."""

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
        for name in ("edge_index", "unit_shifts"):
            v = getattr(self, name)
            setattr(nl, name, None if v is None else (v.clone() if torch.is_tensor(v) else v.copy()))
        return nl

    def build(self, positions: np.ndarray, cell: np.ndarray, pbc: Union[bool, list]) -> "NeighborList":
        if self.backend == "device":
            self.edge_index, self.unit_shifts = neighbor_pairs_device(positions, cell, pbc, self.r_max + self.skin)
            return self
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
