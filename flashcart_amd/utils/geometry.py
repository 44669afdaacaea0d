"""Edge-vector helpers (reference src/flashcart/utils/geometry.py)."""

from typing import Union

import numpy as np
import torch


def uses_periodic_shifts(pbc: object) -> bool:
    """True when any periodic flag is set, or when the flags are unavailable (reference ``geometry.py:7-22``)."""
    if torch.is_tensor(pbc):
        return bool(torch.any(pbc).item())
    if pbc is None:
        return True
    return bool(np.any(pbc))


def shift_vectors(cell: torch.Tensor, shifts: torch.Tensor, idx_i: torch.Tensor, batch: torch.Tensor,
                  antisymmetric: bool = False) -> torch.Tensor:
    """Cartesian periodic translation S . cell[batch[i]] of every edge (reference ``geometry.py:52``).

    One structure: a single (E,3) x (3,3) product; several: per-edge sums of the three
    scaled lattice vectors (a per-edge batched 1x3 @ 3x3 product is far slower).
    ``antisymmetric``: the per-edge sums also for one structure, each element evaluated as
    (s0 c0 + s1 c1) + s2 c2 with one rounding per operation, so the translation of -S is the
    exact negation of that of S (a library matrix product does not promise one summation
    order for all rows). The per-edge sums run as one kernel (``fc_shift_vectors``) for a
    float32 device cell that is not differentiated.
    """
    if cell.shape[0] == 1 and not antisymmetric:
        return shifts.to(cell.dtype) @ cell[0]
    if cell.is_cuda and cell.dtype == torch.float32 and not shifts.is_floating_point() and \
            not (torch.is_grad_enabled() and cell.requires_grad):
        from flashcart_amd.o3 import _ops
        return _ops.shift_vectors(cell, shifts, idx_i, batch)  # the expression below in one kernel
    s = shifts.to(cell.dtype)
    c = cell[0].unsqueeze(0) if cell.shape[0] == 1 else cell[batch[idx_i]]
    return s[:, 0:1] * c[:, 0] + s[:, 1:2] * c[:, 1] + s[:, 2:3] * c[:, 2]


def get_edge_vectors(positions, cell, shifts, edge_index, batch, use_shifts: bool = True) -> torch.Tensor:
    """pos[j] - pos[i] (+ S . cell) with plain tensor ops (reference ``geometry.py:25-53``).

    The model itself evaluates edge vectors inside the fused edge-geometry kernel;
    this helper is kept for callers of the reference utility.
    """
    idx_i, idx_j = edge_index[0], edge_index[1]
    if not use_shifts:
        return positions[idx_j] - positions[idx_i]
    return positions[idx_j] - positions[idx_i] + shift_vectors(cell, shifts, idx_i, batch)


def to_voigt6(t: Union[np.ndarray, torch.Tensor]):
    """Symmetrised Voigt order xx, yy, zz, yz, xz, xy (reference ``geometry.py:56-77``)."""
    comps = [t[..., 0, 0], t[..., 1, 1], t[..., 2, 2], (t[..., 1, 2] + t[..., 2, 1]) / 2,
             (t[..., 0, 2] + t[..., 2, 0]) / 2, (t[..., 0, 1] + t[..., 1, 0]) / 2]
    if isinstance(t, torch.Tensor):
        return torch.stack(comps, dim=-1)
    return np.stack(comps, axis=-1)
