"""Ghost-atom feature exchange through the LAMMPS ML-IAP data object
(reference src/flashcart/utils/lammps.py).

With domain decomposition, every rank evaluates its owned atoms plus ghost copies of
atoms owned by neighbouring ranks. Before each interaction layer after the first, the
ghost rows of the node features must be refreshed from their owners, and during
differentiation the ghost-row gradients must be added back to the owners. LAMMPS
(KOKKOS ML-IAP) performs both transfers through ``data.forward_exchange(src, dst,
width)`` and ``data.reverse_exchange(src, dst, width)``; this module wraps them as
autograd-aware custom operators whose backward is the opposite transfer.

The exchange calls run outside the HIP library (LAMMPS owns the communication). The
op names are the reference's (``flashcart::lammps_forward_exchange`` /
``flashcart::lammps_reverse_exchange``).
"""

from __future__ import annotations

from contextlib import contextmanager
from typing import Any, Iterator, Optional

import torch

_LAMMPS_DATA: Optional[Any] = None


@contextmanager
def lammps_data_slot(lammps_data: Any) -> Iterator[None]:
    """Make ``lammps_data`` the process-wide exchange object for the enclosed evaluation
    (forward and backward must both run inside). The previous object is restored on exit."""
    global _LAMMPS_DATA
    previous = _LAMMPS_DATA
    _LAMMPS_DATA = lammps_data
    try:
        yield
    finally:
        _LAMMPS_DATA = previous


def _active_data() -> Any:
    data = _LAMMPS_DATA
    if data is None or not hasattr(data, "forward_exchange") or not hasattr(data, "reverse_exchange"):
        raise RuntimeError(
            "LAMMPS ghost exchange requires an ML-IAP data object with forward_exchange/reverse_exchange. "
            "Evaluate the model inside flashcart_amd.utils.lammps.lammps_data_slot(data).")
    return data


def _sync(t: torch.Tensor) -> None:
    # LAMMPS launches on its own stream: order our work before and after its copies.
    if t.is_cuda and torch.cuda.current_stream(t.device) != torch.cuda.default_stream(t.device):
        torch.cuda.synchronize(t.device)


def _exchange(t: torch.Tensor, forward: bool) -> torch.Tensor:
    data = _active_data()
    t = t.contiguous()
    out = torch.empty_like(t)
    _sync(t)
    (data.forward_exchange if forward else data.reverse_exchange)(t, out, t.shape[-1])
    _sync(t)
    return out


@torch.library.custom_op("flashcart::lammps_forward_exchange", mutates_args=())
def lammps_forward_exchange(feats: torch.Tensor) -> torch.Tensor:
    """(ntotal, C) features -> copy whose ghost rows hold their owners' features."""
    return _exchange(feats, True)


@torch.library.custom_op("flashcart::lammps_reverse_exchange", mutates_args=())
def lammps_reverse_exchange(grads: torch.Tensor) -> torch.Tensor:
    """(ntotal, C) gradients -> copy with ghost rows added to their owners and zeroed."""
    return _exchange(grads, False)


@lammps_forward_exchange.register_fake
def _(feats):
    return feats.new_empty(feats.shape)


@lammps_reverse_exchange.register_fake
def _(grads):
    return grads.new_empty(grads.shape)


lammps_forward_exchange.register_autograd(lambda ctx, g: lammps_reverse_exchange(g))
lammps_reverse_exchange.register_autograd(lambda ctx, g: lammps_forward_exchange(g))


def lammps_exchange_features(feats: torch.Tensor, nlocal: int, ntotal: int) -> torch.Tensor:
    """Pad owned features (nlocal, C) with zero ghost rows to (ntotal, C) and fill the
    ghost rows from their owners (reference utils/lammps.py:159-196)."""
    if feats.shape[0] == nlocal and ntotal > nlocal:
        feats = torch.cat([feats, feats.new_zeros((ntotal - nlocal, *feats.shape[1:]))], dim=0)
    elif feats.shape[0] != ntotal:
        raise RuntimeError(f"LAMMPS feature exchange expected {nlocal} or {ntotal} rows, got {feats.shape[0]}.")
    return lammps_forward_exchange(feats)
