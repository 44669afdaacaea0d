"""Receiver-sorted graph metadata (CSR) shared by every convolution op of one forward.

The reference recomputes ``rowptr`` with ``searchsorted`` inside each tensor-product
launch (src/flashcart/o3/_tensor_product.py:396-405) and scatters sender gradients
with atomics. Here the receiver CSR and a stable sender ordering are computed once
per neighbour list on the GPU and reused by the forward and backward of every layer,
so sender-side reductions are segmented sums in a fixed order.
"""

from __future__ import annotations

from dataclasses import dataclass
from typing import Optional

import torch

from flashcart_amd import _lib


@dataclass
class GraphCSR:
    n_nodes: int           # receiver rows
    n_sender_rows: int     # rows of the sender features (>= n_nodes with ghosts)
    idx_i: torch.Tensor    # int32 (E,) receivers, sorted
    idx_j: torch.Tensor    # int32 (E,) senders
    rowptr: torch.Tensor   # int32 (n_nodes + 1,)
    sender_perm: torch.Tensor  # int32 (E,) edges ordered by sender (stable)
    sender_ptr: torch.Tensor   # int32 (n_sender_rows + 1,)

    @property
    def n_edges(self) -> int:
        return int(self.idx_i.shape[0])

    def struct(self) -> "_lib.CSR":
        return _lib.csr_struct(self.n_nodes, self.n_edges, self.idx_j, self.rowptr, self.sender_perm,
                               self.sender_ptr, self.n_sender_rows)


def rowptr_from_sorted(idx_sorted: torch.Tensor, n_rows: int) -> torch.Tensor:
    """lower_bound CSR of a sorted int32 index vector, computed by the HIP library."""
    _lib.require_device("idx", idx_sorted, torch.int32)
    out = torch.empty(n_rows + 1, dtype=torch.int32, device=idx_sorted.device)
    lib = _lib.load()
    _lib.check(lib.fc_csr_from_sorted(idx_sorted.shape[0], idx_sorted.data_ptr(), n_rows, out.data_ptr(),
                                      _lib.stream_of(idx_sorted)), "fc_csr_from_sorted")
    return out


def build_graph(edge_index: torch.Tensor, n_nodes: int, n_sender_rows: Optional[int] = None,
                check_sorted: bool = True) -> GraphCSR:
    """Build the CSR metadata of a receiver-sorted edge list ``edge_index = [idx_i; idx_j]``."""
    if edge_index.dim() != 2 or edge_index.shape[0] != 2:
        raise ValueError(f"edge_index must have shape (2, E), got {tuple(edge_index.shape)}.")
    if not edge_index.is_cuda:
        raise RuntimeError("flashcart_amd graphs live on the GPU; move edge_index to a ROCm device.")
    n_send = int(n_nodes if n_sender_rows is None else n_sender_rows)
    idx_i = edge_index[0].to(torch.int32).contiguous()
    idx_j = edge_index[1].to(torch.int32).contiguous()
    if check_sorted and idx_i.numel() > 1:
        torch._assert_async((idx_i[1:] >= idx_i[:-1]).all(), "edge_index[0] (receivers) must be sorted.")
    rowptr = rowptr_from_sorted(idx_i, n_nodes)
    sender_perm = torch.argsort(idx_j, stable=True).to(torch.int32)
    sender_ptr = rowptr_from_sorted(idx_j[sender_perm.long()].contiguous(), n_send)
    return GraphCSR(int(n_nodes), n_send, idx_i, idx_j, rowptr, sender_perm, sender_ptr)
