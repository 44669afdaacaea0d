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
class EdgePairs:
    """Edges (i <- j, S) and (j <- i, -S) of a full neighbour list.

    The radial MLP of an interaction layer reads only the edge length, which is bitwise the
    same for both edges of a pair when the shift vectors are exact negations of each other
    (``utils.geometry.shift_vectors(..., antisymmetric=True)``); the pair's weights are then
    formed once and read by both edges (``fc_csr.pair_slot``). No counterpart in the
    reference, which forms the weights of every edge (src/flashcart/nn/layers.py:357-364).
    """
    slot: torch.Tensor   # int32 (E,): 2p for the lower edge of pair p, 2p + 1 for its reverse
    edge: torch.Tensor   # int32 (P,): the lower edge of each pair, in edge order
    upper: torch.Tensor  # int32 (P,): the other edge of each pair
    reverse: torch.Tensor  # int32 (E,): the reverse of every edge

    @property
    def n_pairs(self) -> int:
        return int(self.edge.shape[0])


class GraphCSR:
    """Receiver CSR of an edge list and a sender order of its edges.

    n_nodes: receiver rows; n_sender_rows: rows of the sender features (>= n_nodes with ghosts);
    idx_i / idx_j: int32 (E,) receivers (sorted) and senders; rowptr: int32 (n_nodes + 1,).
    sender_perm / sender_ptr: the edges grouped by sender (int32 (E,)) and the group bounds
    (int32 (n_sender_rows + 1,)), formed on first use: with a complete edge pairing the edges sent
    by node n are the reverses of the edges it receives (``reverse[rowptr[n]:rowptr[n+1]]``, group
    bounds = rowptr), otherwise a stable sort of idx_j.
    """

    def __init__(self, n_nodes: int, n_sender_rows: int, idx_i: torch.Tensor, idx_j: torch.Tensor,
                 rowptr: torch.Tensor, sender_perm: Optional[torch.Tensor] = None,
                 sender_ptr: Optional[torch.Tensor] = None):
        self.n_nodes = int(n_nodes)
        self.n_sender_rows = int(n_sender_rows)
        self.idx_i, self.idx_j, self.rowptr = idx_i, idx_j, rowptr
        self._sender_perm, self._sender_ptr = sender_perm, sender_ptr

    @property
    def n_edges(self) -> int:
        return int(self.idx_i.shape[0])

    def _senders(self) -> None:
        if self._sender_perm is not None:
            return
        pairs = next((p for p in self.__dict__.get("_pairs", {}).values() if p is not None), None)
        if pairs is not None and self.n_sender_rows == self.n_nodes:
            self._sender_perm, self._sender_ptr = pairs.reverse, self.rowptr
            return
        self._sender_perm, self._sender_ptr = self.sort_senders()

    def sort_senders(self):
        """(sender_perm, sender_ptr) by a stable sort of idx_j, whatever the pairing."""
        perm = torch.argsort(self.idx_j, stable=True).to(torch.int32)
        return perm, rowptr_from_sorted(self.idx_j[perm.long()].contiguous(), self.n_sender_rows)

    def set_senders(self, sender_perm: torch.Tensor, sender_ptr: torch.Tensor) -> None:
        self._sender_perm, self._sender_ptr = sender_perm, sender_ptr

    @property
    def sender_perm(self) -> torch.Tensor:
        self._senders()
        return self._sender_perm

    @property
    def sender_ptr(self) -> torch.Tensor:
        self._senders()
        return self._sender_ptr

    def struct(self, senders: bool = True) -> "_lib.CSR":
        if not senders:
            return _lib.csr_struct(self.n_nodes, self.n_edges, self.idx_j, self.rowptr, None, None,
                                   self.n_sender_rows)
        return _lib.csr_struct(self.n_nodes, self.n_edges, self.idx_j, self.rowptr, self.sender_perm,
                               self.sender_ptr, self.n_sender_rows)

    def request_edge_pairs(self, shifts: Optional[torch.Tensor]):
        """Launch the pairing of this edge list for ``shifts`` without waiting for it (the host
        reads its counters in ``edge_pairs``, so work queued in between overlaps them). Returns
        the sender order a complete pairing gives, (reverse, rowptr), when the pairing is still
        pending (None when it is decided already or cannot apply): valid once ``edge_pairs``
        confirms the pairing."""
        cache = self.__dict__.setdefault("_pairs", {})
        key = _shift_key(shifts)
        pending = self.__dict__.setdefault("_pending", {})
        if key in cache:
            return None
        if key not in pending:
            if not pairable(self, shifts):
                cache.clear()
                cache[key] = None
                return None
            self._pending = pending = {key: launch_edge_pairs(self, shifts)}
        if self.n_sender_rows != self.n_nodes:
            return None
        return pending[key][0].reverse, self.rowptr

    def edge_pairs(self, shifts: Optional[torch.Tensor]) -> Optional[EdgePairs]:
        """The pairing of this edge list (cached per shift tensor), or None when some edge has no
        unique reverse (ghost senders, half lists, duplicate or unsorted edges)."""
        cache = self.__dict__.setdefault("_pairs", {})
        key = _shift_key(shifts)
        if key not in cache:
            self.request_edge_pairs(shifts)
            if key not in cache:
                pairs, counts = self._pending.pop(key)
                cache.clear()
                cache[key] = pairs if pairs_complete(counts, self.n_edges) else None
        return cache[key]

    def set_edge_pairs(self, shifts: Optional[torch.Tensor], pairs: Optional[EdgePairs]) -> None:
        """Record the pairing of this edge list for ``shifts`` (computed elsewhere, e.g. in a graph)."""
        self.__dict__["_pairs"] = {_shift_key(shifts): pairs}
        self.__dict__["_pending"] = {}


def _shift_key(shifts: Optional[torch.Tensor]):
    return None if shifts is None else (shifts.data_ptr(), tuple(shifts.shape), shifts._version)


def pairable(csr: GraphCSR, shifts: Optional[torch.Tensor]) -> bool:
    """Shapes and types under which ``fc_edge_pairs`` can pair the whole edge list."""
    n_edges = csr.n_edges
    if n_edges == 0 or n_edges % 2:
        return False
    return shifts is None or (not shifts.is_floating_point() and not shifts.is_complex()
                              and tuple(shifts.shape) == (n_edges, 3))


def launch_edge_pairs(csr: GraphCSR, shifts: Optional[torch.Tensor]):
    """Launch ``fc_edge_pairs`` without waiting for it (usable under HIP graph capture):
    returns the pairing and its device counters [unpaired edges, pairs]; the pairing is valid
    only when the counters read [0, E / 2] (``pairs_complete``)."""
    n_edges = csr.n_edges
    dev = csr.idx_i.device
    sh = None if shifts is None else shifts.to(device=dev, dtype=torch.int32).contiguous()
    lib = _lib.load()
    n_ws = int(lib.fc_edge_pairs_workspace(n_edges))
    if n_ws < 0:
        _lib.check(-n_ws, "fc_edge_pairs_workspace")
    slot = torch.empty(n_edges, dtype=torch.int32, device=dev)
    edge = torch.empty(n_edges // 2, dtype=torch.int32, device=dev)
    upper = torch.empty(n_edges // 2, dtype=torch.int32, device=dev)
    reverse = torch.empty(n_edges, dtype=torch.int32, device=dev)
    counts = torch.empty(2, dtype=torch.int32, device=dev)
    ws = torch.empty(max(n_ws, 1), dtype=torch.int32, device=dev)
    keep = csr.struct(senders=False)
    _lib.check(lib.fc_edge_pairs(keep, csr.idx_i.data_ptr(), _lib.ptr(sh), slot.data_ptr(), edge.data_ptr(),
                                 upper.data_ptr(), reverse.data_ptr(), n_edges // 2, counts.data_ptr(),
                                 ws.data_ptr(), n_ws, _lib.stream_of(csr.idx_i)),
               "fc_edge_pairs")
    if not torch.cuda.is_current_stream_capturing():
        # the counters travel to pinned host memory behind the pairing kernels; reading them
        # waits for that copy only, not for the work queued after it
        host = torch.empty(2, dtype=torch.int32, pin_memory=True)
        host.copy_(counts, non_blocking=True)
        done = torch.cuda.Event()
        done.record(torch.cuda.current_stream(dev))
        while len(_READBACK) >= 16:  # launches whose counters were never checked
            _READBACK.pop(next(iter(_READBACK)))
        _READBACK[counts.data_ptr()] = (counts, host, done)
    return EdgePairs(slot, edge, upper, reverse), counts


# device counters of launched pairings -> (counters, pinned host copy, event after the copy)
_READBACK = {}


def pairs_complete(counts: torch.Tensor, n_edges: int) -> bool:
    """Host check of ``launch_edge_pairs``'s counters: waits for the pinned copy queued behind
    the pairing when there is one (work queued after it keeps the GPU busy), else reads the
    device counters (a full synchronisation)."""
    pending = _READBACK.pop(counts.data_ptr(), None)
    if pending is not None and pending[0] is counts:
        pending[2].synchronize()
        values = pending[1].tolist()
    else:
        values = counts.tolist()
    unpaired, n_pairs = (int(v) for v in values)
    return unpaired == 0 and 2 * n_pairs == n_edges


def find_edge_pairs(csr: GraphCSR, shifts: Optional[torch.Tensor]) -> Optional[EdgePairs]:
    """Pair every edge with its reverse on the GPU (``fc_edge_pairs``); None unless all edges
    pair up. ``shifts``: integer cell translations (E, 3), or None without periodic shifts.
    Reads the two pair counters back to the host (one synchronisation)."""
    if not pairable(csr, shifts):
        return None
    pairs, counts = launch_edge_pairs(csr, shifts)
    return pairs if pairs_complete(counts, csr.n_edges) else None


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
    return GraphCSR(int(n_nodes), n_send, idx_i, idx_j, rowptr)
