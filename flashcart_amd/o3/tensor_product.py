"""Weighted irreducible Cartesian tensor products (reference src/flashcart/o3/tensor_product.py)."""

from typing import Optional

import torch
import torch.nn as nn

from flashcart_amd.o3 import _ops
from flashcart_amd.o3._graph import GraphCSR
from flashcart_amd.o3.kernel_config import KERNEL_L_MAX
from flashcart_amd.o3.utils import count_output_paths, get_irreps_slices


class TensorProduct(nn.Module):
    """Weighted products of irreducible Cartesian tensor features.

    Constructor, attributes (``in1_dim``, ``in2_dim``, ``in1_slices``, ``in2_slices``,
    ``out_paths``, ``n_total_paths``) and ``forward`` semantics follow the reference
    (``src/flashcart/o3/tensor_product.py:12-172``): one path per allowed
    (l1, l2) -> l_out coupling, per-path per-feature weights, optional path reduction,
    and a convolution mode when ``idx_i``/``idx_j`` are given (in1 gathered from the
    senders, summed at the sorted receivers). Evaluation runs the HIP kernels;
    ``use_triton`` is kept for configuration compatibility.

    ``forward`` additionally accepts ``graph`` (a :class:`GraphCSR` built once per
    neighbour list) so that the receiver CSR and sender ordering are not rebuilt by
    every call, ``alpha``, a scale folded into the kernel output, and ``alpha_div``, a
    one-element device tensor the output is divided by on the device.
    """

    def __init__(self, in1_l_max: int, in2_l_max: int, out_l_max: int, in1_features: int, in2_features: int,
                 symmetric_product: bool = False, use_triton: bool = False, shared_weights: bool = False,
                 reduce_paths: bool = False):
        super().__init__()
        if not (in1_features == in2_features or in1_features == 1 or in2_features == 1):
            raise ValueError("Input dimensions must match unless one of them is 1. "
                             f"Provided: {in1_features=} and {in2_features=}.")
        if max(in1_l_max, in2_l_max, out_l_max) > KERNEL_L_MAX:
            raise NotImplementedError(
                f"TensorProduct supports ranks <= {KERNEL_L_MAX}; got in1_l_max={in1_l_max}, "
                f"in2_l_max={in2_l_max}, out_l_max={out_l_max}.")
        if symmetric_product and (in1_l_max != in2_l_max or in1_features != in2_features):
            raise ValueError("symmetric_product requires identical input layouts.")
        self.in1_l_max = in1_l_max
        self.in2_l_max = in2_l_max
        self.out_l_max = out_l_max
        self.in1_features = in1_features
        self.in2_features = in2_features
        self.symmetric_product = symmetric_product
        self.use_triton = use_triton
        self.shared_weights = shared_weights
        self.reduce_paths = reduce_paths
        self.in1_dim = sum((2 * l + 1) * in1_features for l in range(in1_l_max + 1))
        self.in2_dim = sum((2 * l + 1) * in2_features for l in range(in2_l_max + 1))
        self.in1_slices = get_irreps_slices(in1_l_max, in1_features)
        self.in2_slices = get_irreps_slices(in2_l_max, in2_features)
        self.out_paths, self.n_total_paths = count_output_paths(in1_l_max, in2_l_max, out_l_max,
                                                                symmetric_product=symmetric_product)
        # (in1_offs, in2_offs, out_sizes, n_paths_per_l, n_total_paths) of the op schema
        self.op_meta = _ops.tp_meta(in1_l_max, in2_l_max, out_l_max, in1_features, in2_features,
                                    symmetric_product, reduce_paths)

    @property
    def out_features(self) -> int:
        return max(self.in1_features, self.in2_features)

    @property
    def out_dim(self) -> int:
        c = self.out_features
        return sum((2 * l + 1) * (min(n, 1) if self.reduce_paths else n) * c for l, n in enumerate(self.out_paths))

    def forward(self, in1: torch.Tensor, in2: torch.Tensor, weights: torch.Tensor,
                idx_i: Optional[torch.Tensor] = None, idx_j: Optional[torch.Tensor] = None,
                graph: Optional[GraphCSR] = None, alpha: float = 1.0,
                alpha_div: Optional[torch.Tensor] = None) -> torch.Tensor:
        if in1.shape[-1] != self.in1_dim:
            raise RuntimeError(f"Incorrect last dimension for in1. Expected {self.in1_dim}, got {in1.shape[-1]}.")
        if in2.shape[-1] != self.in2_dim:
            raise RuntimeError(f"Incorrect last dimension for in2. Expected {self.in2_dim}, got {in2.shape[-1]}.")
        if self.symmetric_product and in1 is not in2:
            torch._assert_async((in1 == in2).all(), "Symmetric product requires in1 == in2.")
        rowptr = sender_perm = sender_ptr = None
        if graph is not None:
            idx_i, idx_j = graph.idx_i, graph.idx_j
            rowptr, sender_perm, sender_ptr = graph.rowptr, graph.sender_perm, graph.sender_ptr
        elif (idx_i is None) != (idx_j is None):
            raise ValueError("idx_i and idx_j must be given together.")
        return _ops.tp_fwd(in1, in2, _ops.param_alias(weights), idx_i, idx_j, self.in1_l_max, self.in2_l_max,
                           self.out_l_max,
                           self.in1_features, self.in2_features, self.symmetric_product, self.shared_weights,
                           *self.op_meta, self.reduce_paths, rowptr, sender_perm, sender_ptr, float(alpha), None,
                           alpha_div)

    def __repr__(self) -> str:
        return (f"{self.__class__.__name__}({self.in1_l_max} x {self.in2_l_max} -> {self.out_l_max}, "
                f"in1_features={self.in1_features}, in2_features={self.in2_features}, "
                f"symmetric={self.symmetric_product}, use_triton={self.use_triton}, "
                f"paths={self.out_paths}, total_paths={self.n_total_paths}, reduce_paths={self.reduce_paths})")
