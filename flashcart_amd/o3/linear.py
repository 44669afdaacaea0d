"""Equivariant linear maps (reference src/flashcart/o3/linear.py, src/flashcart/o3/_linear.py)."""

from typing import Optional, Sequence

import torch
import torch.nn as nn

from flashcart_amd.o3 import _ops
from flashcart_amd.o3.kernel_config import KERNEL_L_MAX
from flashcart_amd.o3.utils import get_irreps_slices


def make_linear_metadata(device, in_l_max: int, out_l_max: int, in_features: int, out_features: int,
                         in_paths: Sequence[int], weight_scale: Optional[float]):
    """Per-rank metadata and scales (reference ``o3/_linear.py:113-166``).

    Rows: (input offset, output offset, packed-weight offset, components, input
    channels incl. paths, output channels) for every rank shared by input and output.
    Default scale at rank l: (in_features * in_paths[l]) ** -0.5.
    """
    common = min(in_l_max, out_l_max)
    paths = list(in_paths)
    in_sl = get_irreps_slices(in_l_max, in_features, paths)
    out_sl = get_irreps_slices(out_l_max, out_features, [1] * (out_l_max + 1))
    if weight_scale is not None:
        scales = [float(weight_scale)] * (common + 1)
    else:
        scales = [float(in_features * paths[l]) ** -0.5 for l in range(common + 1)]
    meta, woff = [], 0
    for l in range(common + 1):
        f_in = in_features * paths[l]
        meta.append([in_sl[l][0], out_sl[l][0], woff, 2 * l + 1, f_in, out_features])
        woff += f_in * out_features
    out_size = sum((2 * l + 1) * out_features for l in range(out_l_max + 1))
    return (torch.tensor(meta, dtype=torch.int64, device=device), torch.tensor(scales, device=device), woff,
            out_size)


class LinearLayer(nn.Module):
    """Per-rank channel (and path) mixing ``out_l = x_l @ (W_l * s_l)^T``.

    Same constructor, parameters (``weight`` ParameterList of (out_features,
    in_features * in_paths[l]) matrices, N(0,1) init) and buffers as the reference
    (``src/flashcart/o3/linear.py:11-128``), so reference state dicts load unchanged.
    Evaluation runs the MFMA GEMM of the HIP library.
    """

    def __init__(self, in_l_max: int, out_l_max: int, in_features: int, out_features: int,
                 in_paths: Optional[Sequence[int]] = None, weight_scale: Optional[float] = None,
                 use_triton: bool = False):
        super().__init__()
        if max(in_l_max, out_l_max) > KERNEL_L_MAX:
            raise NotImplementedError(f"LinearLayer supports ranks <= {KERNEL_L_MAX}.")
        self.in_l_max = in_l_max
        self.out_l_max = out_l_max
        self.in_features = in_features
        self.out_features = out_features
        self.in_paths = [1] * (in_l_max + 1) if in_paths is None else [int(p) for p in in_paths]
        self.weight_scale = weight_scale
        self.use_triton = use_triton
        if len(self.in_paths) != in_l_max + 1:
            raise ValueError(f"Expected {in_l_max + 1} in_paths, got {len(self.in_paths)}.")
        self.common_l_max = min(in_l_max, out_l_max)
        self.in_dim = sum((2 * l + 1) * in_features * self.in_paths[l] for l in range(in_l_max + 1))
        self.out_dim = sum((2 * l + 1) * out_features for l in range(out_l_max + 1))
        meta, scale, n_weight, out_size = make_linear_metadata(torch.device("cpu"), in_l_max, out_l_max,
                                                               in_features, out_features, self.in_paths,
                                                               weight_scale)
        rows = [[int(v) for v in r] for r in meta.tolist()]
        self.meta_lists = tuple([r[i] for r in rows] for i in range(6))
        self.register_buffer("meta", meta, persistent=False)
        self.register_buffer("scale", scale, persistent=False)
        self._scale_list = [float(s) for s in scale.tolist()]
        self.n_weight = int(n_weight)
        if int(out_size) != self.out_dim:
            raise RuntimeError(f"Metadata out_size mismatch: {out_size} != {self.out_dim}.")
        self.weight = nn.ParameterList()
        for l in range(self.common_l_max + 1):
            self.weight.append(nn.Parameter(torch.randn(out_features, in_features * self.in_paths[l])))

    def forward(self, x: torch.Tensor, alpha: float = 1.0, residual: Optional[torch.Tensor] = None) -> torch.Tensor:
        """``residual`` (same shape as the output) is added in the GEMM epilogue."""
        if x.shape[-1] != self.in_dim:
            raise RuntimeError(f"Incorrect last dimension for x. Expected {self.in_dim}, got {x.shape[-1]}.")
        return _ops.linear_fwd(x, [_ops.param_alias(w) for w in self.weight], self.in_l_max, self.out_l_max,
                               self.in_features, self.out_features, self.in_paths, self._scale_list, float(alpha),
                               residual)

    def input_grad(self, grad_out: torch.Tensor, alpha: float = 1.0,
                   residual: Optional[torch.Tensor] = None) -> torch.Tensor:
        """Gradient of ``forward`` wrt its input (the MFMA dgrad, outside autograd), plus
        ``residual`` (a tensor of the input's shape) added in the GEMM epilogue."""
        return _ops.linear_bwd(grad_out, list(self.weight), self.in_l_max, self.out_l_max, self.in_features,
                               self.out_features, self.in_paths, self._scale_list, float(alpha), residual)

    def extra_repr(self) -> str:
        return (f"in_l_max={self.in_l_max}, out_l_max={self.out_l_max}, in_features={self.in_features}, "
                f"out_features={self.out_features}, in_paths={self.in_paths}, out_dim={self.out_dim}, "
                f"n_weights={self.n_weight}, use_triton={self.use_triton}")
