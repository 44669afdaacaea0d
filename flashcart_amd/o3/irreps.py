"""Expand direction vectors into irreducible Cartesian tensors (reference src/flashcart/o3/irreps.py)."""

import torch
import torch.nn as nn

from flashcart_amd.o3 import _ops
from flashcart_amd.o3.kernel_config import KERNEL_L_MAX


class Irreps(nn.Module):
    """Eq. (1) components of ranks 0..l_max, ``(l_max + 1) ** 2`` per vector.

    Same constructor and methods as the reference module (reference
    ``src/flashcart/o3/irreps.py:9-80``). ``use_triton`` is kept for configuration and
    checkpoint compatibility; evaluation always runs the HIP kernel, which requires a
    float32 ROCm tensor.
    """

    def __init__(self, l_max: int, use_triton: bool = False):
        super().__init__()
        if l_max > KERNEL_L_MAX:
            raise RuntimeError(
                f"Irreps supports l_max <= {KERNEL_L_MAX}, got {l_max=} (the rank compiled into the HIP kernels)."
            )
        self.l_max = l_max
        self.use_triton = use_triton

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        x = torch.nn.functional.normalize(x, dim=-1)
        return self.forward_normalized(x)

    def forward_normalized(self, x: torch.Tensor) -> torch.Tensor:
        r2 = x.pow(2).sum(dim=-1)
        torch._assert_async(((r2 - 1.0).abs() <= 1.0e-5).all(),
                            "Irreps.forward_normalized requires unit-length input vectors.")
        return _ops.irreps_fwd(x, self.l_max)

    def __repr__(self):
        return (f"{self.__class__.__name__}(l_max={self.l_max}, use_triton={self.use_triton}, "
                f"output_dim={(self.l_max + 1) ** 2})")
