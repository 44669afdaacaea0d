"""Radial bases and the polynomial cutoff (reference src/flashcart/nn/radial.py).

Buffers keep the reference names and values so state dicts load unchanged; the
evaluation is the HIP radial kernel (value and analytic derivative).
"""

import math
from typing import Literal

import torch
import torch.nn as nn

from flashcart_amd import _lib
from flashcart_amd.o3 import _ops


class BesselBasis(nn.Module):
    """sqrt(2/r_max) * sin(n pi r / r_max) / r, n = 1..n_radial (reference ``nn/radial.py:8-57``)."""

    def __init__(self, n_radial: int, r_max: float):
        super().__init__()
        if n_radial <= 0:
            raise ValueError(f"n_radial must be positive. Provided: {n_radial}.")
        if r_max <= 0.0:
            raise ValueError(f"r_max must be positive. Provided: {r_max}.")
        dtype = torch.get_default_dtype()
        self.n_radial = n_radial
        self._r_max = float(r_max)
        self.register_buffer("bessel_weights", (math.pi / r_max) * torch.arange(1, n_radial + 1, dtype=dtype))
        self.register_buffer("r_cutoff", torch.tensor(r_max, dtype=dtype))
        self.register_buffer("pre_factor", torch.tensor(math.sqrt(2.0 / r_max), dtype=dtype))

    def forward(self, distances: torch.Tensor) -> torch.Tensor:
        feats, _ = _ops.radial_fwd(distances, _lib.BASIS_BESSEL, self.n_radial, 0.0, self._r_max, 0)
        return feats

    def __repr__(self) -> str:
        return f"{self.__class__.__name__}(r_cutoff={self._r_max}, n_radial={self.n_radial})"


class ChebyshevBasis(nn.Module):
    """Chebyshev T_0..T_{n-1} of the mapped distance (reference ``nn/radial.py:60-129``)."""

    def __init__(self, n_radial: int, r_max: float, r_min: float = 0.0,
                 mapping: Literal["cosine", "affine"] = "affine"):
        super().__init__()
        if r_max <= r_min:
            raise ValueError(f"Expected r_max > r_min. Provided: r_min={r_min}, r_max={r_max}.")
        if mapping not in ("cosine", "affine"):
            raise ValueError(f"Expected mapping to be 'cosine' or 'affine'. Provided: {mapping}.")
        if n_radial > 32:
            raise ValueError("The HIP radial kernel supports at most 32 basis functions.")
        dtype = torch.get_default_dtype()
        self.n_radial = n_radial
        self.mapping = mapping
        self._r_min, self._r_max = float(r_min), float(r_max)
        self.register_buffer("r_min", torch.tensor(r_min, dtype=dtype))
        self.register_buffer("r_max", torch.tensor(r_max, dtype=dtype))

    @property
    def basis_kind(self) -> int:
        return _lib.BASIS_CHEBYSHEV_COSINE if self.mapping == "cosine" else _lib.BASIS_CHEBYSHEV_AFFINE

    def forward(self, distances: torch.Tensor) -> torch.Tensor:
        feats, _ = _ops.radial_fwd(distances, self.basis_kind, self.n_radial, self._r_min, self._r_max, 0)
        return feats

    def __repr__(self) -> str:
        return (f"{self.__class__.__name__}(n_radial={self.n_radial}, r_min={self._r_min:.4g}, "
                f"r_max={self._r_max:.4g}, mapping={self.mapping})")


class PolynomialCutoff(nn.Module):
    """1 - c1 t^p + c2 t^(p+1) - c3 t^(p+2), t = r / r_max, zero beyond r_max (reference ``nn/radial.py:132-245``)."""

    def __init__(self, r_max: float, poly_order: int = 6):
        super().__init__()
        if poly_order < 2:
            raise ValueError(f"Polynomial order must be >= 2. Provided: {poly_order}.")
        dtype = torch.get_default_dtype()
        self.poly_order_value = int(poly_order)
        self._r_max = float(r_max)
        self.register_buffer("poly_order", torch.tensor(poly_order, dtype=torch.long))
        self.register_buffer("r_max", torch.tensor(r_max, dtype=dtype))
        self.register_buffer("coeff1", torch.tensor((poly_order + 1.0) * (poly_order + 2.0) / 2.0, dtype=dtype))
        self.register_buffer("coeff2", torch.tensor(poly_order * (poly_order + 2.0), dtype=dtype))
        self.register_buffer("coeff3", torch.tensor(poly_order * (poly_order + 1.0) / 2.0, dtype=dtype))

    def forward(self, distances: torch.Tensor) -> torch.Tensor:
        _, env = _ops.radial_fwd(distances, _lib.BASIS_NONE, 1, 0.0, self._r_max, self.poly_order_value)
        return env

    @staticmethod
    def calculate_envelope(distances: torch.Tensor, r_max, poly_order: int, coeff1=None, coeff2=None,
                           coeff3=None) -> torch.Tensor:
        """Envelope without a module instance (coefficients are implied by ``poly_order``)."""
        _, env = _ops.radial_fwd(distances, _lib.BASIS_NONE, 1, 0.0, float(r_max), int(poly_order))
        return env

    def __repr__(self) -> str:
        return f"{self.__class__.__name__}(r_max={self._r_max:.4g}, poly_order={self.poly_order_value})"
