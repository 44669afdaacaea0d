"""Network layers: radial basis/cutoff, interaction, product, gates, norms, readout."""

from flashcart_amd.nn.radial import BesselBasis, ChebyshevBasis, PolynomialCutoff
from flashcart_amd.nn.layers import (
    EnergyReadoutLayer,
    EquivariantGatedLayer,
    InteractionLayer,
    LinearLayer,
    ProductLayer,
    RescaledSiLULayer,
    RMSLayerNorm,
    ScaleShiftEnergyLayer,
)

__all__ = [
    "BesselBasis",
    "ChebyshevBasis",
    "PolynomialCutoff",
    "EnergyReadoutLayer",
    "EquivariantGatedLayer",
    "InteractionLayer",
    "LinearLayer",
    "ProductLayer",
    "RescaledSiLULayer",
    "RMSLayerNorm",
    "ScaleShiftEnergyLayer",
]
