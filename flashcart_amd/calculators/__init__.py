"""Front-ends: ASE calculator and LAMMPS ML-IAP interface (reference src/flashcart/calculators)."""

from flashcart_amd.calculators.ase import FlashCartCalculator
from flashcart_amd.calculators.lammps_mliap import (
    FlashCartLAMMPSUnified,
    SingleRankMLIAPData,
    build_lammps_unified,
    graph_dict_from_mliap,
    save_lammps_unified,
)

__all__ = ["FlashCartCalculator", "FlashCartLAMMPSUnified", "SingleRankMLIAPData", "build_lammps_unified",
           "graph_dict_from_mliap", "save_lammps_unified"]
