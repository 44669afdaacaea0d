from flashcart_amd.model.atomistic import AtomisticModel
from flashcart_amd.model.flashcart import FlashCartPotential

__all__ = ["AtomisticModel", "FlashCartPotential"]
