"""MI355X-native FlashCart energy + forces path (HIP kernels behind a C ABI).

Subpackages mirror the reference's (``o3``, ``nn``, ``model``, ``calculators``, ``data``,
``utils``); :func:`alias_as_flashcart` lets code written against ``import flashcart`` run
on this package unchanged.
"""

import importlib
import sys

_SUBMODULES = ("o3", "o3.utils", "nn", "model", "calculators", "calculators.lammps_mliap", "data", "utils",
               "utils.lammps")


def alias_as_flashcart() -> None:
    """Register this package and its subpackages under the reference's module names
    (``flashcart``, ``flashcart.o3``, ``flashcart.nn``, ``flashcart.model``,
    ``flashcart.calculators``, ``flashcart.data``, ``flashcart.utils``, ...), so that
    ``import flashcart.o3`` and ``from flashcart.model import FlashCartPotential`` resolve
    here. Call it before the first ``import flashcart``; an already imported ``flashcart``
    (the reference itself) is left alone."""
    if "flashcart" in sys.modules and sys.modules["flashcart"] is not sys.modules[__name__]:
        raise RuntimeError("a different `flashcart` package is already imported; alias before importing it.")
    sys.modules["flashcart"] = sys.modules[__name__]
    for name in _SUBMODULES:
        sys.modules[f"flashcart.{name}"] = importlib.import_module(f"{__name__}.{name}")
