"""Maximal tensor rank of the HIP kernels in use.

The reference reads ``FLASHCART_KERNEL_L_MAX`` before generating its kernels at import
(src/flashcart/o3/kernel_config.py:10-24, default 3). Here the kernels are generated and
compiled ahead of time: ``libflashcart_hip.so`` for ranks 0..3 and, when built with
``FLASHCART_KERNEL_L_MAX=4 python -m flashcart_amd.build``, ``libflashcart_hip_l4.so`` for
ranks 0..4. The variable, read at import as in the reference, selects the library
(``flashcart_amd._lib.library_path``) and the limit the modules check (``NotImplementedError``
above it, as the reference's generated kernels raise).
"""
import os

COMPILED_L_MAX = 4  # the highest rank any build of the library supports
DEFAULT_L_MAX = 3
_ENV = "FLASHCART_KERNEL_L_MAX"


def kernel_l_max() -> int:
    v = os.environ.get(_ENV)
    if v is None:
        return DEFAULT_L_MAX
    v = int(v)
    if v < 0:
        raise RuntimeError(f"{_ENV} must be non-negative, got {v}.")
    if v > COMPILED_L_MAX:
        raise RuntimeError(
            f"{_ENV}={v} exceeds the highest rank the HIP kernels can be built for ({COMPILED_L_MAX})."
        )
    return v


KERNEL_L_MAX: int = kernel_l_max()
