"""Maximal tensor rank compiled into the HIP kernels.

The reference reads ``FLASHCART_KERNEL_L_MAX`` before generating its kernels at
import (src/flashcart/o3/kernel_config.py:10-24). Here the kernels are generated and
compiled ahead of time for ranks 0..3; the variable may lower the limit but cannot
raise it above what the library was built with.
"""
import os

COMPILED_L_MAX = 3
_ENV = "FLASHCART_KERNEL_L_MAX"


def kernel_l_max() -> int:
    v = os.environ.get(_ENV)
    if v is None:
        return COMPILED_L_MAX
    v = int(v)
    if v > COMPILED_L_MAX:
        raise RuntimeError(
            f"{_ENV}={v} exceeds the rank compiled into libflashcart_hip.so ({COMPILED_L_MAX}); "
            "regenerate the kernels with a higher limit to use it."
        )
    return v


KERNEL_L_MAX: int = kernel_l_max()
