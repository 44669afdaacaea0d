"""Rank-4 kernels (the library built with FLASHCART_KERNEL_L_MAX=4) against the oracle.

The reference generates kernels for any FLASHCART_KERNEL_L_MAX and tests rank 4 only when the
variable is set (tests/o3/test_tensor_product.py:76-77, tests/o3/test_linear.py:31 of the
reference). Here the variable selects libflashcart_hip_l4.so at import, so the checks run in a
process of their own with it set (tests/rank4_checks.py); skipped when that library has not been
built (``FLASHCART_KERNEL_L_MAX=4 python -m flashcart_amd.build``).
"""

import os
import subprocess
import sys

import pytest

from flashcart_amd import _lib

pytestmark = pytest.mark.gpu
ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


@pytest.mark.skipif(not os.path.exists(_lib.library_path(4)),
                    reason="libflashcart_hip_l4.so not built (FLASHCART_KERNEL_L_MAX=4 python -m flashcart_amd.build)")
def test_rank4_kernels_against_oracle():
    env = dict(os.environ, FLASHCART_KERNEL_L_MAX="4")
    res = subprocess.run([sys.executable, "-u", os.path.join(ROOT, "tests", "rank4_checks.py")], env=env,
                         capture_output=True, text=True, timeout=900, cwd=ROOT)
    print(res.stdout[-4000:])
    assert res.returncode == 0, res.stdout[-3000:] + res.stderr[-3000:]
    assert "all rank-4 checks passed" in res.stdout
