"""The bench configuration at its full size (25,000-atom fcc alloy, C=128, L_max=3), checked
through properties that hold at any size (the float64 oracle is too slow for it; the same
model is checked against the oracle on small cells in tests/test_gpu_model.py):

* translation invariance: forces sum to zero;
* rotation equivariance: a quarter turn about z (and a general rotation) rotates the forces
  and keeps the energy;
* periodic images: the 2x1x1 supercell has twice the energy and the same force on every
  image of an atom.

The positions sit on a 2^-10 A grid and the lattice constant is 29/8 A, so positions, their
quarter-turn images and the supercell's images are exact in float32 and every edge vector
is the same number in both evaluations; the comparisons then see only the kernels'
summation order. A general rotation also changes the float32 rounding of the positions
(7.6e-6 A at |x| > 64 A); with force constants of tens of eV/A^2 that alone moves forces
by a few 1e-4 eV/A, so that case is held to 1e-3 eV/A.

Bars: energies 1e-5 relative, forces 1e-4 eV/A absolute (the north star's).
"""

import numpy as np
import pytest
import torch

from flashcart_amd.data import AtomicGraph
from flashcart_amd.data.synthetic import fcc_alloy, model_config
from tests.helpers import assert_close

pytestmark = pytest.mark.gpu
DEV = "cuda"
ELEMENTS = ["Cu", "Ni", "Fe", "Cr"]
N = 25_000


@pytest.fixture(scope="module")
def system():
    from tests.test_gpu_model import _model
    z, pos, cell, pbc = fcc_alloy(25, 25, 10, a=3.625, jitter=0.05, seed=0)
    pos = np.round(pos * 1024.0) / 1024.0
    model = _model(model_config(ELEMENTS, 128, 3, avg_neighbors=43.6), seed=1234).to(DEV)
    model.requires_grad_(False)
    e0, f0 = _predict(model, z, pos, cell, pbc)
    return model, z, pos, cell, pbc, e0, f0


def _predict(model, z, pos, cell, pbc):
    g = AtomicGraph.from_arrays(z, pos, ELEMENTS, 5.0, cell=cell, pbc=pbc)
    out = model.predict(g.to(DEV), compute_forces=True)
    return float(out["energy"].double().sum()), out["forces"].double().cpu()


def test_forces_sum_to_zero(system):
    *_, e0, f0 = system
    assert np.isfinite(e0) and f0.shape == (N, 3)
    # each component is a sum of 25,000 float32 forces of order 1 eV/A
    assert float(f0.sum(0).abs().max()) < 2e-3, f"net force {f0.sum(0).tolist()}"


def test_quarter_turn(system):
    model, z, pos, cell, pbc, e0, f0 = system
    rot = np.array([[0.0, -1.0, 0.0], [1.0, 0.0, 0.0], [0.0, 0.0, 1.0]])
    e1, f1 = _predict(model, z, pos @ rot.T, cell @ rot.T, pbc)
    assert abs(e1 - e0) <= 1e-5 * abs(e0), f"energy {e1} vs {e0}"
    assert_close(f1, f0 @ torch.as_tensor(rot.T), 0.0, 1e-4, "quarter-turn forces")


def test_general_rotation(system):
    model, z, pos, cell, pbc, e0, f0 = system
    q, _ = np.linalg.qr(np.random.default_rng(3).standard_normal((3, 3)))
    rot = q * np.sign(np.linalg.det(q))  # proper rotation
    e1, f1 = _predict(model, z, pos @ rot.T, cell @ rot.T, pbc)
    assert abs(e1 - e0) <= 1e-5 * abs(e0), f"energy {e1} vs {e0}"
    assert_close(f1, f0 @ torch.as_tensor(rot.T), 0.0, 1e-3, "rotated forces")


def test_supercell_images(system):
    model, z, pos, cell, pbc, e0, f0 = system
    cell2 = cell.copy()
    cell2[0] *= 2
    e2, f2 = _predict(model, np.concatenate([z, z]), np.concatenate([pos, pos + cell[0]]), cell2, pbc)
    assert abs(e2 - 2 * e0) <= 1e-5 * abs(2 * e0), f"supercell energy {e2} vs 2 x {e0}"
    assert_close(f2[:N], f0, 0.0, 1e-4, "supercell forces (first image)")
    assert_close(f2[N:], f0, 0.0, 1e-4, "supercell forces (second image)")
