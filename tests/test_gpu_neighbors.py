"""Device neighbour list (``fc_neighbor_list_device``) against the host list.

The host list is pinned by brute force and the reference's count known answers
(tests/test_host.py); the device list must return the identical pairs in the identical
order (bit-exact index work): same edge_index, same integer shifts.
"""

import numpy as np
import pytest
import torch

from flashcart_amd.data.neighbors import NeighborList, neighbor_pairs, neighbor_pairs_device
from flashcart_amd.data.synthetic import fcc_alloy, molecules, water_box
from oracle.neighbors import brute_force_pairs

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _same(pos, cell, pbc, cutoff, what):
    """Device list == host list, and on systems small enough for it == the brute-force oracle
    (the edge-set contract of the reference, in canonical (i, j, S) order)."""
    ei_h, sh_h = neighbor_pairs(pos, cell, pbc, cutoff)
    ei_d, sh_d = neighbor_pairs_device(torch.as_tensor(np.asarray(pos, dtype=np.float64), device=DEV), cell, pbc,
                                       cutoff)
    assert ei_d.dtype == torch.int64 and sh_d.dtype == torch.int32
    assert ei_d.shape == (2, ei_h.shape[1]), f"{what}: {ei_d.shape[1]} pairs on the device, {ei_h.shape[1]} on the host"
    assert np.array_equal(ei_d.cpu().numpy(), ei_h), f"{what}: edge_index differs"
    assert np.array_equal(sh_d.cpu().numpy(), sh_h), f"{what}: shifts differ"
    if len(pos) <= 2000 and np.any(pbc) and abs(np.linalg.det(np.asarray(cell, dtype=float))) > 1e-7 \
            or not np.any(pbc):
        got = [tuple(int(v) for v in row) for row in
               np.concatenate([ei_d.cpu().numpy().T, sh_d.cpu().numpy().astype(np.int64)], axis=1)]
        assert got == brute_force_pairs(pos, cell, pbc, cutoff), f"{what}: differs from the brute-force oracle"
    return ei_h.shape[1]


@pytest.mark.parametrize("cells,cutoff", [((4, 4, 4), 5.0), ((3, 3, 3), 6.0), ((6, 5, 4), 5.0)])
def test_fcc_periodic(cells, cutoff):
    z, pos, cell, pbc = fcc_alloy(*cells, seed=sum(cells))
    assert _same(pos, cell, pbc, cutoff, f"fcc {cells}") > 0


def test_water_box():
    z, pos, cell, pbc = water_box(64, seed=3)
    _same(pos, cell, pbc, 5.0, "water")


def test_triclinic_unwrapped():
    """Skewed cell, positions outside the cell (negative and beyond one period)."""
    rng = np.random.default_rng(4)
    cell = np.array([[7.0, 0.0, 0.0], [2.5, 6.5, 0.0], [-1.5, 1.0, 8.0]])
    frac = rng.uniform(-1.3, 2.2, size=(90, 3))
    _same(frac @ cell, cell, True, 4.5, "triclinic")


def test_small_cell_many_images():
    """Cell thinner than the cutoff along every axis: several images per pair."""
    cell = np.array([[2.2, 0.0, 0.0], [0.4, 2.6, 0.0], [0.0, 0.3, 3.1]])
    pos = np.array([[0.1, 0.2, 0.3], [1.2, 1.5, 1.9], [2.0, 0.5, 2.8]])
    _same(pos, cell, True, 5.5, "small cell")


def test_open_and_mixed_boundaries():
    for k, (zz, pp) in enumerate(molecules(3, 6, 20, seed=7)):
        _same(pp, np.zeros((3, 3)), False, 5.0, f"molecule {k}")
    z, pos, cell, _ = fcc_alloy(4, 4, 3, seed=5)
    pos = pos + np.array([0.0, 0.0, 3.0])
    _same(pos, cell, [True, True, False], 5.0, "slab")
    _same(pos, cell, [False, True, False], 5.0, "wire")


def test_md_steps_and_backend():
    """Perturbed positions over several steps, built from device positions through
    NeighborList(backend="device")."""
    z, pos, cell, pbc = fcc_alloy(5, 5, 5, seed=1)
    rng = np.random.default_rng(2)
    for step in range(3):
        pos = pos + rng.normal(scale=0.05, size=pos.shape)
        nl = NeighborList(5.0, skin=0.5, backend="device").build(torch.as_tensor(pos, device=DEV), cell, pbc)
        ref = NeighborList(5.0, skin=0.5).build(pos, cell, pbc)
        assert np.array_equal(nl.edge_index.cpu().numpy(), ref.edge_index), f"step {step}"
        assert np.array_equal(nl.unit_shifts.cpu().numpy(), ref.unit_shifts), f"step {step}"
        assert torch.equal(nl.copy().edge_index, nl.edge_index)


def test_cfg4_size():
    z, pos, cell, pbc = fcc_alloy(25, 25, 10, a=3.6, jitter=0.05, seed=0)
    n_pairs = _same(pos, cell, pbc, 6.0, "fcc 25k, r_max + skin")
    assert n_pairs > 25_000 * 70


def test_dense_atoms_fall_back_to_the_host_list():
    """More than 1,024 pairs per atom (fcc within 15 A: about 1,200): the device list reports
    its size limit and neighbor_pairs_device returns the host list's pairs instead."""
    z, pos, cell, pbc = fcc_alloy(9, 9, 9, seed=8)
    n = _same(pos, cell, pbc, 15.0, "fcc, 15 A cutoff")
    assert n > 1100 * len(pos)


def test_empty_and_single_atom():
    ei, sh = neighbor_pairs_device(torch.zeros(0, 3, dtype=torch.float64, device=DEV), np.eye(3) * 5, True, 3.0)
    assert ei.shape == (2, 0) and sh.shape == (0, 3)
    _same(np.array([[0.5, 0.5, 0.5]]), np.eye(3) * 2.0, True, 4.5, "one atom, its own images")
