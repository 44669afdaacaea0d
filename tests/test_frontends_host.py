"""Host-side logic of the front-ends (no GPU): ML-IAP graph construction, the ghost
exchange operators and the calculator's neighbour-list reuse rule."""

import numpy as np
import pytest
import torch

from flashcart_amd.data.synthetic import fcc_alloy, model_config


class _Data:
    def __init__(self):
        self.nlocal, self.ntotal, self.npairs = 2, 3, 3
        self.pair_i = np.array([0, 0, 1, 7], dtype=np.int32)  # one entry past npairs, ignored
        self.pair_j = np.array([1, 2, 0, 7], dtype=np.int32)
        self.rij = np.array([[1.0, 0, 0], [0, 1.0, 0], [-1.0, 0, 0], [9, 9, 9]])
        self.elems = np.array([1, 0, 1, 5], dtype=np.int32)


def test_graph_dict_from_mliap():
    from flashcart_amd.calculators.lammps_mliap import graph_dict_from_mliap
    g = graph_dict_from_mliap(_Data(), ["H", "O"], device="cpu", dtype=torch.float32, validate=True)
    assert g["edge_index"].tolist() == [[0, 0, 1], [1, 2, 0]]
    assert g["vectors"].shape == (3, 3) and g["vectors"].dtype == torch.float32
    assert g["atom_types"].tolist() == [1, 0, 1]
    assert g["atomic_numbers"].tolist() == [8, 1, 8]
    assert g["batch"].shape == (2,) and g["lammps_exchange"] is True and g["use_shifts"] is False
    bad = _Data()
    bad.pair_j = np.array([1, 3, 0], dtype=np.int32)
    with pytest.raises(ValueError, match="pair_j"):
        graph_dict_from_mliap(bad, ["H", "O"], device="cpu", validate=True)


class _Exchange:
    """Ghost rows 2..3 are images of owned rows 1 and 0."""

    owner = torch.tensor([1, 0])

    def forward_exchange(self, src, dst, width):
        dst[:2] = src[:2]
        dst[2:] = src[self.owner]

    def reverse_exchange(self, src, dst, width):
        dst.copy_(src)
        dst[2:] = 0
        dst.index_add_(0, self.owner, src[2:])


def test_exchange_ops_are_adjoint_and_need_a_slot():
    from flashcart_amd.utils.lammps import lammps_data_slot, lammps_exchange_features
    x = torch.randn(2, 5, dtype=torch.float64, requires_grad=True)
    y = torch.randn(4, 5, dtype=torch.float64)
    with lammps_data_slot(_Exchange()):
        out = lammps_exchange_features(x, 2, 4)
        assert torch.equal(out[2], x[1].detach()) and torch.equal(out[3], x[0].detach())
        (g,) = torch.autograd.grad((out * y).sum(), x)
    # d/dx <F x, y> = F^T y: owners collect their ghosts' weights
    assert torch.allclose(g, y[:2] + y[2:].flip(0))
    with pytest.raises(RuntimeError, match="lammps_data_slot"):
        lammps_exchange_features(x, 2, 4)
    with pytest.raises(RuntimeError, match="rows"):
        with lammps_data_slot(_Exchange()):
            lammps_exchange_features(torch.zeros(3, 5), 2, 4)


class _Atoms:
    def __init__(self, z, p, cell, pbc):
        self.z, self.p, self.cell, self.pbc = np.asarray(z), np.asarray(p, float), np.asarray(cell), pbc

    def get_positions(self):
        return self.p.copy()

    def get_atomic_numbers(self):
        return self.z.copy()

    def get_cell(self):
        return self.cell.copy()

    def get_pbc(self):
        return np.array([self.pbc] * 3)

    def copy(self):
        return _Atoms(self.z, self.p, self.cell, self.pbc)


def test_calculator_reuse_rule_and_ignored_options():
    from flashcart_amd.calculators import FlashCartCalculator
    from flashcart_amd.model import FlashCartPotential
    model = FlashCartPotential.from_config(model_config(["Cu", "Ni", "Fe", "Cr"], 8, 2, avg_neighbors=42.0))
    with pytest.warns(UserWarning, match="ignored"):
        FlashCartCalculator(model=model, compile_mode="default")
    with pytest.raises(ValueError):
        FlashCartCalculator()
    calc = FlashCartCalculator(model=model, skin=1.0)
    z, p, cell, _ = fcc_alloy(1, 1, 2, seed=0)
    calc.atoms = _Atoms(z, p, cell, True)
    g0 = calc._get_graph(["positions", "numbers"])
    calc.atoms = _Atoms(z, p + 0.4, cell, True)          # every atom moved 0.69 A > skin / 2
    assert calc._get_graph(["positions"]) is not g0
    g1 = calc._cached_graph
    calc.atoms = _Atoms(z, p + 0.4 + 0.2, cell, True)    # 0.35 A < skin / 2: reuse
    g2 = calc._get_graph(["positions"])
    assert calc._cached_graph is g1 and g2.edge_index is g1.edge_index
    assert np.allclose(g2.positions.numpy(), p + 0.6)
    assert calc._get_graph(["numbers"]) is not g1 and calc._cached_graph is not g1  # other change: rebuild
    # skin-extended list holds every pair within r_max + skin
    d = np.linalg.norm(g0.positions.numpy()[g0.edge_index[1].numpy()] + g0.shifts.numpy() @ cell
                       - g0.positions.numpy()[g0.edge_index[0].numpy()], axis=1)
    assert d.max() > 5.0 and d.max() <= 6.0 + 1e-9
