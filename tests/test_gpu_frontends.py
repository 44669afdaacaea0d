"""GPU parity of the front-ends: the ASE-style calculator and the LAMMPS ML-IAP interface.

Calculator results (energy, forces, stress) are checked against the float64 oracle
(stress via the virtual-strain derivative, pinned by finite differences on the CPU).
The LAMMPS path is checked by re-expressing a periodic structure the way a
single-rank LAMMPS run hands it over — owned atoms, ghost images for every periodic
neighbour, pair vectors — evaluating edge forces through ``compute_forces`` with a
stand-in data object whose exchange hooks copy owner features to ghosts (and add
ghost gradients back), and folding ghost forces onto their owners as LAMMPS's reverse
communication does. Energies and forces must equal the periodic-graph prediction.
"""

import numpy as np
import pytest
import torch

from flashcart_amd.data import AtomicGraph
from flashcart_amd.data.synthetic import fcc_alloy, model_config, molecules
from oracle import model as OM
from tests.helpers import assert_close

pytestmark = pytest.mark.gpu
DEV = "cuda"


class Atoms:
    """Minimal structure object with the methods the calculator reads."""

    def __init__(self, numbers, positions, cell=None, pbc=False):
        self.numbers = np.asarray(numbers)
        self.positions = np.asarray(positions, dtype=np.float64)
        self.cell = np.zeros((3, 3)) if cell is None else np.asarray(cell, dtype=np.float64)
        self.pbc = np.broadcast_to(np.asarray(pbc, dtype=bool), (3,)).copy()
        self.calc = None

    def get_positions(self):
        return self.positions.copy()

    def get_atomic_numbers(self):
        return self.numbers.copy()

    def get_cell(self):
        return self.cell.copy()

    def get_pbc(self):
        return self.pbc.copy()

    def copy(self):
        return Atoms(self.numbers, self.positions, self.cell, self.pbc)


def _model(cfg, seed):
    from flashcart_amd.model import FlashCartPotential
    torch.manual_seed(seed)
    m = FlashCartPotential.from_config(cfg)
    g = torch.Generator().manual_seed(seed + 1)
    with torch.no_grad():
        for name, p in m.named_parameters():
            if "output_linear" in name:
                p.copy_(0.5 * torch.randn(p.shape, generator=g))
    return m


def _oracle(model, atoms, stress=False):
    g = AtomicGraph.from_arrays(atoms.numbers, atoms.positions, model.elements, model.r_max, cell=atoms.cell,
                                pbc=atoms.pbc, dtype=torch.float64)
    return OM.predict(model.state_dict(), model.to_model_config(), g.to_dict(), compute_stress=stress)


def test_calculator_energy_forces_stress():
    from flashcart_amd.calculators import FlashCartCalculator
    z, p, cell, pbc = fcc_alloy(2, 2, 1, seed=5)
    cfg = model_config(["Cu", "Ni", "Fe", "Cr"], 16, 3, avg_neighbors=42.0)
    model = _model(cfg, 21)
    ref = _oracle(model, Atoms(z, p, cell, pbc), stress=True)
    calc = FlashCartCalculator(model=model, device=DEV)
    atoms = Atoms(z, p, cell, pbc)
    calc.calculate(atoms, ["energy", "forces", "stress"])
    r = calc.results
    assert isinstance(r["energy"], float)
    assert abs(r["energy"] - float(ref["energy"][0])) <= 1e-5 * abs(float(ref["energy"][0])) + 1e-6
    assert_close(torch.as_tensor(r["forces"]), ref["forces"], 0.0, 1e-4, "calculator forces")
    assert r["stress"].shape == (6,)
    assert_close(torch.as_tensor(r["stress"]), ref["stress"][0], 1e-4, 1e-6, "calculator stress")


def test_calculator_skin_reuse_matches_rebuild():
    from flashcart_amd.calculators import FlashCartCalculator
    z, p, cell, pbc = fcc_alloy(2, 2, 1, seed=6)
    cfg = model_config(["Cu", "Ni", "Fe", "Cr"], 16, 2, avg_neighbors=42.0)
    model = _model(cfg, 22).to(DEV)
    reuse = FlashCartCalculator(model=model, skin=1.0)
    fresh = FlashCartCalculator(model=model, skin=0.0)
    rng = np.random.default_rng(0)
    atoms = Atoms(z, p, cell, pbc)
    e0 = reuse.get_potential_energy(atoms)
    graph0 = reuse._cached_graph
    for step in range(3):
        atoms = atoms.copy()
        atoms.positions = atoms.positions + rng.normal(0, 0.05, atoms.positions.shape)
        e_reuse, f_reuse = reuse.get_potential_energy(atoms), reuse.get_forces(atoms)
        e_new, f_new = fresh.get_potential_energy(atoms), fresh.get_forces(atoms)
        assert reuse._cached_graph is graph0  # connectivity kept while displacements < skin / 2
        assert abs(e_reuse - e_new) <= 1e-5 * abs(e_new)
        assert np.abs(f_reuse - f_new).max() < 1e-4
    assert e0 != e_new


def test_calculator_molecule_and_atomic_offsets():
    from flashcart_amd.calculators import FlashCartCalculator
    (z, p), = molecules(1, 12, 12, seed=3)
    cfg = model_config(["H", "C", "N", "O"], 8, 2, avg_neighbors=6.0)
    model = _model(cfg, 23)
    with torch.no_grad():
        model.scale_shift.shifts.copy_(torch.tensor([-0.5, -3.0, -2.0, -4.0]))
    ref = _oracle(model, Atoms(z, p))
    calc = FlashCartCalculator(model=model, device=DEV, add_atomic_offsets=True)
    e = calc.get_potential_energy(Atoms(z, p))
    types = {1: 0, 6: 1, 7: 2, 8: 3}
    offset = sum([-0.5, -3.0, -2.0, -4.0][types[int(k)]] for k in z)
    assert abs(e - (float(ref["energy"][0]) + offset)) <= 1e-5 * abs(float(ref["energy"][0])) + 1e-5
    assert_close(torch.as_tensor(calc.get_forces()), ref["forces"], 0.0, 1e-4, "molecule forces")


class MLIAPData:
    """Single-rank stand-in for the ML-IAP data object: owned atoms plus ghost images."""

    def __init__(self, graph, n_local, with_f=False):
        ei = graph.edge_index.numpy()
        shifts = graph.shifts.numpy()
        pos = graph.positions.double().numpy()
        cell = graph.cell[0].double().numpy()
        ghost_of, owner = {}, []
        pair_j = np.empty(ei.shape[1], dtype=np.int32)
        for e, (j, s) in enumerate(zip(ei[1], map(tuple, shifts))):
            if s == (0, 0, 0):
                pair_j[e] = j
                continue
            key = (int(j), s)
            if key not in ghost_of:
                ghost_of[key] = n_local + len(owner)
                owner.append(int(j))
            pair_j[e] = ghost_of[key]
        self.owner = np.asarray(owner, dtype=np.int64)
        self.nlocal = n_local
        self.ntotal = n_local + len(owner)
        self.npairs = ei.shape[1]
        self.pair_i = ei[0].astype(np.int32)
        self.pair_j = pair_j
        self.rij = pos[ei[1]] + shifts @ cell - pos[ei[0]]
        types = graph.atom_types.numpy()
        self.elems = np.concatenate([types, types[self.owner]]).astype(np.int32)
        self.eflag = True
        self.eatoms = np.zeros(self.ntotal)
        self.energy = None
        self.pair_forces = None
        if with_f:
            self.f = np.zeros((self.ntotal, 3))

    def forward_exchange(self, src, dst, width):
        own = torch.as_tensor(self.owner, device=src.device)
        dst[: self.nlocal] = src[: self.nlocal]
        dst[self.nlocal:] = src[own]

    def reverse_exchange(self, src, dst, width):
        own = torch.as_tensor(self.owner, device=src.device)
        dst.copy_(src)
        dst[self.nlocal:] = 0
        dst.index_add_(0, own, src[self.nlocal:])

    def fold_ghosts(self, f):
        out = f[: self.nlocal].copy()
        np.add.at(out, self.owner, f[self.nlocal:])
        return out


def _pair_forces_to_atoms(data, pf):
    f = np.zeros((data.ntotal, 3))
    np.add.at(f, data.pair_i, pf)
    np.add.at(f, data.pair_j, -pf)
    return data.fold_ghosts(f)


class PairData(MLIAPData):
    def update_pair_forces(self, pf):
        self.pair_forces = pf.detach().cpu().numpy() if torch.is_tensor(pf) else np.asarray(pf)


@pytest.mark.parametrize("use_f", [False, True], ids=["update_pair_forces", "data_f"])
def test_lammps_mliap_matches_periodic_oracle(use_f):
    from flashcart_amd.calculators import FlashCartLAMMPSUnified
    z, p, cell, pbc = fcc_alloy(2, 2, 2, seed=9)
    cfg = model_config(["Cu", "Ni", "Fe", "Cr"], 16, 3, avg_neighbors=42.0)
    model = _model(cfg, 24)
    with torch.no_grad():
        model.scale_shift.shifts.copy_(torch.tensor([0.1, -0.2, 0.3, -0.4]))
    g = AtomicGraph.from_arrays(z, p, cfg["elements"], 5.0, cell=cell, pbc=pbc)
    # the oracle's periodic prediction (float64, CPU) of the same structure and parameters
    ref = OM.predict(model.state_dict(), model.to_model_config(), g.to_dict(), compute_forces=True)
    model = model.to(DEV)
    unified = FlashCartLAMMPSUnified(model, add_atomic_offsets=True)
    data = MLIAPData(g, len(z), with_f=True) if use_f else PairData(g, len(z))
    data.rij = torch.as_tensor(data.rij, dtype=torch.float32, device=DEV)  # device array, as KOKKOS hands over
    unified.compute_forces(data)
    assert data.ntotal > data.nlocal  # ghosts present: exchange hooks exercised
    shift = float(model.scale_shift.shifts.double()[g.atom_types].sum())
    e_ref = float(ref["energy"][0])
    assert abs(data.energy - (e_ref + shift)) <= 1e-5 * abs(e_ref) + 1e-6
    assert_close(torch.as_tensor(data.eatoms[: data.nlocal]),
                 ref["node_energies"].double().cpu() + model.scale_shift.shifts.double().cpu()[g.atom_types],
                 1e-5, 1e-6, "eatoms")
    forces = data.fold_ghosts(data.f) if use_f else _pair_forces_to_atoms(data, data.pair_forces)
    assert_close(torch.as_tensor(forces), ref["forces"], 0.0, 1e-4, "LAMMPS forces")


def test_single_rank_mliap_data_matches_oracle():
    """The packaged single-rank ML-IAP layout (``SingleRankMLIAPData``: ghosts per periodic
    image, device arrays, pair forces kept on the device) reproduces the oracle's periodic
    prediction of the same structure."""
    from flashcart_amd.calculators import FlashCartLAMMPSUnified, SingleRankMLIAPData
    z, p, cell, pbc = fcc_alloy(3, 2, 2, seed=11)
    cfg = model_config(["Cu", "Ni", "Fe", "Cr"], 16, 3, avg_neighbors=42.0)
    model = _model(cfg, 31)
    g = AtomicGraph.from_arrays(z, p, cfg["elements"], 5.0, cell=cell, pbc=pbc)
    ref = OM.predict(model.state_dict(), model.to_model_config(), g.to_dict(), compute_forces=True)
    model = model.to(DEV)
    data = SingleRankMLIAPData(g, device=DEV)
    FlashCartLAMMPSUnified(model).compute_forces(data)
    assert data.ntotal > data.nlocal and data.pair_forces.is_cuda
    e_ref = float(ref["energy"][0])
    assert abs(data.energy - e_ref) <= 1e-5 * abs(e_ref) + 1e-6
    assert_close(data.atom_forces(), ref["forces"], 0.0, 1e-4, "LAMMPS forces (single-rank data)")
