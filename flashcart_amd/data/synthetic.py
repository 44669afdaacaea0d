"""Seeded synthetic structures of the benchmark configurations.

* ``fcc_alloy``: periodic fcc random alloy (lattice constant a, n_species equal
  fractions by seeded permutation, Gaussian jitter).
* ``water_box``: periodic water-like box: O uniform with a minimum-image O-O
  distance, two H per O at 0.96 A with a 104.5 degree H-O-H angle, random
  orientation.
* ``molecules``: non-periodic random-walk molecules of C/H/N/O.
* ``model_config``: the packaged default architecture (l_max_hidden_feats=2,
  correlation=3, sigmoid gates, layer norm, cosine Chebyshev radial basis, radial and
  readout widths [64, 64]) with the given channels, edge rank and cutoff.
* ``fcc25k_system`` / ``StepGraphs`` / ``fcc25k_model``: the benchmark workload of
  BASELINE configuration 4 (25x25x10 fcc cells, a = 3.6 A, MD-style steps of N(0, 0.01^2) A,
  C = 128, L_max = 3, seed 1234), shared by bench.py and the full-size parity test.
"""

from __future__ import annotations

from typing import Dict, List, Tuple

import numpy as np
import torch

_Z = {"H": 1, "C": 6, "N": 7, "O": 8, "Cr": 24, "Fe": 26, "Ni": 28, "Cu": 29}


def fcc_alloy(nx: int, ny: int, nz: int, a: float = 3.6, elements=("Cu", "Ni", "Fe", "Cr"), jitter: float = 0.05,
              seed: int = 0):
    rng = np.random.default_rng(seed)
    basis = np.array([[0, 0, 0], [0.5, 0.5, 0], [0.5, 0, 0.5], [0, 0.5, 0.5]])
    grid = np.stack(np.meshgrid(np.arange(nx), np.arange(ny), np.arange(nz), indexing="ij"), -1).reshape(-1, 3)
    pos = ((grid[:, None, :] + basis[None]) * a).reshape(-1, 3)
    n = pos.shape[0]
    per = n // len(elements)
    species = np.concatenate([np.full(per + (1 if k < n % len(elements) else 0), k)
                              for k, _ in enumerate(elements)])
    species = species[rng.permutation(n)]
    numbers = np.array([_Z[elements[s]] for s in species])
    pos = pos + rng.normal(0.0, jitter, size=pos.shape)
    cell = np.diag([nx * a, ny * a, nz * a]).astype(np.float64)
    return numbers, pos, cell, np.array([True, True, True])


def _random_rotation(rng) -> np.ndarray:
    q = rng.normal(size=4)
    q /= np.linalg.norm(q)
    w, x, y, z = q
    return np.array([[1 - 2 * (y * y + z * z), 2 * (x * y - z * w), 2 * (x * z + y * w)],
                     [2 * (x * y + z * w), 1 - 2 * (x * x + z * z), 2 * (y * z - x * w)],
                     [2 * (x * z - y * w), 2 * (y * z + x * w), 1 - 2 * (x * x + y * y)]])


def water_box(n_molecules: int = 512, density: float = 1.0, min_oo: float = 2.5, seed: int = 0):
    rng = np.random.default_rng(seed)
    mass = 18.01528 / 6.02214076e23  # g per molecule
    L = (n_molecules * mass / density * 1e24) ** (1.0 / 3.0)  # Angstrom
    O = np.empty((0, 3))
    while O.shape[0] < n_molecules:
        c = rng.uniform(0.0, L, size=3)
        if O.shape[0]:
            dv = O - c
            dv -= L * np.round(dv / L)
            if np.min(np.linalg.norm(dv, axis=1)) < min_oo:
                continue
        O = np.vstack([O, c])
    half = np.deg2rad(104.5) / 2
    local = 0.96 * np.array([[np.sin(half), np.cos(half), 0.0], [-np.sin(half), np.cos(half), 0.0]])
    pos, numbers = [], []
    for o in O:
        R = _random_rotation(rng)
        pos += [o, o + R @ local[0], o + R @ local[1]]
        numbers += [8, 1, 1]
    return np.array(numbers), np.array(pos), np.diag([L, L, L]).astype(np.float64), np.array([True] * 3)


def molecules(n_mol: int = 512, n_min: int = 20, n_max: int = 50, probs=(0.3, 0.5, 0.1, 0.1),
              bond=(1.0, 1.5), min_dist: float = 0.9, seed: int = 0) -> List[Tuple[np.ndarray, np.ndarray]]:
    rng = np.random.default_rng(seed)
    syms = np.array([6, 1, 7, 8])
    out = []
    for _ in range(n_mol):
        n = int(rng.integers(n_min, n_max + 1))
        pos = [np.zeros(3)]
        while len(pos) < n:
            v = rng.normal(size=3)
            step = pos[-1] + v / np.linalg.norm(v) * rng.uniform(*bond)
            if np.min(np.linalg.norm(np.array(pos) - step, axis=1)) < min_dist:
                continue
            pos.append(step)
        out.append((rng.choice(syms, size=n, p=probs), np.array(pos)))
    return out


def model_config(elements, n_hidden_feats: int, l_max_edge_attrs: int, r_max: float = 5.0,
                 avg_neighbors: float = 1.0, n_interactions: int = 2) -> Dict:
    """Constructor config of FlashCartPotential with the packaged default architecture."""
    return dict(
        elements=list(elements), r_max=r_max, r_min=0.0, n_hidden_feats=n_hidden_feats, l_max_hidden_feats=2,
        l_max_edge_attrs=l_max_edge_attrs, n_radial=8, n_interactions=n_interactions, correlation=3,
        path_reduced_product=False, element_agnostic_interaction=True, element_agnostic_product=True,
        n_element_interaction_features=16, nonlinearity=True, gate_activation="sigmoid", gate_bias=True,
        layer_norm=True, hidden_radial=[64, 64], hidden_readout=[64, 64], radial_mapping="cosine",
        cutoff_poly_order=6, avg_neighbors=float(avg_neighbors), atomic_shifts=[0.0] * len(elements),
        fit_atomic_shifts=False, use_triton=True,
    )


FCC25K_R_MAX = 5.0
FCC25K_SIGMA_STEP = 0.01
FCC25K_SKIN = 1.0
FCC25K_ELEMENTS = ("Cu", "Ni", "Fe", "Cr")


def fcc25k_system(nx=25, ny=25, nz=10, seed=0):
    """fcc random alloy, a = 3.6 A, jitter 0.05 A, 4 species."""
    return fcc_alloy(nx, ny, nz, a=3.6, jitter=0.05, seed=seed)


class StepGraphs:
    """Per-step graphs of an MD-style run with exact r_max connectivity from a skin list (host side).

    Step k perturbs the previous positions by N(0, sigma^2) (rng seed ``seed``); the host cell list
    at r_max + skin is rebuilt when an atom moved more than skin / 2 since the last build, and each
    step keeps the pairs within r_max (in the list's (i, j, S) order)."""

    def __init__(self, numbers, pos, cell, pbc, elements, n_steps, seed=1, r_max=FCC25K_R_MAX,
                 sigma=FCC25K_SIGMA_STEP, skin=FCC25K_SKIN):
        from flashcart_amd.data.graph import numbers_to_types
        from flashcart_amd.data.neighbors import neighbor_pairs
        self.types = torch.as_tensor(numbers_to_types(numbers, elements))
        self.numbers = numbers
        self.cell = cell
        self.pbc = pbc
        rng = np.random.default_rng(seed)
        self.graphs = []
        ref_pos, skin_list = None, None
        cur = pos.copy()
        n_rebuild = 0
        for _ in range(n_steps):
            cur = cur + rng.normal(0.0, sigma, size=cur.shape)
            if ref_pos is None or np.max(np.linalg.norm(cur - ref_pos, axis=1)) >= skin / 2:
                ref_pos = cur.copy()
                skin_list = neighbor_pairs(cur, cell, pbc, r_max + skin)
                n_rebuild += 1
            ei, sh = skin_list
            v = cur[ei[1]] - cur[ei[0]] + sh @ cell
            keep = np.einsum("ij,ij->i", v, v) < r_max * r_max
            self.graphs.append((cur.astype(np.float64), ei[:, keep].copy(), sh[keep].copy()))
        self.n_rebuild = n_rebuild

    def graph(self, k, device="cpu"):
        """Step k as an AtomicGraph with float32 positions and cell."""
        from flashcart_amd.data.graph import AtomicGraph
        pos, ei, sh = self.graphs[k]
        n = pos.shape[0]
        return AtomicGraph(
            positions=torch.as_tensor(pos, dtype=torch.float32, device=device),
            cell=torch.as_tensor(self.cell, dtype=torch.float32, device=device).unsqueeze(0),
            pbc=torch.as_tensor(self.pbc, device=device).unsqueeze(0),
            shifts=torch.as_tensor(sh, dtype=torch.long, device=device),
            edge_index=torch.as_tensor(ei, dtype=torch.long, device=device),
            atom_types=self.types.to(device), atomic_numbers=torch.as_tensor(self.numbers, device=device),
            n_atoms=torch.tensor([n], dtype=torch.long, device=device), use_shifts=True)


def fcc25k_model(avg_neighbors, channels=128, l_max=3):
    """The benchmark model: default architecture, random init from torch.manual_seed(1234),
    frozen parameters (inference)."""
    from flashcart_amd.model import FlashCartPotential
    cfg = model_config(list(FCC25K_ELEMENTS), channels, l_max, r_max=FCC25K_R_MAX, avg_neighbors=avg_neighbors)
    torch.manual_seed(1234)
    model = FlashCartPotential.from_config(cfg)
    for p in model.parameters():
        p.requires_grad_(False)
    return model, cfg
