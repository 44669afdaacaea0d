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
"""

from __future__ import annotations

from typing import Dict, List, Tuple

import numpy as np

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
