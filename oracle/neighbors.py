"""Oracle: brute-force neighbour list (small systems only).

TEST INFRASTRUCTURE ONLY. Restates the reference's edge-set contract
(src/flashcart/data/neighbors.py:120-143): all (i, j, S) with
|pos[j] - pos[i] + S.cell| < cutoff over periodic images S, excluding i == j with
S = 0, sorted by receiver i (within a receiver: j, then S, the canonical order).
Pinned by the reference's neighbour-count known answers
(tests/data/test_data.py:96-108) and by periodic-image existence checks.
"""

import itertools
import math

import numpy as np


def brute_force_pairs(pos, cell, pbc, cutoff, n_img=None):
    """Every (i, j, Sx, Sy, Sz) as a sorted list of tuples. ``n_img``: images -n_img..n_img per
    periodic axis (default: enough for the cutoff, from the cell's plane spacings)."""
    pos = np.asarray(pos, dtype=np.float64).reshape(-1, 3)
    cell = np.asarray(cell, dtype=np.float64).reshape(3, 3)
    pbc = np.broadcast_to(np.asarray(pbc, dtype=bool), (3,))
    ranges = []
    if n_img is None and np.any(pbc) and len(pos):
        # unwrapped positions: pairs can need shifts as large as the spread of the fractional
        # coordinates plus the cutoff's reach
        frac = pos @ np.linalg.inv(cell)
        spread = frac.max(axis=0) - frac.min(axis=0)
    for a in range(3):
        if not pbc[a]:
            ranges.append(range(0, 1))
            continue
        if n_img is None:
            other = np.cross(cell[(a + 1) % 3], cell[(a + 2) % 3])
            spacing = abs(float(np.dot(cell[a], other))) / float(np.linalg.norm(other))
            k = int(math.ceil(cutoff / spacing)) + int(math.ceil(spread[a])) + 1
        else:
            k = n_img
        ranges.append(range(-k, k + 1))
    out = []
    diff = pos[None, :, :] - pos[:, None, :]          # [i, j] = pos[j] - pos[i]
    for S in itertools.product(*ranges):
        v = diff + np.asarray(S, dtype=np.float64) @ cell
        d2 = np.einsum("ijk,ijk->ij", v, v)
        for i, j in zip(*np.nonzero(d2 < cutoff * cutoff)):
            if i == j and S == (0, 0, 0):
                continue
            out.append((int(i), int(j)) + tuple(S))
    out.sort()
    return out
