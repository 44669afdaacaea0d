"""Oracle: brute-force neighbour list (small systems only).

TEST INFRASTRUCTURE ONLY. Restates the reference's edge-set contract
(src/flashcart/data/neighbors.py:120-143): all (i, j, S) with
|pos[j] - pos[i] + S.cell| < cutoff over periodic images S, excluding i == j with
S = 0, sorted by receiver i (within a receiver: j, then S, the canonical order).
Pinned by the reference's neighbour-count known answers
(tests/data/test_data.py:96-108) and by periodic-image existence checks.
"""

import itertools

import numpy as np


def brute_force_pairs(pos, cell, pbc, cutoff, n_img=2):
    pos = np.asarray(pos, dtype=np.float64)
    cell = np.asarray(cell, dtype=np.float64).reshape(3, 3)
    ranges = [range(-n_img, n_img + 1) if p else range(0, 1) for p in np.broadcast_to(pbc, (3,))]
    out = []
    for i in range(len(pos)):
        for j in range(len(pos)):
            for S in itertools.product(*ranges):
                if i == j and S == (0, 0, 0):
                    continue
                v = pos[j] - pos[i] + np.asarray(S) @ cell
                if v @ v < cutoff * cutoff:
                    out.append((i, j) + tuple(S))
    out.sort()
    return out
