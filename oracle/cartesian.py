"""Oracle: numeric (float64) construction of the Cartesian expansion and tensor product.

TEST INFRASTRUCTURE ONLY. Imported by tests/, __graft_entry__.smoke() and the
bench's cpu_baseline leg as the checker; never by the flashcart_amd package.

This module reaches the reference's definitions by a route independent of the
HIP code generator (flashcart_amd/codegen), so the two check each other:

* the STF projection is the orthogonal projector onto symmetric traceless tensors
  of the full 3^L space, built numerically with an SVD (a traceless symmetric part
  is Frobenius-orthogonal to every Sym(delta (x) Q) term, so this equals the
  c_k(L) detracer of reference src/flashcart/o3/_codegen_tensor_product.py:362-388
  applied after the permutation average of :298-319);
* Eq. (1) (reference src/flashcart/o3/_codegen_irreps.py:3-14,147-164) is built as
  (2l-1)!!/l! * sum_m (-1)^m (2l-2m-1)!!/(2l-1)!! * P_m * Sym(r^(l-2m) (x) delta^m),
  where P_m = l!/((l-2m)! m! 2^m) converts the permutation average into the
  reference's sum over distinct placements; the delta factors are constants, so the
  polynomial (and its derivative) is the reference's for any input vector;
* path coefficients B[a,b,c] are evaluated as numbers on stored unit vectors;
* N(l1,l2,lo) is the closed form of reference _codegen_tensor_product.py:102-142.

Pinned by (tests/test_oracle_*.py): the reference's einsum closed forms for the 15
canonical l<=3 paths (tests/o3/test_codegen_tensor_product.py:101-202 of the
reference), explicit l<=3 expansion polynomials, tracelessness/symmetry, rotation
equivariance, and agreement with the exact rational derivation.
"""

from __future__ import annotations

import itertools
import math
from functools import lru_cache
from typing import Dict, List, Tuple

import numpy as np

# Stored components (count_x, count_y, count_z), reference
# src/flashcart/o3/_codegen_common.py:37-73 (layout contract): explicit orders for ranks 0..3;
# from rank 4 on, the components with no z by descending x count, then those with one z.
STORED = {
    0: [(0, 0, 0)],
    1: [(1, 0, 0), (0, 1, 0), (0, 0, 1)],
    2: [(2, 0, 0), (0, 2, 0), (1, 1, 0), (1, 0, 1), (0, 1, 1)],
    3: [(3, 0, 0), (2, 1, 0), (2, 0, 1), (1, 2, 0), (1, 1, 1), (0, 2, 1), (0, 3, 0)],
    4: [(a, 4 - a, 0) for a in range(4, -1, -1)] + [(a, 3 - a, 1) for a in range(3, -1, -1)],
}


def dfact(n: int) -> int:
    return 1 if n <= 0 else n * dfact(n - 2)


def full_index(abc: Tuple[int, int, int]) -> int:
    """Flat index (last axis fastest) of the sorted multi-index with a x's, b y's, c z's."""
    a, b, c = abc
    flat = 0
    for d in (0,) * a + (1,) * b + (2,) * c:
        flat = flat * 3 + d
    return flat


@lru_cache(maxsize=None)
def sym_projector(L: int) -> np.ndarray:
    """Orthogonal projector (3^L x 3^L) onto fully symmetric tensors."""
    n = 3 ** L
    P = np.zeros((n, n))
    perms = list(itertools.permutations(range(L)))
    for flat, idx in enumerate(itertools.product(range(3), repeat=L)):
        for p in perms:
            q = tuple(idx[p[i]] for i in range(L))
            P[flat, np.ravel_multi_index(q, (3,) * L) if L else 0] += 1.0 / len(perms)
    return P


@lru_cache(maxsize=None)
def stf_projector(L: int) -> np.ndarray:
    """Orthogonal projector onto symmetric traceless rank-L tensors (numeric, via SVD)."""
    n = 3 ** L
    if L < 2:
        return sym_projector(L)
    S = sym_projector(L)
    # trace map: (3^(L-2) x 3^L), contracting the first two axes
    T = np.zeros((3 ** (L - 2), n))
    for rest_flat, rest in enumerate(itertools.product(range(3), repeat=L - 2)):
        for a in range(3):
            T[rest_flat, np.ravel_multi_index((a, a) + rest, (3,) * L)] = 1.0
    # basis of the symmetric subspace, then the null space of the trace within it
    u, s, _ = np.linalg.svd(S)
    Bsym = u[:, s > 0.5]
    _, s2, vt = np.linalg.svd(T @ Bsym)
    rank = int((s2 > 1e-10).sum())
    N = vt[rank:].T
    Q = Bsym @ N
    assert Q.shape[1] == 2 * L + 1
    return Q @ Q.T


@lru_cache(maxsize=None)
def reconstruction_matrix(l: int) -> np.ndarray:
    """(3^l, 2l+1): full components from stored ones, via the least-squares inverse of the selection.

    The stored components determine a symmetric traceless tensor uniquely; the full
    tensor is recovered as the unique element of the STF subspace whose stored
    entries match (solved numerically, independent of the tracelessness recursion).
    """
    if l == 0:
        return np.ones((1, 1))
    P = stf_projector(l)
    u, s, _ = np.linalg.svd(P)
    Q = u[:, s > 0.5]                       # (3^l, 2l+1) orthonormal basis of the STF space
    sel = [full_index(abc) for abc in STORED[l]]
    A = Q[sel, :]                           # stored entries of the basis tensors
    return Q @ np.linalg.inv(A)


def tp_norm(l1: int, l2: int, lo: int) -> float:
    """N(l1,l2,lo) = shuffle * ICTP closed form (reference _codegen_tensor_product.py:102-142)."""
    k = (l1 + l2 - lo) // 2
    J = l1 + l2 + lo
    J1, J2, J3 = J - 2 * l1 - 1, J - 2 * l2 - 1, J - 2 * lo - 1
    f = math.factorial
    num = f(l1) * f(l2) * dfact(2 * lo - 1) * f((J1 + 1) // 2) * f((J2 + 1) // 2)
    den = f(lo) * dfact(J1) * dfact(J2) * dfact(J3) * f(J // 2)
    return f(lo) / (f(l1 - k) * f(l2 - k)) * num / den


def allowed(l1: int, l2: int, lo: int) -> bool:
    return abs(l1 - l2) <= lo <= l1 + l2 and (l1 + l2 + lo) % 2 == 0


@lru_cache(maxsize=None)
def path_tensor(l1: int, l2: int, lo: int) -> np.ndarray:
    """B[a, b, c] (2lo+1, 2l1+1, 2l2+1): out_a = sum B x_b y_c for stored operands."""
    k = (l1 + l2 - lo) // 2
    M1, M2 = reconstruction_matrix(l1), reconstruction_matrix(l2)
    P = stf_projector(lo)
    sel = [full_index(abc) for abc in STORED[lo]]
    norm = tp_norm(l1, l2, lo)
    B = np.zeros((2 * lo + 1, 2 * l1 + 1, 2 * l2 + 1))
    for b in range(2 * l1 + 1):
        T1 = M1[:, b].reshape((3,) * l1) if l1 else np.array(M1[0, b])
        for c in range(2 * l2 + 1):
            T2 = M2[:, c].reshape((3,) * l2) if l2 else np.array(M2[0, c])
            # contract the last k axes of T1 with the first k axes of T2
            R = np.tensordot(T1, T2, axes=(list(range(l1 - k, l1)), list(range(k))))
            R = np.asarray(R).reshape(-1)
            B[:, b, c] = norm * (P @ R)[sel]
    return B


def enumerate_paths(in1_l_max: int, in2_l_max: int, out_l_max: int, symmetric: bool) -> List[Tuple[int, int, int, bool]]:
    """Weight order: per lo, canonical (l1>=l2, l1 from in1) then exchanged pairs
    (reference src/flashcart/o3/utils.py:157-203)."""
    out = []
    lp = max(in1_l_max, in2_l_max)
    for lo in range(out_l_max + 1):
        for l1 in range(lp + 1):
            for l2 in range(l1 + 1):
                if allowed(l1, l2, lo) and l1 <= in1_l_max and l2 <= in2_l_max:
                    out.append((l1, l2, lo, False))
        if not symmetric:
            for l1 in range(lp + 1):
                for l2 in range(l1):
                    if allowed(l1, l2, lo) and l1 <= in2_l_max and l2 <= in1_l_max:
                        out.append((l1, l2, lo, True))
    return out

