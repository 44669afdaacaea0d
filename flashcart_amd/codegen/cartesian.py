"""Exact (rational) derivation of the irreducible Cartesian expansion and tensor product.

This module is the build-time derivation that the HIP code generator consumes. It
works in exact rational arithmetic (``fractions.Fraction`` for the tensor algebra,
SymPy for the polynomials that are differentiated and printed), so the constants
that reach the kernels are exact before they are rounded to float.

Layout contract (must match the reference bit for bit):

* ``stored_basis`` lists the 2l+1 independent components of a rank-l symmetric
  traceless tensor as (count_x, count_y, count_z); reference
  ``src/flashcart/o3/_codegen_common.py:37-73``.
* Components with two or more z indices are reconstructed from tracelessness,
  T(a,b,c) = -T(a+2,b,c-2) - T(a,b+2,c-2); reference
  ``src/flashcart/o3/_codegen_tensor_product.py:214-250``.

Eq. (1), the expansion of a unit vector (reference
``src/flashcart/o3/_codegen_irreps.py:3-14,147-164``)::

    T^l(r) = (2l-1)!!/l! * sum_m (-1)^m (2l-2m-1)!!/(2l-1)!! * {r^(l-2m) (x) I^m}

where the braces sum over distinct placements (not averaged). The polynomial is
evaluated as written for any input vector; the Kronecker deltas contribute
constants, so its derivative is the unconstrained polynomial derivative.

Eq. (2), one coupling path (l1, l2) -> lo of the tensor product (reference
``src/flashcart/o3/_codegen_tensor_product.py:10-27,102-142,282-414``)::

    TP(T1, T2) = N(l1,l2,lo) * STF_lo( Sym_lo( contract_k(T1 (x) T2) ) ),  k=(l1+l2-lo)/2

with the last k indices of T1 contracted against the first k of T2, Sym the
average over lo! permutations, STF the detracer with
c_k(L) = (-1)^k L! (2L-2k-1)!! / [k! (L-2k)! (2L-1)!! 2^k], and N the closed form
of ``_even_tp_norm`` times the shuffle multiplicity lo!/((l1-k)!(l2-k)!).

The product of one path is bilinear in the stored inputs, so it is represented by
its exact coefficient tensor ``B[a][b][c]``: out_a = sum_{b,c} B[a,b,c] S1_b S2_c.
"""

from __future__ import annotations

import math
from fractions import Fraction
from functools import lru_cache
from itertools import permutations, product
from typing import Dict, List, Tuple

import sympy as sp

Idx = Tuple[int, ...]


def double_factorial(n: int) -> int:
    """n!! with the convention (-1)!! = 1 (and 1 for every negative n)."""
    out = 1
    while n > 1:
        out *= n
        n -= 2
    return out


def stored_basis(l: int) -> List[Tuple[int, int, int]]:
    """(count_x, count_y, count_z) of the stored components of rank l.

    Ranks 0..3 use the explicit reference order; higher ranks list c=0 by
    descending a, then c=1 by descending a (reference
    ``src/flashcart/o3/_codegen_common.py:37-73``).
    """
    explicit = {
        0: [(0, 0, 0)],
        1: [(1, 0, 0), (0, 1, 0), (0, 0, 1)],
        2: [(2, 0, 0), (0, 2, 0), (1, 1, 0), (1, 0, 1), (0, 1, 1)],
        3: [(3, 0, 0), (2, 1, 0), (2, 0, 1), (1, 2, 0), (1, 1, 1), (0, 2, 1), (0, 3, 0)],
    }
    if l in explicit:
        return list(explicit[l])
    comps = [(a, l - a, 0) for a in range(l, -1, -1)]
    comps += [(a, l - 1 - a, 1) for a in range(l - 1, -1, -1)]
    return comps


@lru_cache(maxsize=None)
def reconstruction(l: int) -> Dict[Idx, Dict[int, int]]:
    """Map every full Cartesian index tuple of rank l to integer stored-component weights.

    Returns ``{full_idx: {stored_position: weight}}``; full components with >=2 z
    indices are expanded with the tracelessness recursion.
    """
    if l == 0:
        return {(): {0: 1}}
    pos = {abc: i for i, abc in enumerate(stored_basis(l))}
    memo: Dict[Tuple[int, int, int], Dict[int, int]] = {}

    def comp(a: int, b: int, c: int) -> Dict[int, int]:
        key = (a, b, c)
        if key in memo:
            return memo[key]
        if key in pos:
            out = {pos[key]: 1}
        elif c >= 2:
            out: Dict[int, int] = {}
            for sub in (comp(a + 2, b, c - 2), comp(a, b + 2, c - 2)):
                for k, v in sub.items():
                    out[k] = out.get(k, 0) - v
            out = {k: v for k, v in out.items() if v != 0}
        else:
            raise ValueError(f"component ({a},{b},{c}) of rank {l} is neither stored nor reconstructible")
        memo[key] = out
        return out

    return {idx: comp(idx.count(0), idx.count(1), idx.count(2)) for idx in product(range(3), repeat=l)}


def path_allowed(l1: int, l2: int, lo: int) -> bool:
    """Triangle rule and natural parity (reference ``_codegen_tensor_product.py:145-163``)."""
    return min(l1, l2, lo) >= 0 and abs(l1 - l2) <= lo <= l1 + l2 and (l1 + l2 + lo) % 2 == 0


@lru_cache(maxsize=None)
def tp_norm(l1: int, l2: int, lo: int) -> Fraction:
    """Path normalization N(l1,l2,lo) (reference ``_codegen_tensor_product.py:102-142``)."""
    if not path_allowed(l1, l2, lo):
        raise ValueError(f"path ({l1},{l2},{lo}) is not allowed")
    k = (l1 + l2 - lo) // 2
    J = l1 + l2 + lo
    J1, J2, J3 = J - 2 * l1 - 1, J - 2 * l2 - 1, J - 2 * lo - 1
    f, df = math.factorial, double_factorial
    num = f(l1) * f(l2) * df(2 * lo - 1) * f((J1 + 1) // 2) * f((J2 + 1) // 2)
    den = f(lo) * df(J1) * df(J2) * df(J3) * f(J // 2)
    shuffle = Fraction(f(lo), f(l1 - k) * f(l2 - k))
    return shuffle * Fraction(num, den)


# ---------------------------------------------------------------------------
# Full-tensor algebra over Fractions (dict: full index tuple -> value)
# ---------------------------------------------------------------------------

def _full_from_unit(l: int, position: int) -> Dict[Idx, Fraction]:
    """Full tensor of the stored unit vector e_position of rank l."""
    return {idx: Fraction(w.get(position, 0)) for idx, w in reconstruction(l).items()}


def _contract(T1: Dict[Idx, Fraction], l1: int, T2: Dict[Idx, Fraction], l2: int, k: int) -> Dict[Idx, Fraction]:
    """Outer product with the last k indices of T1 contracted against the first k of T2."""
    lo = l1 + l2 - 2 * k
    out: Dict[Idx, Fraction] = {}
    for idx in product(range(3), repeat=lo):
        head, tail = idx[: l1 - k], idx[l1 - k:]
        s = Fraction(0)
        for cidx in product(range(3), repeat=k):
            s += T1[head + cidx] * T2[cidx + tail]
        out[idx] = s
    return out


def _symmetrize(R: Dict[Idx, Fraction], L: int) -> Dict[Idx, Fraction]:
    """Average over all L! index permutations."""
    if L <= 1:
        return dict(R)
    perms = list(permutations(range(L)))
    inv = Fraction(1, len(perms))
    return {idx: inv * sum((R[tuple(idx[p[i]] for i in range(L))] for p in perms), Fraction(0))
            for idx in product(range(3), repeat=L)}


def _trace_once(R: Dict[Idx, Fraction], L: int) -> Dict[Idx, Fraction]:
    return {rest: sum((R[(a, a) + rest] for a in range(3)), Fraction(0))
            for rest in product(range(3), repeat=L - 2)}


def _detrace(R: Dict[Idx, Fraction], L: int) -> Dict[Idx, Fraction]:
    """STF projection of a symmetric tensor with the c_k(L) detracer coefficients."""
    if L < 2:
        return dict(R)
    out = dict(R)
    traced = R
    perms = list(permutations(range(L)))
    for k in range(1, L // 2 + 1):
        traced = _trace_once(traced, L - 2 * (k - 1))
        ck = Fraction((-1) ** k * math.factorial(L) * double_factorial(2 * L - 2 * k - 1),
                      math.factorial(k) * math.factorial(L - 2 * k) * double_factorial(2 * L - 1) * 2 ** k)
        for idx in out:
            acc = Fraction(0)
            for p in perms:
                q = tuple(idx[p[i]] for i in range(L))
                if all(q[2 * j] == q[2 * j + 1] for j in range(k)):
                    acc += traced[q[2 * k:]]
            out[idx] += ck * acc / len(perms)
    return out


@lru_cache(maxsize=None)
def tp_coefficients(l1: int, l2: int, lo: int) -> Dict[Tuple[int, int, int], Fraction]:
    """Exact bilinear coefficients B[a,b,c] of one path: out_a = sum B[a,b,c] S1_b S2_c.

    ``a`` indexes stored output components, ``b`` the first input and ``c`` the
    second input, all in ``stored_basis`` order. Zero coefficients are omitted.
    """
    if not path_allowed(l1, l2, lo):
        raise ValueError(f"path ({l1},{l2},{lo}) is not allowed")
    k = (l1 + l2 - lo) // 2
    norm = tp_norm(l1, l2, lo)
    out_idx = [tuple([0] * a + [1] * b + [2] * c) for a, b, c in stored_basis(lo)]
    coeffs: Dict[Tuple[int, int, int], Fraction] = {}
    for b in range(2 * l1 + 1):
        T1 = _full_from_unit(l1, b)
        for c in range(2 * l2 + 1):
            T2 = _full_from_unit(l2, c)
            R = _detrace(_symmetrize(_contract(T1, l1, T2, l2, k), lo), lo)
            for a, idx in enumerate(out_idx):
                v = norm * R[idx]
                if v != 0:
                    coeffs[(a, b, c)] = v
    return coeffs


# ---------------------------------------------------------------------------
# Path enumeration (the weight / output layout contract)
# ---------------------------------------------------------------------------

Path = Tuple[int, int, int, bool]  # (l1, l2, lo, swapped)


def enumerate_paths(in1_l_max: int, in2_l_max: int, out_l_max: int, symmetric: bool) -> List[Path]:
    """Paths in weight order: for each lo, canonical (l1>=l2, l1 from in1) then swapped.

    A swapped path (l1 > l2) takes l1 from in2 and l2 from in1 and evaluates the
    canonical contraction with the operands exchanged (reference
    ``src/flashcart/o3/utils.py:157-203``; ``_codegen_tensor_product.py:596-622,964-983``).
    """
    paths: List[Path] = []
    lp = max(in1_l_max, in2_l_max)
    for lo in range(out_l_max + 1):
        for l1 in range(lp + 1):
            for l2 in range(l1 + 1):
                if path_allowed(l1, l2, lo) and l1 <= in1_l_max and l2 <= in2_l_max:
                    paths.append((l1, l2, lo, False))
        if not symmetric:
            for l1 in range(lp + 1):
                for l2 in range(l1):
                    if path_allowed(l1, l2, lo) and l1 <= in2_l_max and l2 <= in1_l_max:
                        paths.append((l1, l2, lo, True))
    return paths


def count_output_paths(in1_l_max: int, in2_l_max: int, out_l_max: int, symmetric: bool = False):
    """Per-output-rank path counts and their total."""
    counts = [0] * (out_l_max + 1)
    for _, _, lo, _ in enumerate_paths(in1_l_max, in2_l_max, out_l_max, symmetric):
        counts[lo] += 1
    return counts, sum(counts)


def operand_coefficients(path: Path) -> Dict[Tuple[int, int, int], Fraction]:
    """Coefficients of a path indexed as (out comp, in1 comp, in2 comp).

    For a swapped path the canonical tensor's operand axes are exchanged, so the
    result is always ``out_a = sum B[a, i1, i2] * in1_i1 * in2_i2``.
    """
    l1, l2, lo, swapped = path
    base = tp_coefficients(l1, l2, lo)
    if not swapped:
        return dict(base)
    return {(a, c, b): v for (a, b, c), v in base.items()}


def operand_ranks(path: Path) -> Tuple[int, int]:
    """(rank read from in1, rank read from in2) of a path."""
    l1, l2, _, swapped = path
    return (l2, l1) if swapped else (l1, l2)


# ---------------------------------------------------------------------------
# Eq. (1): expansion polynomials
# ---------------------------------------------------------------------------

X, Y, Z = sp.symbols("x y z", real=True)


def _pairings(slots: Tuple[int, ...]):
    """All perfect matchings of an even-length slot tuple."""
    if not slots:
        yield []
        return
    first, rest = slots[0], slots[1:]
    for i, partner in enumerate(rest):
        for sub in _pairings(rest[:i] + rest[i + 1:]):
            yield [(first, partner)] + sub


@lru_cache(maxsize=None)
def expansion_polynomials(l: int) -> Tuple[sp.Expr, ...]:
    """Eq. (1) stored components of T^l as SymPy polynomials in x, y, z."""
    from itertools import combinations

    vec = (X, Y, Z)
    pref = sp.Rational(double_factorial(2 * l - 1), math.factorial(l))
    comps = []
    for a, b, c in stored_basis(l):
        idx = (0,) * a + (1,) * b + (2,) * c
        expr = sp.Integer(0)
        for m in range(l // 2 + 1):
            coef = sp.Rational((-1) ** m * double_factorial(2 * l - 2 * m - 1), double_factorial(2 * l - 1))
            placed = sp.Integer(0)
            for vslots in combinations(range(l), l - 2 * m):
                rest = tuple(s for s in range(l) if s not in vslots)
                term = sp.Integer(1)
                for s in vslots:
                    term *= vec[idx[s]]
                for match in _pairings(rest):
                    if all(idx[p] == idx[q] for p, q in match):
                        placed += term
            expr += coef * placed
        comps.append(sp.expand(pref * expr))
    return tuple(comps)


def expansion_dim(l_max: int) -> int:
    return (l_max + 1) ** 2
