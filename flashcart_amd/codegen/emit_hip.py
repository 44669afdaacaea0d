"""Emit HIP C++ device code from the exact Cartesian derivation.

Run at build time (``python -m flashcart_amd.codegen.emit_hip <out_dir>``). It writes

* ``fc_tp_paths.h``: one ``TPPath<R1,R2,LO>`` specialisation per ordered rank triple
  (rank read from in1, rank read from in2, output rank) with straight-line,
  fully unrolled polynomial code for the forward product and both vector-Jacobian
  products, plus the per-edge "A-matrix" form used by the convolution kernels
  (A[a][b] = sum_c B[a,b,c] y_c for an edge-uniform second operand).
* ``fc_expand_poly.h``: Eq. (1) components of ranks 0..L_MAX and their gradients.

This replaces the reference's SymPy -> Triton/PyTorch source emitters
(reference ``src/flashcart/o3/_codegen_tensor_product.py:833-1012,3524-3636`` and
``src/flashcart/o3/_codegen_irreps.py:426-505``): the mathematics is the same, the
target is CDNA4 device code compiled ahead of time by hipcc.
"""

from __future__ import annotations

import os
import sys
from fractions import Fraction
from typing import Dict, List, Tuple

import numpy as np
import sympy as sp

from flashcart_amd.codegen.cartesian import (
    X, Y, Z, expansion_polynomials, path_allowed, tp_coefficients,
)

KERNEL_L_MAX = 3


def flit(v) -> str:
    """Float literal of the float32 value nearest to an exact rational/float."""
    f = np.float32(float(Fraction(v)) if not isinstance(v, float) else v)
    s = np.format_float_scientific(f, unique=True, trim="-")
    if "e" in s:
        mant, exp = s.split("e")
        if "." not in mant:
            mant += ".0"
        s = f"{mant}e{exp}"
    elif "." not in s:
        s += ".0"
    return s + "f"


def ordered_triples(l_max: int) -> List[Tuple[int, int, int]]:
    """All (r1, r2, lo) with r1, r2, lo <= l_max that satisfy the selection rule."""
    return [(r1, r2, lo) for r1 in range(l_max + 1) for r2 in range(l_max + 1)
            for lo in range(l_max + 1) if path_allowed(r1, r2, lo)]


def triple_coefficients(r1: int, r2: int, lo: int) -> Dict[Tuple[int, int, int], Fraction]:
    """B[a, b1, b2] with b1 indexing the in1 operand (rank r1), b2 the in2 operand (rank r2).

    The product is symmetric under operand exchange (Sym removes the order of the
    free indices and both inputs are symmetric), so (r1, r2) with r1 < r2 reuses the
    canonical (r2, r1) tensor with the operand axes exchanged. That is exactly how
    the reference evaluates a "swapped" path.
    """
    if r1 >= r2:
        return dict(tp_coefficients(r1, r2, lo))
    return {(a, c, b): v for (a, b, c), v in tp_coefficients(r2, r1, lo).items()}


def _sum_terms(terms: List[Tuple[Fraction, str]]) -> str:
    """Render sum(coef * expr) with fmaf chains, coefficients folded as float literals."""
    if not terms:
        return "0.0f"
    out = None
    for coef, expr in terms:
        if coef == 1:
            cur = expr
            out = cur if out is None else f"({out} + {cur})"
        elif coef == -1:
            out = f"(-{expr})" if out is None else f"({out} - {expr})"
        else:
            out = f"({flit(coef)} * {expr})" if out is None else f"fmaf({flit(coef)}, {expr}, {out})"
    return out


def emit_triple(r1: int, r2: int, lo: int) -> str:
    B = triple_coefficients(r1, r2, lo)
    n1, n2, no = 2 * r1 + 1, 2 * r2 + 1, 2 * lo + 1
    # structural A entries: (a, b1) -> [(coef, b2)]
    amap: Dict[Tuple[int, int], List[Tuple[Fraction, int]]] = {}
    for (a, b1, b2), v in sorted(B.items()):
        amap.setdefault((a, b1), []).append((v, b2))
    a_entries = sorted(amap)
    L: List[str] = []
    L.append(f"template <> struct TPPath<{r1}, {r2}, {lo}> {{")
    L.append(f"  static constexpr int N1 = {n1}, N2 = {n2}, NO = {no}, NNZ = {len(B)}, NA = {len(a_entries)};")
    # --- direct forward: o[a] = sum_b1 x[b1] * (sum_b2 B y[b2])
    L.append("  __device__ static __forceinline__ void fwd(const float* __restrict__ x, const float* __restrict__ y, float* __restrict__ o) {")
    for a in range(no):
        terms = []
        for (aa, b1) in a_entries:
            if aa != a:
                continue
            inner = _sum_terms([(c, f"y[{b2}]") for c, b2 in amap[(aa, b1)]])
            terms.append((Fraction(1), f"x[{b1}] * {inner}"))
        L.append(f"    o[{a}] = {_sum_terms(terms)};")
    L.append("  }")
    # --- A-matrix from the in2 operand: A[k] for k over structural (a, b1) entries
    L.append("  __device__ static __forceinline__ void amat(const float* __restrict__ y, float* __restrict__ A) {")
    for k, key in enumerate(a_entries):
        L.append(f"    A[{k}] = {_sum_terms([(c, f'y[{b2}]') for c, b2 in amap[key]])};")
    L.append("  }")
    # --- t[a] = sum_b1 A[a,b1] x[b1]
    L.append("  __device__ static __forceinline__ void apply(const float* __restrict__ A, const float* __restrict__ x, float* __restrict__ t) {")
    for a in range(no):
        ks = [(k, b1) for k, (aa, b1) in enumerate(a_entries) if aa == a]
        L.append(f"    t[{a}] = {_sum_terms([(Fraction(1), f'A[{k}] * x[{b1}]') for k, b1 in ks])};")
    L.append("  }")
    # --- m[b1] += sum_a A[a,b1] u[a]
    L.append("  __device__ static __forceinline__ void apply_t(const float* __restrict__ A, const float* __restrict__ u, float* __restrict__ m) {")
    for b1 in range(n1):
        ks = [(k, a) for k, (a, bb) in enumerate(a_entries) if bb == b1]
        if ks:
            body = "m[%d]" % b1
            for k, a in ks:
                body = f"fmaf(A[{k}], u[{a}], {body})"
            L.append(f"    m[{b1}] = {body};")
    L.append("  }")
    # --- gy[b2] += sum_{a,b1} B u[a] x[b1]
    L.append("  __device__ static __forceinline__ void vjp2(const float* __restrict__ u, const float* __restrict__ x, float* __restrict__ gy) {")
    by2: Dict[int, Dict[int, List[Tuple[Fraction, int]]]] = {}
    for (a, b1, b2), v in sorted(B.items()):
        by2.setdefault(b2, {}).setdefault(a, []).append((v, b1))
    for b2 in sorted(by2):
        terms = []
        for a, lst in sorted(by2[b2].items()):
            inner = _sum_terms([(c, f"x[{b1}]") for c, b1 in lst])
            terms.append((Fraction(1), f"u[{a}] * {inner}"))
        L.append(f"    gy[{b2}] += {_sum_terms(terms)};")
    L.append("  }")
    # --- gx[b1] += sum_{a,b2} B u[a] y[b2]
    L.append("  __device__ static __forceinline__ void vjp1(const float* __restrict__ u, const float* __restrict__ y, float* __restrict__ gx) {")
    by1: Dict[int, Dict[int, List[Tuple[Fraction, int]]]] = {}
    for (a, b1, b2), v in sorted(B.items()):
        by1.setdefault(b1, {}).setdefault(a, []).append((v, b2))
    for b1 in sorted(by1):
        terms = []
        for a, lst in sorted(by1[b1].items()):
            inner = _sum_terms([(c, f"y[{b2}]") for c, b2 in lst])
            terms.append((Fraction(1), f"u[{a}] * {inner}"))
        L.append(f"    gx[{b1}] += {_sum_terms(terms)};")
    L.append("  }")
    L.append("};")
    return "\n".join(L)


def emit_tp_header(l_max: int = KERNEL_L_MAX) -> str:
    parts = [
        "// Generated by flashcart_amd/codegen/emit_hip.py -- do not edit.",
        "// Exact Eq. (2) coefficients of every ordered rank triple, rounded once to float32.",
        "#pragma once",
        f"#define FC_KERNEL_L_MAX {l_max}",
        "namespace fc {",
        "template <int R1, int R2, int LO> struct TPPath;",
    ]
    for t in ordered_triples(l_max):
        parts.append(emit_triple(*t))
    parts.append("}  // namespace fc")
    return "\n".join(parts) + "\n"


def _c_expr(expr: sp.Expr) -> str:
    """Render a polynomial in x, y, z as C with float literals."""
    expr = sp.expand(expr)
    if expr == 0:
        return "0.0f"
    terms = []
    for mon, coef in sp.Poly(expr, X, Y, Z).terms():
        factors = []
        for sym, p in zip(("x", "y", "z"), mon):
            factors += [sym] * p
        body = "*".join(factors) if factors else None
        c = Fraction(int(coef.p), int(coef.q))
        if body is None:
            terms.append(flit(c))
        elif c == 1:
            terms.append(body)
        elif c == -1:
            terms.append(f"-{body}")
        else:
            terms.append(f"{flit(c)}*{body}")
    return " + ".join(terms).replace("+ -", "- ")


def emit_expand_header(l_max: int = KERNEL_L_MAX) -> str:
    L = [
        "// Generated by flashcart_amd/codegen/emit_hip.py -- do not edit.",
        "// Eq. (1) stored components of ranks 0..L and their polynomial gradients.",
        "#pragma once",
        f"#define FC_KERNEL_L_MAX {l_max}",
        "namespace fc {",
        "template <int L> struct Expand;",
    ]
    for l in range(l_max + 1):
        polys = expansion_polynomials(l)
        L.append(f"template <> struct Expand<{l}> {{")
        L.append(f"  static constexpr int N = {2 * l + 1};")
        L.append("  __device__ static __forceinline__ void fwd(float x, float y, float z, float* __restrict__ t) {")
        for a, p in enumerate(polys):
            L.append(f"    t[{a}] = {_c_expr(p)};")
        L.append("  }")
        L.append("  // g[3] += sum_a gt[a] * dT_a/d(x,y,z)")
        L.append("  __device__ static __forceinline__ void bwd(float x, float y, float z, const float* __restrict__ gt, float* __restrict__ g) {")
        for k, s in enumerate((X, Y, Z)):
            terms = []
            for a, p in enumerate(polys):
                d = sp.diff(p, s)
                if d != 0:
                    terms.append(f"gt[{a}] * ({_c_expr(d)})")
            if terms:
                L.append(f"    g[{k}] += " + " + ".join(terms) + ";")
        L.append("  }")
        # second-order helpers (training): directional derivative and Hessian-vector product
        L.append("  // dt[a] = sum_j dT_a/du_j du_j")
        L.append("  __device__ static __forceinline__ void jvp(float x, float y, float z, const float* __restrict__ du, "
                 "float* __restrict__ dt) {")
        for a, p in enumerate(polys):
            terms = [f"du[{j}] * ({_c_expr(sp.diff(p, s))})" for j, s in enumerate((X, Y, Z)) if sp.diff(p, s) != 0]
            L.append(f"    dt[{a}] = " + (" + ".join(terms) if terms else "0.0f") + ";")
        L.append("  }")
        L.append("  // h[i] += sum_a gt[a] sum_j d2T_a/(du_i du_j) du[j]")
        L.append("  __device__ static __forceinline__ void hvp(float x, float y, float z, const float* __restrict__ gt, "
                 "const float* __restrict__ du, float* __restrict__ h) {")
        for i, si in enumerate((X, Y, Z)):
            terms = []
            for a, p in enumerate(polys):
                for j, sj in enumerate((X, Y, Z)):
                    d2 = sp.diff(p, si, sj)
                    if d2 != 0:
                        terms.append(f"gt[{a}] * du[{j}] * ({_c_expr(d2)})")
            if terms:
                L.append(f"    h[{i}] += " + " + ".join(terms) + ";")
        L.append("  }")
        L.append("};")
    L.append("}  // namespace fc")
    return "\n".join(L) + "\n"


def write_all(out_dir: str, l_max: int = KERNEL_L_MAX) -> List[str]:
    """Write both headers for ranks 0..l_max (3: the default library; 4: the library built with
    FLASHCART_KERNEL_L_MAX=4), rewriting a file only when its text changes."""
    os.makedirs(out_dir, exist_ok=True)
    written = []
    for name, text in (("fc_tp_paths.h", emit_tp_header(l_max)), ("fc_expand_poly.h", emit_expand_header(l_max))):
        path = os.path.join(out_dir, name)
        old = open(path).read() if os.path.exists(path) else None
        if old != text:
            with open(path + ".tmp", "w") as fh:
                fh.write(text)
            os.replace(path + ".tmp", path)
        written.append(path)
    return written


if __name__ == "__main__":
    out = sys.argv[1] if len(sys.argv) > 1 else os.path.join(os.path.dirname(__file__), "..", "csrc", "generated")
    for p in write_all(out, int(sys.argv[2]) if len(sys.argv) > 2 else KERNEL_L_MAX):
        print(p)
