"""Differentiable PyTorch statements for second derivatives of the standalone ops.

The forward and first backward of every op run as HIP kernels, and so do the second
derivatives of everything on the model's path. The standalone ``irreps`` (Eq. 1) and
``radial`` (radial basis, envelope) ops differentiate their first backward through the
statements here instead; they run with torch on the tensors' own device, only inside a
second-order backward, like the reference's torch layers (src/flashcart/nn/radial.py).
``rms_mean`` (the RMS norm's mean invariant) and the rescaled-SiLU derivatives serve the
first- and second-order formulas of auxiliary outputs.

Each function evaluates exactly what the matching kernel evaluates (same expressions,
clamps and masks), so first derivatives taken here agree with the kernels' to rounding.
"""

from __future__ import annotations

import math
from functools import lru_cache

import torch

from flashcart_amd import _lib

Tensor = torch.Tensor

SILU_SCALE = 1.6765324703310907  # RescaledSiLULayer, src/flashcart/nn/layers.py:12-45


# ---------------------------------------------------------------------------
# Eq. (1): the stored components of T^l(r) as polynomials in (x, y, z)
# ---------------------------------------------------------------------------

@lru_cache(maxsize=None)
def _expansion_table(l_max: int):
    """(monomial exponents [(a, b, c)], coefficient rows) of every stored component of
    ranks 0..l_max, from the exact polynomials the kernels are generated from."""
    import sympy as sp
    from flashcart_amd.codegen.cartesian import X, Y, Z, expansion_polynomials

    monos = [(a, b, c) for deg in range(l_max + 1) for a in range(deg + 1) for b in range(deg + 1 - a)
             for c in [deg - a - b]]
    index = {m: i for i, m in enumerate(monos)}
    coef = [[0.0] * ((l_max + 1) ** 2) for _ in monos]
    col = 0
    for l in range(l_max + 1):
        for poly in expansion_polynomials(l):
            for exps, v in sp.Poly(poly, X, Y, Z).terms():
                coef[index[tuple(int(e) for e in exps)]][col] = float(v)
            col += 1
    return monos, coef


def expansion(u: Tensor, l_max: int) -> Tensor:
    """(n, (l_max+1)^2) Eq. (1) components of the rows of ``u`` (n, 3) (``irreps_fwd``)."""
    monos, coef = _expansion_table(int(l_max))
    powers = [[torch.ones_like(u[:, k])] for k in range(3)]
    for k in range(3):
        for _ in range(l_max):
            powers[k].append(powers[k][-1] * u[:, k])
    cols = [powers[0][a] * powers[1][b] * powers[2][c] for a, b, c in monos]
    table = torch.tensor(coef, dtype=u.dtype, device=u.device)
    return torch.stack(cols, dim=-1) @ table


# ---------------------------------------------------------------------------
# Radial basis and envelope (flashcart_amd/csrc/fc_expand.hip radial_eval / envelope_eval)
# ---------------------------------------------------------------------------

def radial_basis(d: Tensor, basis: int, n_radial: int, r_min: float, r_max: float) -> Tensor:
    if basis == _lib.BASIS_BESSEL:
        w = (math.pi / r_max) * torch.arange(1, n_radial + 1, dtype=d.dtype, device=d.device)
        return math.sqrt(2.0 / r_max) * w * torch.sinc(d.unsqueeze(-1) * w / math.pi)
    t = (d - r_min) / (r_max - r_min)
    x = torch.cos(t * math.pi) if basis == _lib.BASIS_CHEBYSHEV_COSINE else 2.0 * t - 1.0
    terms = [torch.ones_like(x), x]
    for _ in range(2, n_radial):
        terms.append(2.0 * x * terms[-1] - terms[-2])
    return torch.stack(terms[:n_radial], dim=-1)


def envelope(d: Tensor, r_max: float, poly_order: int) -> Tensor:
    """1 - c1 t^p + c2 t^(p+1) - c3 t^(p+2) in the factored form (1-t)^3 sum_k C(k+2,2) t^k,
    masked beyond r_max and clamped to [0, 1]."""
    dc = torch.clamp(d, min=0.0)
    t = dc / r_max
    g = torch.zeros_like(t)
    for k in range(poly_order - 1, -1, -1):
        g = g * t + 0.5 * (k + 1) * (k + 2)
    s = 1.0 - t
    env = s * s * s * g * (dc < r_max).to(d.dtype)
    return torch.clamp(env, min=0.0, max=1.0)


# ---------------------------------------------------------------------------
# Node-wise layers
# ---------------------------------------------------------------------------

@lru_cache(maxsize=None)
def _rank0_metric(l: int):
    """M_l[b, c]: the (l, l, 0) path's coefficients, inv_l = sum_bc M_l[b, c] x_b x_c."""
    from flashcart_amd.codegen.cartesian import tp_coefficients

    m = [[0.0] * (2 * l + 1) for _ in range(2 * l + 1)]
    for (a, b, c), v in tp_coefficients(l, l, 0).items():
        m[b][c] = float(v)
    return m


def rms_mean(x: Tensor, l_max: int, channels: int) -> Tensor:
    """m[n] = mean_c sum_l inv_l[c] / ((2l+1)(l_max+1))."""
    n = x.shape[0]
    xs = x.reshape(n, -1, channels)
    m = torch.zeros(n, channels, dtype=x.dtype, device=x.device)
    for l in range(l_max + 1):
        xl = xs[:, l * l:(l + 1) ** 2]
        M = torch.tensor(_rank0_metric(l), dtype=x.dtype, device=x.device)
        m = m + (xl * torch.einsum("bc,ncf->nbf", M, xl)).sum(1) / ((2 * l + 1) * (l_max + 1))
    return m.mean(-1)


def silu_grad(pre: Tensor) -> Tensor:
    """d/dx of 1.6765 * x * sigmoid(x)."""
    s = torch.sigmoid(pre)
    return SILU_SCALE * s * (1.0 + pre * (1.0 - s))


def silu_grad2(pre: Tensor) -> Tensor:
    """d^2/dx^2 of 1.6765 * x * sigmoid(x)."""
    s = torch.sigmoid(pre)
    return SILU_SCALE * s * (1.0 - s) * (2.0 + pre * (1.0 - 2.0 * s))


# ---------------------------------------------------------------------------
# Second derivative of a first backward, by differentiating a torch restatement
# ---------------------------------------------------------------------------

def vjp_of_vjp(fn, primals, first_wrt, grad_out, cotangent, need_primals, need_grad_out):
    """Backward of a first-order backward, by differentiating a torch restatement twice.

    The first-order backward returns d<grad_out, fn(*primals)>/d primals[k] for k in
    ``first_wrt``; ``cotangent`` holds one tensor (or None) per such k. Returns the
    gradients of <cotangent, first-order result> with respect to every primal flagged in
    ``need_primals`` and every grad_out entry flagged in ``need_grad_out`` (None where not
    requested or independent).

    The restatement is evaluated on detached copies, so the inner differentiation stays
    inside it and never runs nodes of the caller's graph. The result is therefore not
    differentiable again: a third derivative (this backward under create_graph) raises."""
    if torch.is_grad_enabled():
        raise NotImplementedError("third derivatives of the elementwise layers are not provided "
                                  "(a second-order backward was run with create_graph=True).")
    none = ([None] * len(primals), [None] * len(grad_out))
    with torch.enable_grad():
        ps = [None if p is None else p.detach().requires_grad_(True) for p in primals]
        gos = [None if g is None else g.detach().requires_grad_(True) for g in grad_out]
        outs = fn(*ps)
        if not isinstance(outs, (tuple, list)):
            outs = (outs,)
        pairs = [(o, g) for o, g in zip(outs, gos) if o is not None and g is not None]
        if not pairs:
            return none
        firsts = torch.autograd.grad([o for o, _ in pairs], [ps[k] for k in first_wrt],
                                     [g for _, g in pairs], create_graph=True, allow_unused=True)
        live = [(f, c) for f, c in zip(firsts, cotangent) if f is not None and c is not None]
        sel_p = [k for k, need in enumerate(need_primals) if need and ps[k] is not None]
        sel_g = [k for k, need in enumerate(need_grad_out) if need and gos[k] is not None]
        if not live or not (sel_p or sel_g):
            return none
        res = torch.autograd.grad([f for f, _ in live], [ps[k] for k in sel_p] + [gos[k] for k in sel_g],
                                  [c for _, c in live], allow_unused=True)
    gp = [None] * len(primals)
    gg = [None] * len(grad_out)
    for k, r in zip(sel_p, res[:len(sel_p)]):
        gp[k] = r
    for k, r in zip(sel_g, res[len(sel_p):]):
        gg[k] = r
    return gp, gg
