"""CPU checks of the torch statements used for second derivatives of the standalone ops.

``flashcart_amd.o3._torch_math`` restates Eq. (1), the radial bases, the envelope and the RMS
norm's mean invariant so autograd can differentiate the first backward of the standalone
ops (and route gradients of auxiliary outputs). Here each statement is compared in float64
with the oracle's (values, first and second derivatives), and the double-vjp helper with
plain nested autograd. The statements use the kernels' forms (the factored envelope, the
rank-0 metric of the RMS norm), so agreement with the oracle's textbook forms pins them.
"""

import math

import pytest
import torch

from flashcart_amd import _lib
from flashcart_amd.o3 import _torch_math as M
from oracle import model as OM
from oracle import ops as O


def _hvp(fn, x, seed):
    """(value, gradient, Hessian-vector product) of sum(r * fn(x)) for fixed random r, v."""
    g = torch.Generator().manual_seed(seed)
    x = x.detach().clone().requires_grad_(True)
    y = fn(x)
    r = torch.randn(y.shape, generator=g, dtype=y.dtype)
    (gx,) = torch.autograd.grad((y * r).sum(), x, create_graph=True)
    v = torch.randn(x.shape, generator=g, dtype=x.dtype)
    h = None
    if gx.requires_grad:  # a linear map has a constant gradient
        (h,) = torch.autograd.grad((gx * v).sum(), x, allow_unused=True)
    return y.detach(), gx.detach(), (torch.zeros_like(x) if h is None else h)


def _same(a, b, what):
    for k, (p, q) in enumerate(zip(a, b)):
        scale = float(q.abs().max()) + 1e-30
        assert float((p - q).abs().max()) <= 1e-11 * max(scale, 1.0), f"{what}[{k}]"


@pytest.mark.parametrize("l_max", [1, 2, 3])
def test_expansion_matches_oracle(l_max):
    x = torch.randn(50, 3, dtype=torch.float64, generator=torch.Generator().manual_seed(l_max))
    _same(_hvp(lambda t: M.expansion(t, l_max), x, 1), _hvp(lambda t: O.irreps(t, l_max), x, 1), "expansion")


@pytest.mark.parametrize("basis", ["affine", "cosine", "bessel"])
def test_radial_basis_matches_oracle(basis):
    code = {"affine": _lib.BASIS_CHEBYSHEV_AFFINE, "cosine": _lib.BASIS_CHEBYSHEV_COSINE,
            "bessel": _lib.BASIS_BESSEL}[basis]
    d = 0.3 + 4.5 * torch.rand(64, dtype=torch.float64, generator=torch.Generator().manual_seed(2))

    def ref(t):
        return O.bessel(t, 8, 5.0) if basis == "bessel" else O.chebyshev(t, 8, 5.0, 0.2, basis)

    r_min = 0.0 if basis == "bessel" else 0.2
    _same(_hvp(lambda t: M.radial_basis(t, code, 8, r_min, 5.0), d, 3), _hvp(ref, d, 3), "radial")


@pytest.mark.parametrize("p", [3, 6, 8])
def test_envelope_matches_oracle(p):
    # inside the cutoff, beyond it, and negative distances (clamped)
    d = torch.cat([torch.linspace(-0.5, 4.99, 97, dtype=torch.float64), torch.tensor([5.3, 6.0], dtype=torch.float64)])
    a = _hvp(lambda t: M.envelope(t, 5.0, p), d, 4)
    b = _hvp(lambda t: O.cutoff(t, 5.0, p), d, 4)
    for k, (x, y) in enumerate(zip(a, b)):
        # the expanded form cancels near the cutoff: compare with an absolute bar
        assert float((x - y).abs().max()) <= 1e-9 * (1 + float(y.abs().max())), f"envelope[{k}]"


@pytest.mark.parametrize("l_max,C", [(1, 4), (2, 8), (3, 4)])
def test_rms_mean_matches_oracle(l_max, C):
    """The mean invariant through the (l, l, 0) metric, used to route gradients of the
    norm's scale output: the norm built on it equals the oracle's (TP-based) norm."""
    g = torch.Generator().manual_seed(l_max)
    w = 1.0 + 0.2 * torch.randn(l_max + 1, C, dtype=torch.float64, generator=g)
    x = torch.randn(6, (l_max + 1) ** 2 * C, dtype=torch.float64, generator=g)
    sd = {f"n.weights.{l}": w[l] for l in range(l_max + 1)}
    gain = torch.cat([w[l].repeat(2 * l + 1) for l in range(l_max + 1)]).view(1, -1)

    def mine(t):
        return t * torch.rsqrt(M.rms_mean(t, l_max, C) + 1e-6).unsqueeze(-1) * gain

    _same(_hvp(mine, x, 7), _hvp(lambda t: OM.rms_norm(sd, "n", t, l_max, C, 1e-6), x, 7), "rms")


def test_silu_derivatives():
    x = torch.linspace(-6, 6, 101, dtype=torch.float64).requires_grad_(True)
    y = O.silu(x)
    (d1,) = torch.autograd.grad(y.sum(), x, create_graph=True)
    (d2,) = torch.autograd.grad(d1.sum(), x)
    assert torch.allclose(M.silu_grad(x.detach()), d1.detach(), atol=1e-13)
    assert torch.allclose(M.silu_grad2(x.detach()), d2, atol=1e-13)


def test_vjp_of_vjp_matches_nested_autograd():
    """<c, d<g, f(x, w)>/dx> differentiated wrt x, w and g, against nested autograd."""
    gen = torch.Generator().manual_seed(1)
    x = torch.randn(7, 3, dtype=torch.float64, generator=gen)
    w = torch.randn(3, 4, dtype=torch.float64, generator=gen)
    gout = torch.randn(7, 4, dtype=torch.float64, generator=gen)
    c = torch.randn(7, 3, dtype=torch.float64, generator=gen)

    def f(a, b):
        return torch.tanh(a @ b) * a.sum(-1, keepdim=True)

    with torch.no_grad():  # as inside a backward pass without create_graph
        gp, gg = M.vjp_of_vjp(f, [x, w], [0], [gout], [c], [True, True], [True])
    with pytest.raises(NotImplementedError):  # a third derivative is refused, not silently wrong
        M.vjp_of_vjp(f, [x, w], [0], [gout], [c], [True, True], [True])
    xx, ww, go = (t.clone().requires_grad_(True) for t in (x, w, gout))
    (gx,) = torch.autograd.grad((f(xx, ww) * go).sum(), xx, create_graph=True)
    want = torch.autograd.grad((gx * c).sum(), [xx, ww, go])
    for a, b in zip(gp + gg, want):
        assert torch.allclose(a, b, atol=1e-12)
