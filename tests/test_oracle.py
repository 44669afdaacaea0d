"""Pin the CPU oracle against known answers (no GPU).

Each oracle function gets a check that a plausible slip (wrong normalization, a
transposed operand, a dropped trace term, a wrong index) would fail:
* tensor product: the reference's einsum closed forms for the 15 canonical l<=3
  paths (reference tests/o3/test_codegen_tensor_product.py:101-202), evaluated on
  full Cartesian tensors built with the exact tracelessness recursion; rotation
  equivariance of every path; output symmetric and traceless;
* expansion: explicit l<=3 polynomials, T^l(r).r^(x)l == 1 on the sphere (fixes
  normalization and tracelessness together), rotation equivariance;
* radial: numpy chebvander (reference tests/nn/test_radial.py:35-46), the cutoff
  closed form and its value/derivative conditions at r_max (tests/nn/test_radial.py:8-31),
  the Bessel closed form;
* linear: an explicit per-rank loop;
* model: rotation/translation/permutation invariance, forces = -dE/dR by central
  finite differences, batched == per-structure (reference tests/model/test_flashcart.py:43-167).
"""

import itertools
import math

import numpy as np
import pytest
import torch

from flashcart_amd.codegen.cartesian import reconstruction
from oracle import cartesian as OC
from oracle import ops as O

DT = torch.float64


def _rec_matrix(l):
    M = np.zeros((3 ** l, 2 * l + 1))
    for f, idx in enumerate(itertools.product(range(3), repeat=l)):
        for k, v in reconstruction(l)[idx].items():
            M[f, k] = v
    return torch.as_tensor(M, dtype=DT)


def _full(l, stored):  # stored (n, 2l+1) -> (n, 3,..,3)
    if l == 0:
        return stored[:, 0]
    return (stored @ _rec_matrix(l).T).reshape(stored.shape[0], *([3] * l))


def _stored(l, full):
    if l == 0:
        return full.reshape(-1, 1)
    sel = [OC.full_index(abc) for abc in OC.STORED[l]]
    return full.reshape(full.shape[0], -1)[:, sel]


def _einsum_closed_form(l1, l2, lo, A, B):
    eye = torch.eye(3, dtype=DT)
    if lo == 0:
        norm = {0: 1.0, 1: 1.0, 2: 2.0 / 3.0, 3: 2.0 / 5.0}[l1]
        sub = {0: "a,a->a", 1: "ai,ai->a", 2: "aij,aij->a", 3: "aijk,aijk->a"}[l1]
        return norm * torch.einsum(sub, A, B)
    key = (l1, l2, lo)
    if key == (1, 0, 1):
        return torch.einsum("ai,a->ai", A, B)
    if key == (2, 1, 1):
        return torch.einsum("aij,aj->ai", A, B)
    if key == (3, 2, 1):
        return (2.0 / 3.0) * torch.einsum("aijk,ajk->ai", A, B)
    if key in ((1, 1, 2), (3, 3, 2)):
        sub = "ai,aj->aij" if key == (1, 1, 2) else "aijk,ajkl->ail"
        xy = torch.einsum(sub, A, B)
        xy = xy + xy.transpose(1, 2)
        z = torch.einsum("ai,ai->a" if key == (1, 1, 2) else "aijk,aijk->a", A, B)
        return 0.75 * (xy - (2.0 / 3.0) * torch.einsum("a,ij->aij", z, eye))
    if key == (2, 0, 2):
        return torch.einsum("aij,a->aij", A, B)
    if key == (2, 2, 2):
        xy = torch.einsum("aij,ajk->aik", A, B)
        xy = xy + xy.transpose(1, 2)
        z = torch.einsum("aij,aij->a", A, B)
        return xy - (2.0 / 3.0) * torch.einsum("a,ij->aij", z, eye)
    if key == (3, 1, 2):
        return torch.einsum("aijk,ak->aij", A, B)
    if key in ((2, 1, 3), (3, 2, 3)):
        if key == (2, 1, 3):
            xy, z, c = torch.einsum("aij,ak->aijk", A, B), torch.einsum("aij,aj->ai", A, B), 5.0 / 9.0
        else:
            xy, z, c = torch.einsum("aijk,akl->aijl", A, B), torch.einsum("aijk,ajk->ai", A, B), 5.0 / 6.0
        xy = xy + xy.permute(0, 2, 3, 1) + xy.permute(0, 3, 1, 2)
        ze = torch.einsum("ai,jk->aijk", z, eye)
        ze = ze + ze.permute(0, 2, 3, 1) + ze.permute(0, 3, 1, 2)
        return c * (xy - 0.4 * ze)
    if key == (3, 0, 3):
        return torch.einsum("aijk,a->aijk", A, B)
    raise KeyError(key)


CANONICAL = [(0, 0, 0), (1, 1, 0), (2, 2, 0), (3, 3, 0), (1, 0, 1), (2, 1, 1), (3, 2, 1), (2, 0, 2), (1, 1, 2),
             (2, 2, 2), (3, 3, 2), (3, 1, 2), (3, 0, 3), (2, 1, 3), (3, 2, 3)]


def _path_eval(l1, l2, lo, x, y):
    return torch.einsum("abc,nb,nc->na", torch.as_tensor(OC.path_tensor(l1, l2, lo), dtype=DT), x, y)


@pytest.mark.parametrize("path", CANONICAL, ids=lambda p: f"{p[0]}{p[1]}{p[2]}")
def test_tp_path_matches_einsum_closed_form(path):
    l1, l2, lo = path
    g = torch.Generator().manual_seed(sum(path) * 31 + l1)
    x = torch.randn(5, 2 * l1 + 1, dtype=DT, generator=g)
    y = torch.randn(5, 2 * l2 + 1, dtype=DT, generator=g)
    want = _stored(lo, _einsum_closed_form(l1, l2, lo, _full(l1, x), _full(l2, y)))
    got = _path_eval(l1, l2, lo, x, y)
    assert torch.allclose(got, want, atol=1e-11, rtol=0), (got - want).abs().max()


def _random_rotation(seed):
    g = torch.Generator().manual_seed(seed)
    q, r = torch.linalg.qr(torch.randn(3, 3, dtype=DT, generator=g))
    q = q * torch.sign(torch.diagonal(r))
    if torch.det(q) < 0:
        q[:, 0] = -q[:, 0]
    return q


def _rotate(l, stored, R):
    if l == 0:
        return stored
    T = _full(l, stored)
    for ax in range(1, l + 1):
        T = torch.movedim(torch.tensordot(T, R, dims=([ax], [1])), -1, ax)
    return _stored(l, T)


ALL_PATHS = [(a, b, c) for a in range(4) for b in range(a + 1) for c in range(4) if OC.allowed(a, b, c)]
# rank-4 paths (the kernels of a FLASHCART_KERNEL_L_MAX=4 build): every canonical path with a rank 4
RANK4_PATHS = [(a, b, c) for a in range(5) for b in range(a + 1) for c in range(5)
               if OC.allowed(a, b, c) and 4 in (a, b, c)]


@pytest.mark.parametrize("path", ALL_PATHS + RANK4_PATHS, ids=lambda p: f"{p[0]}{p[1]}{p[2]}")
def test_tp_path_rotation_equivariant_and_traceless(path):
    l1, l2, lo = path
    R = _random_rotation(7)
    g = torch.Generator().manual_seed(3)
    x = torch.randn(4, 2 * l1 + 1, dtype=DT, generator=g)
    y = torch.randn(4, 2 * l2 + 1, dtype=DT, generator=g)
    a = _path_eval(l1, l2, lo, _rotate(l1, x, R), _rotate(l2, y, R))
    b = _rotate(lo, _path_eval(l1, l2, lo, x, y), R)
    assert torch.allclose(a, b, atol=1e-10)
    # the full output reconstructed from the stored entries must be the one the projector built
    full = OC.stf_projector(lo)
    if lo >= 2:
        out = _full(lo, _path_eval(l1, l2, lo, x, y)).reshape(4, -1)
        assert torch.allclose(out @ torch.as_tensor(full, dtype=DT).T, out, atol=1e-10)


def test_exchanged_paths_are_operand_swaps():
    """A swapped path (l1 from in2) evaluates the canonical contraction with exchanged operands."""
    g = torch.Generator().manual_seed(0)
    for l1, l2, lo in [(1, 0, 1), (2, 1, 1), (3, 2, 1), (3, 1, 2), (2, 1, 3), (3, 2, 3)]:
        x = torch.randn(3, 2 * l1 + 1, dtype=DT, generator=g)
        y = torch.randn(3, 2 * l2 + 1, dtype=DT, generator=g)
        in1 = torch.cat([torch.zeros(3, l2 * l2, dtype=DT), y, torch.zeros(3, 16 - (l2 + 1) ** 2, dtype=DT)], 1)
        in2 = torch.cat([torch.zeros(3, l1 * l1, dtype=DT), x, torch.zeros(3, 16 - (l1 + 1) ** 2, dtype=DT)], 1)
        paths = OC.enumerate_paths(3, 3, 3, False)
        p = paths.index((l1, l2, lo, True))
        w = torch.zeros(3, len(paths), dtype=DT)
        w[:, p] = 1.0
        out = O.tensor_product(in1, in2, w, None, None, 3, 3, 3, 1, 1)
        per = [sum(1 for q in paths if q[2] == l) for l in range(4)]
        off = sum((2 * l + 1) * per[l] for l in range(lo))
        q = sum(1 for t in paths[:p] if t[2] == lo)
        block = out[:, off:off + (2 * lo + 1) * per[lo]].reshape(3, 2 * lo + 1, per[lo])[:, :, q]
        assert torch.allclose(block, _path_eval(l1, l2, lo, x, y), atol=1e-12)


def test_expansion_closed_forms():
    r = torch.tensor([[0.3, -0.5, 0.2], [1.0, 2.0, -0.7]], dtype=DT)
    x, y, z = r[:, 0], r[:, 1], r[:, 2]
    got = O.irreps(r, 3)
    want = torch.stack([
        torch.ones_like(x), x, y, z,
        1.5 * x * x - 0.5, 1.5 * y * y - 0.5, 1.5 * x * y, 1.5 * x * z, 1.5 * y * z,
        2.5 * x ** 3 - 1.5 * x, 2.5 * x * x * y - 0.5 * y, 2.5 * x * x * z - 0.5 * z, 2.5 * x * y * y - 0.5 * x,
        2.5 * x * y * z, 2.5 * y * y * z - 0.5 * z, 2.5 * y ** 3 - 1.5 * y,
    ], dim=1)
    assert torch.allclose(got, want, atol=1e-14)


@pytest.mark.parametrize("path", RANK4_PATHS, ids=lambda p: f"{p[0]}{p[1]}{p[2]}")
def test_rank4_paths_match_exact_derivation(path):
    """The oracle's numeric path tensors (SVD projectors over the 3^l spaces) against the exact
    rational coefficients of the HIP code generator (flashcart_amd/codegen/cartesian.py): two
    independent routes to the same Eq. (2) coefficients, at the ranks no golden vector covers."""
    from flashcart_amd.codegen.cartesian import tp_coefficients
    l1, l2, lo = path
    B = OC.path_tensor(l1, l2, lo)
    exact = np.zeros_like(B)
    for (a, b, c), v in tp_coefficients(l1, l2, lo).items():
        exact[a, b, c] = float(v)
    assert np.abs(B - exact).max() <= 1e-12 * max(1.0, np.abs(exact).max())


def test_rank4_expansion_legendre_components():
    """On unit vectors the all-x and all-y components of Eq. (1) are Legendre polynomials:
    P_4(x) = (35 x^4 - 30 x^2 + 3) / 8 (as 1.5 x^2 - 0.5 and 2.5 x^3 - 1.5 x are P_2, P_3 above);
    stored order of rank 4: (4,0,0) first, (0,4,0) fifth."""
    g = torch.Generator().manual_seed(4)
    r = torch.randn(40, 3, dtype=DT, generator=g)
    r = r / r.norm(dim=1, keepdim=True)
    T4 = O.irreps(r, 4)[:, 16:25]

    def p4(t):
        return (35 * t ** 4 - 30 * t ** 2 + 3) / 8

    assert torch.allclose(T4[:, 0], p4(r[:, 0]), atol=1e-13)
    assert torch.allclose(T4[:, 4], p4(r[:, 1]), atol=1e-13)


@pytest.mark.parametrize("l", [1, 2, 3, 4])
def test_expansion_normalised_and_traceless_on_sphere(l):
    g = torch.Generator().manual_seed(l)
    r = torch.randn(50, 3, dtype=DT, generator=g)
    r = r / r.norm(dim=1, keepdim=True)
    T = O.irreps(r, l)[:, l * l:(l + 1) ** 2]
    full = _full(l, T)
    rr = r
    for _ in range(l - 1):
        rr = torch.einsum("n...,nk->n...k", rr, r)
    assert torch.allclose((full * rr).reshape(50, -1).sum(1), torch.ones(50, dtype=DT), atol=1e-12)
    R = _random_rotation(l)
    assert torch.allclose(O.irreps(r @ R.T, l)[:, l * l:], _rotate(l, T, R), atol=1e-12)


@pytest.mark.parametrize("mapping", ["affine", "cosine"])
@pytest.mark.parametrize("n_radial", [1, 5, 8])
def test_chebyshev_matches_numpy(mapping, n_radial):
    r = torch.linspace(0.5, 4.0, 33, dtype=DT)
    t = ((r - 0.5) / 3.5).numpy()
    x = np.cos(t * np.pi) if mapping == "cosine" else 2 * t - 1
    want = np.polynomial.chebyshev.chebvander(x, n_radial - 1)
    assert np.allclose(O.chebyshev(r, n_radial, 4.0, 0.5, mapping).numpy(), want, atol=1e-12)


@pytest.mark.parametrize("p", [3, 4, 5, 6])
def test_cutoff_closed_form_and_smoothness(p):
    r = torch.cat([torch.linspace(0.0, 4.0 - 1e-6, 101, dtype=DT), torch.tensor([4.0, 4.5, 8.0], dtype=DT)])
    x = (r / 4.0).numpy()
    poly = 1 - (p + 1) * (p + 2) / 2 * x ** p + p * (p + 2) * x ** (p + 1) - p * (p + 1) / 2 * x ** (p + 2)
    want = np.clip(poly * (r.numpy() < 4.0), 0, 1)
    assert np.allclose(O.cutoff(r, 4.0, p).numpy(), want, atol=1e-12)
    # value, first and second derivative vanish at the cutoff
    s = torch.tensor([4.0 - 1e-4], dtype=DT, requires_grad=True)
    e = O.cutoff(s, 4.0, p)
    (d1,) = torch.autograd.grad(e.sum(), s, create_graph=True)
    (d2,) = torch.autograd.grad(d1.sum(), s)
    assert abs(float(e)) < 1e-9 and abs(float(d1)) < 1e-5 and abs(float(d2)) < 0.1


def test_bessel_closed_form():
    r = torch.linspace(0.1, 5.0, 40, dtype=DT)
    n = torch.arange(1, 9, dtype=DT)
    want = math.sqrt(2 / 5.0) * torch.sin(n * math.pi * r.unsqueeze(-1) / 5.0) / r.unsqueeze(-1)
    assert torch.allclose(O.bessel(r, 8, 5.0), want, atol=1e-12)


def test_linear_matches_loop():
    g = torch.Generator().manual_seed(0)
    paths = [1, 2, 3]
    fin, fout = 3, 4
    x = torch.randn(6, sum((2 * l + 1) * fin * paths[l] for l in range(3)), dtype=DT, generator=g)
    ws = [torch.randn(fout, fin * paths[l], dtype=DT, generator=g) for l in range(3)]
    got = O.linear(x, ws, 2, 3, fin, fout, paths)
    off, cols = 0, []
    for l in range(3):
        k = fin * paths[l]
        s = k ** -0.5
        for m in range(2 * l + 1):
            xv = x[:, off + m * k: off + (m + 1) * k]
            cols.append(torch.stack([(xv * ws[l][o]).sum(1) * s for o in range(fout)], 1))
        off += (2 * l + 1) * k
    cols.append(torch.zeros(6, 7 * fout, dtype=DT))
    assert torch.allclose(got, torch.cat(cols, 1), atol=1e-12)
