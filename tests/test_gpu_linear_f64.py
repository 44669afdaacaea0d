"""Float64 equivariant linear maps (``fc_linear_*_f64``) against the float64 oracle.

The reference runs its linear ops in float64 when given float64 tensors (use_fp64,
src/flashcart/o3/_linear.py:328-343; its test tests/o3/test_linear.py:25-60 holds the float64
kernels to 1e-10 of the PyTorch path). Here the bar is 1e-12 relative to the largest entry:
both sides are float64 sums of the same products in different orders.
"""

import pytest
import torch

from oracle import ops as O
from tests.helpers import assert_close

pytestmark = pytest.mark.gpu
DEV = "cuda"
CFGS = [(0, 0, 16, 20, None), (2, 2, 16, 20, None), (3, 3, 32, 16, [3, 5, 5, 4]), (3, 1, 8, 24, [1, 2, 3, 1]),
        (1, 3, 8, 8, None), (2, 0, 4, 8, [2, 3, 1])]


def _close(got, want, what, rel=1e-12):
    assert got.dtype == torch.float64, f"{what}: {got.dtype}"
    want = want.detach().double().cpu()
    assert_close(got, want, 0.0, rel * max(float(want.abs().max()) if want.numel() else 0.0, 1e-300), what)


def _layer(lin, lout, fin, fout, paths, seed):
    from flashcart_amd import o3

    torch.manual_seed(seed)
    return o3.LinearLayer(lin, lout, fin, fout, in_paths=paths).to(DEV, torch.float64)


@pytest.mark.parametrize("cfg", CFGS)
def test_layer_float64(cfg):
    """o3.LinearLayer cast to float64: output, input gradient and weight gradients (the split
    row reduction at n = 3000, one part at n = 37)."""
    lin, lout, fin, fout, paths = cfg
    lay = _layer(lin, lout, fin, fout, paths, 11)
    for n in (37, 3000):
        x = torch.randn(n, lay.in_dim, device=DEV, dtype=torch.float64, requires_grad=True)
        out = lay(x)
        xd = x.detach().cpu().requires_grad_()
        wd = [w.detach().cpu().requires_grad_() for w in lay.weight]
        ref = O.linear(xd, wd, lin, lout, fin, fout, paths)
        _close(out, ref, f"fwd n={n}")
        g = torch.randn_like(out)
        got = torch.autograd.grad(out, [x] + list(lay.weight), g)
        want = torch.autograd.grad(ref, [xd] + wd, g.cpu())
        for k, (a, b) in enumerate(zip(got, want)):
            _close(a, b, f"grad {k} n={n}")


def test_gradcheck_float64():
    """Finite differences through the HIP path (float64 is what gradcheck needs): input and
    weights of a map with paths, unequal ranks and a residual."""
    lay = _layer(2, 3, 3, 4, [1, 2, 2], 3)
    x = torch.randn(5, lay.in_dim, device=DEV, dtype=torch.float64, requires_grad=True)
    r = torch.randn(5, lay.out_dim, device=DEV, dtype=torch.float64, requires_grad=True)
    ws = list(lay.weight)
    assert torch.autograd.gradcheck(lambda a, b, *w: lay(a, residual=b), (x, r, *ws), eps=1e-6, atol=1e-8)


def test_residual_and_zero_ranks():
    """Output ranks above the shared ones are zero, or the residual's values; the residual is
    added to the shared ranks (also in place, residual = output buffer of the dgrad)."""
    from flashcart_amd.o3 import _ops

    lay = _layer(1, 3, 8, 8, None, 5)
    n = 100
    x = torch.randn(n, lay.in_dim, device=DEV, dtype=torch.float64)
    r = torch.randn(n, lay.out_dim, device=DEV, dtype=torch.float64)
    with torch.no_grad():
        out = lay(x, residual=r)
        plain = lay(x)
    _close(out, plain + r, "residual")
    assert float(plain[:, (1 + 3) * 8:].abs().max()) == 0.0
    go = torch.randn(n, lay.out_dim, device=DEV, dtype=torch.float64)
    res = torch.randn(n, lay.in_dim, device=DEV, dtype=torch.float64)
    with torch.no_grad():
        gx = lay.input_grad(go, residual=res)
        gx0 = _ops.linear_bwd(go, list(lay.weight), 1, 3, 8, 8, [1, 1], lay._scale_list)
    _close(gx, gx0 + res, "dgrad residual")


@pytest.mark.parametrize("cfg", CFGS[1:4])
def test_reference_ops_float64(cfg):
    """torch.ops.flashcart.linear_fwd / linear_bwd / linear_dbwd with the reference's arguments
    for float64 tensors (use_fp64 = True): outputs and first and second derivatives."""
    import flashcart_amd.o3._second_order  # noqa: F401

    lin, lout, fin, fout, paths = cfg
    lay = _layer(lin, lout, fin, fout, paths, 7)
    n = 41
    x = torch.randn(n, lay.in_dim, device=DEV, dtype=torch.float64)
    ws = [w.detach().clone() for w in lay.weight]
    scale = lay.scale.to(torch.float64)
    args = (lay.meta, lay.out_dim, True, "ieee", *lay.meta_lists, scale)
    out = torch.ops.flashcart.linear_fwd(x, ws, *args)
    xd = x.cpu().requires_grad_()
    wd = [w.cpu().requires_grad_() for w in ws]
    ref = O.linear(xd, wd, lin, lout, fin, fout, paths)
    _close(out, ref, "linear_fwd")
    go = torch.randn(n, lay.out_dim, device=DEV, dtype=torch.float64)
    gx, gws = torch.ops.flashcart.linear_bwd(go, x, ws, True, True, True, "ieee", *lay.meta_lists, scale)
    rgx, *rgw = torch.autograd.grad(ref, [xd] + wd, go.cpu(), create_graph=True)
    _close(gx, rgx, "linear_bwd grad_x")
    for l, (a, b) in enumerate(zip(gws, rgw)):
        _close(a, b, f"linear_bwd grad_weight[{l}]")
    xa = x.clone().requires_grad_()
    wa = [w.clone().requires_grad_() for w in ws]
    goa = go.clone().requires_grad_()
    o = torch.ops.flashcart.linear_fwd(xa, wa, *args)
    g1 = torch.autograd.grad(o, [xa] + wa, goa, create_graph=True)
    cots = [torch.randn_like(t) for t in g1]
    s2 = sum((a * c).sum() for a, c in zip(g1, cots))
    got2 = torch.autograd.grad(s2, [goa, xa] + wa, allow_unused=True)
    god = go.cpu().requires_grad_()
    rg1 = torch.autograd.grad(O.linear(xd, wd, lin, lout, fin, fout, paths), [xd] + wd, god, create_graph=True)
    rs2 = sum((a * c.cpu()).sum() for a, c in zip(rg1, cots))
    want2 = torch.autograd.grad(rs2, [god, xd] + wd, allow_unused=True)
    for k, (a, b) in enumerate(zip(got2, want2)):
        b = torch.zeros(a.shape, dtype=torch.float64) if b is None else b
        _close(torch.zeros_like(b) if a is None else a, b, f"linear_dbwd input {k}")


def test_reference_ops_fp64_accumulation_of_float32():
    """use_fp64 = True with float32 tensors: float64 accumulation, the result rounded once to
    float32 (within one float32 rounding of the float64 oracle on the float32 inputs)."""
    lin, lout, fin, fout, paths = 3, 3, 32, 16, [3, 5, 5, 4]
    lay = _layer(lin, lout, fin, fout, paths, 9).float()
    n = 64
    x = torch.randn(n, lay.in_dim, device=DEV, dtype=torch.float32)
    ws = [w.detach().clone() for w in lay.weight]
    out = torch.ops.flashcart.linear_fwd(x, ws, lay.meta, lay.out_dim, True, "ieee", *lay.meta_lists, lay.scale)
    assert out.dtype == torch.float32
    ref = O.linear(x.double().cpu(), [w.double().cpu() for w in ws], lin, lout, fin, fout, paths)
    assert_close(out, ref, 2 ** -23, 1e-30, "fp64 accumulation, float32 output")
    go = torch.randn(n, lay.out_dim, device=DEV)
    gx, gws = torch.ops.flashcart.linear_bwd(go, x, ws, True, True, True, "ieee", *lay.meta_lists, lay.scale)
    assert gx.dtype == torch.float32 and all(g.dtype == torch.float32 for g in gws)
    xd = x.double().cpu().requires_grad_()
    wd = [w.double().cpu().requires_grad_() for w in ws]
    want = torch.autograd.grad(O.linear(xd, wd, lin, lout, fin, fout, paths), [xd] + wd, go.double().cpu())
    for k, (a, b) in enumerate(zip([gx] + gws, want)):
        assert_close(a, b, 2 ** -23, 1e-30, f"fp64 accumulation grad {k}")


def test_wgrad_entry_points():
    """fc_linear_wgrad_f64 through the C ABI: the workspace query, a split reduction (several
    parts), the same sums with one part (few rows), a subset of ranks, and zero rows."""
    import ctypes

    from flashcart_amd import _lib

    lib = _lib.load()
    lin = lout = 3
    fin, fout, paths = 64, 32, [1, 2, 1, 1]
    g = torch.Generator().manual_seed(4)
    ws = [torch.randn(fout, fin * paths[l], generator=g, dtype=torch.float64).to(DEV) for l in range(4)]
    scale = [0.5 + l for l in range(4)]
    desc = _lib.linear_desc(lin, lout, fin, fout, paths, ws, scale)
    assert isinstance(desc, _lib.LinearDescF64)
    in_dim = sum((2 * l + 1) * fin * paths[l] for l in range(4))
    out_dim = 16 * fout
    stream = torch.cuda.current_stream().cuda_stream
    for n, subset in ((5000, (0, 1, 2, 3)), (200, (0, 1, 2, 3)), (5000, (2,)), (0, (0, 3))):
        x = torch.randn(n, in_dim, generator=g, dtype=torch.float64)
        go = torch.randn(n, out_dim, generator=g, dtype=torch.float64)
        outs = [torch.full_like(w, float("nan")) if l in subset else None for l, w in enumerate(ws)]
        ptrs = (_lib.c_vp * 4)(*[o.data_ptr() if o is not None else None for o in outs])
        need = lib.fc_linear_wgrad_f64_workspace(ctypes.byref(desc), n, ptrs)
        assert need >= 0
        if n == 5000:
            assert need > 0, "a long reduction is split over workgroups"
        buf = torch.empty(max(need, 1), dtype=torch.float64, device=DEV)
        xd, god = x.to(DEV), go.to(DEV)
        if need > 0:  # too little workspace is refused
            assert lib.fc_linear_wgrad_f64(ctypes.byref(desc), n, god.data_ptr(), xd.data_ptr(), 0.75, ptrs,
                                           buf.data_ptr(), need - 1, stream) == 6
        st = lib.fc_linear_wgrad_f64(ctypes.byref(desc), n, god.data_ptr(), xd.data_ptr(), 0.75, ptrs, buf.data_ptr(),
                                     need, stream)
        assert st == 0, _lib.load().fc_status_string(st)
        io = oo = 0
        for l in range(4):
            k, m = fin * paths[l], 2 * l + 1
            if l in subset:
                want = go[:, oo:oo + m * fout].reshape(n * m, fout).t() @ x[:, io:io + m * k].reshape(n * m, k)
                _close(outs[l], want * (0.75 * scale[l]), f"wgrad n={n} rank {l}")
            io += m * k
            oo += m * fout
