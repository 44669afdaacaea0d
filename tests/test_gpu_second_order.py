"""Second derivatives on the GPU (force-loss training) against the float64 CPU oracle.

Every op is checked the same way: y = op(inputs); with a random grad_out r (itself a
differentiable input) the first-order gradients g_k = d<r, y>/d input_k are taken with
create_graph=True, contracted with random cotangents c_k, and s = sum_k <c_k, g_k> is
differentiated with respect to every input and r. That exercises every term of the
backward op's own backward. The oracle runs the same expressions in float64 through torch
autograd. Bar: every second-order gradient within 2e-4 of its largest magnitude (float32
kernels against float64).

The model test compares the parameter gradients of a force-matching loss with the
oracle's (``oracle.model.force_loss_grads``).
"""

import math

import pytest
import torch

from oracle import model as OM
from oracle import ops as O
from tests.helpers import assert_close

pytestmark = pytest.mark.gpu
DEV = "cuda"
REL = 2e-4


def _second_order(fn, inputs, seed):
    """(outputs, first grads, second grads wrt inputs and grad_out) of fn at ``inputs``."""
    g = torch.Generator().manual_seed(seed)
    outs = fn(*inputs)
    outs = outs if isinstance(outs, (tuple, list)) else (outs,)
    rs = [torch.randn(o.shape, generator=g, dtype=torch.float64).to(o.device, o.dtype).requires_grad_(True)
          for o in outs]
    inner = sum((o * r).sum() for o, r in zip(outs, rs))
    firsts = torch.autograd.grad(inner, inputs, create_graph=True)
    cs = [torch.randn(f.shape, generator=g, dtype=torch.float64).to(f.device, f.dtype) for f in firsts]
    s = sum((f * c).sum() for f, c in zip(firsts, cs))
    seconds = torch.autograd.grad(s, list(inputs) + rs, allow_unused=True)
    return outs, firsts, seconds


def _compare(fn_gpu, fn_ref, inputs, seed=0, rel=REL):
    """Run the second-order probe on the GPU (float32) and on the oracle (float64)."""
    gi = [x.to(DEV, torch.float32).requires_grad_(True) for x in inputs]
    ri = [x.to("cpu", torch.float64).requires_grad_(True) for x in inputs]
    og, fg, sg = _second_order(fn_gpu, gi, seed)
    orf, fr, sr = _second_order(fn_ref, ri, seed)
    for k, (a, b) in enumerate(zip(og, orf)):
        assert_close(a, b, 0.0, 1e-5 * float(b.abs().max()) + 1e-6, f"output {k}")
    for k, (a, b) in enumerate(zip(fg, fr)):
        assert_close(a, b, 0.0, 1e-5 * float(b.abs().max()) + 1e-6, f"first-order grad {k}")
    for k, (a, b) in enumerate(zip(sg, sr)):
        if b is None:
            assert a is None or float(a.abs().max()) == 0.0, f"second-order grad {k} should vanish"
            continue
        assert a is not None, f"second-order grad {k} missing"
        assert_close(a, b, 0.0, rel * float(b.abs().max()) + 1e-7, f"second-order grad {k}")


def _tp_case(conv, shared, sym, l1, l2, lo, f1, f2, n=11, e=57, seed=0):
    from flashcart_amd.o3 import _ops
    from flashcart_amd.codegen.cartesian import count_output_paths
    g = torch.Generator().manual_seed(seed)
    C = max(f1, f2)
    _, P = count_output_paths(l1, l2, lo, sym)
    rows = e if conv else n
    in1 = torch.randn(n, (l1 + 1) ** 2 * f1, generator=g, dtype=torch.float64)
    in2 = torch.randn(rows, (l2 + 1) ** 2 * f2, generator=g, dtype=torch.float64)
    w = torch.randn((P * C,) if shared else (rows, P * C), generator=g, dtype=torch.float64)
    if conv:
        idx_i = torch.sort(torch.randint(0, n, (e,), generator=g)).values
        idx_j = torch.randint(0, n, (e,), generator=g)
    else:
        idx_i = idx_j = None
    meta = _ops.tp_meta(l1, l2, lo, f1, f2, sym, False)

    def gpu(a, b, ww):
        ii = idx_i.to(DEV) if conv else None
        jj = idx_j.to(DEV) if conv else None
        return _ops.tp_fwd(a, b, ww, ii, jj, l1, l2, lo, f1, f2, sym, shared, *meta, False)

    def ref(a, b, ww):
        return O.tensor_product(a, b, ww, idx_i, idx_j, l1, l2, lo, f1, f2, symmetric_product=sym,
                                shared_weights=shared)

    return gpu, ref, [in1, in2, w]


@pytest.mark.parametrize("conv,shared,sym,l1,l2,lo,f1,f2", [
    (True, False, False, 2, 2, 2, 8, 1),    # interaction: nodes x edge attrs, per-edge weights
    (True, False, False, 3, 3, 3, 4, 1),
    (True, True, False, 1, 2, 2, 8, 8),
    (False, True, False, 2, 2, 2, 8, 8),    # product step: node-wise, shared weights
    (False, False, False, 3, 1, 2, 4, 4),
    (False, True, True, 2, 2, 0, 8, 8),     # RMS invariants: symmetric paths
])
def test_tp_second_order(conv, shared, sym, l1, l2, lo, f1, f2):
    gpu, ref, inputs = _tp_case(conv, shared, sym, l1, l2, lo, f1, f2, seed=l1 * 7 + lo)
    _compare(gpu, ref, inputs, seed=3)


@pytest.mark.parametrize("in_l,out_l,fin,fout,paths", [(2, 2, 8, 16, [1, 1, 1]), (3, 1, 4, 8, [1, 3, 2, 1]),
                                                       (1, 3, 16, 8, [2, 1])])
def test_linear_second_order(in_l, out_l, fin, fout, paths):
    from flashcart_amd.o3 import _ops
    g = torch.Generator().manual_seed(in_l * 10 + out_l)
    n = 13
    in_dim = sum((2 * l + 1) * fin * paths[l] for l in range(in_l + 1))
    common = min(in_l, out_l)
    x = torch.randn(n, in_dim, generator=g, dtype=torch.float64)
    ws = [torch.randn(fout, fin * paths[l], generator=g, dtype=torch.float64) for l in range(common + 1)]
    scale = [float(fin * paths[l]) ** -0.5 for l in range(common + 1)]

    def gpu(xx, *w):
        return _ops.linear_fwd(xx, list(w), in_l, out_l, fin, fout, paths, scale)

    def ref(xx, *w):
        return O.linear(xx, list(w), in_l, out_l, fin, fout, paths)

    _compare(gpu, ref, [x] + ws, seed=5)


@pytest.mark.parametrize("act,bias", [(1, True), (0, False), (1, False)])
def test_dense_second_order(act, bias):
    from flashcart_amd.o3 import _ops
    g = torch.Generator().manual_seed(act * 2 + bias)
    n, k, m = 37, 24, 40
    x = torch.randn(n, k, generator=g, dtype=torch.float64)
    w = torch.randn(m, k, generator=g, dtype=torch.float64)
    b = torch.randn(m, generator=g, dtype=torch.float64)
    s = k ** -0.5

    def gpu(xx, ww, *bb):
        return _ops.dense_fwd(xx, ww, bb[0] if bb else None, s, act)[0]

    def ref(xx, ww, *bb):
        y = O.dense(xx, ww, bb[0] if bb else None, s)
        return O.silu(y) if act else y

    _compare(gpu, ref, [x, w] + ([b] if bias else []), seed=7)


def test_dense_chain_second_order():
    """Two stacked SiLU layers: the second layer's dense_bwd reads the first layer's
    pre-activation output, whose gradient must reach x and the first weight."""
    from flashcart_amd.o3 import _ops
    g = torch.Generator().manual_seed(11)
    x = torch.randn(29, 16, generator=g, dtype=torch.float64)
    w1 = torch.randn(32, 16, generator=g, dtype=torch.float64)
    w2 = torch.randn(8, 32, generator=g, dtype=torch.float64)

    def gpu(xx, a, b):
        h = _ops.dense_fwd(xx, a, None, 0.25, 1)[0]
        return _ops.dense_fwd(h, b, None, 32 ** -0.5, 1)[0]

    def ref(xx, a, b):
        return O.silu(O.dense(O.silu(O.dense(xx, a, None, 0.25)), b, None, 32 ** -0.5))

    _compare(gpu, ref, [x, w1, w2], seed=2)


@pytest.mark.parametrize("n,offset", [(4096, 0), (1001, 0), (4096, 1)])
def test_silu_grad_mix(n, offset):
    """fc_silu_grad_mix against the float64 derivatives of the rescaled SiLU, obtained by
    differentiating O.silu with torch.autograd (vector path, scalar tail, unaligned operands)."""
    from flashcart_amd.o3 import _ops
    g = torch.Generator().manual_seed(n + offset)
    a, b, p, d = (4 * torch.randn(n + offset, generator=g, dtype=torch.float64) for _ in range(4))
    pp = p.clone().requires_grad_(True)
    (f1,) = torch.autograd.grad(O.silu(pp).sum(), pp, create_graph=True)
    (f2,) = torch.autograd.grad(f1.sum(), pp)
    want1, want2 = (a * f1 + d).detach()[offset:], (a * b * f2)[offset:]
    ga, gb, gp, gd = (t.to(DEV, torch.float32)[offset:] for t in (a, b, p, d))
    o1, o2 = _ops.silu_grad_mix(ga, gp, add=gd, b=gb, need1=True, need2=True)
    # float32 inputs and sigmoid: 1e-5 relative, plus 2e-6 of the largest magnitude where
    # 1 - sigmoid(pre) cancels (large pre)
    assert_close(o1, want1, 1e-5, 2e-6 * float(want1.abs().max()), "a f'(pre) + add")
    assert_close(o2, want2, 1e-5, 2e-6 * float(want2.abs().max()), "a b f''(pre)")
    o1n, none = _ops.silu_grad_mix(ga, gp)
    assert none is None
    w1 = (a * f1).detach()[offset:]
    assert_close(o1n, w1, 1e-5, 2e-6 * float(w1.abs().max()), "a f'(pre)")


@pytest.mark.parametrize("l_max", [1, 2, 3])
def test_irreps_second_order(l_max):
    from flashcart_amd.o3 import _ops
    g = torch.Generator().manual_seed(l_max)
    x = torch.randn(41, 3, generator=g, dtype=torch.float64)
    _compare(lambda xx: _ops.irreps_fwd(xx, l_max), lambda xx: O.irreps(xx, l_max), [x], seed=l_max)


@pytest.mark.parametrize("basis", ["affine", "cosine", "bessel"])
def test_radial_second_order(basis):
    from flashcart_amd import _lib
    from flashcart_amd.o3 import _ops
    code = {"affine": _lib.BASIS_CHEBYSHEV_AFFINE, "cosine": _lib.BASIS_CHEBYSHEV_COSINE,
            "bessel": _lib.BASIS_BESSEL}[basis]
    g = torch.Generator().manual_seed(code)
    d = 0.5 + 4.2 * torch.rand(53, generator=g, dtype=torch.float64)  # inside (0, r_max)
    r_min, r_max, n_rad, p = 0.0, 5.0, 8, 6

    def gpu(dd):
        return _ops.radial_fwd(dd, code, n_rad, r_min, r_max, p)

    def ref(dd):
        f = O.bessel(dd, n_rad, r_max) if basis == "bessel" else O.chebyshev(dd, n_rad, r_max, r_min, basis)
        return f, O.cutoff(dd, r_max, p)

    _compare(gpu, ref, [d], seed=4)


@pytest.mark.parametrize("l_max,use_shift,basis", [(2, True, "affine"), (3, False, "affine"), (3, True, "cosine"),
                                                   (1, False, "bessel"), (0, True, "cosine")])
def test_edge_geometry_second_order(l_max, use_shift, basis):
    """Some edges reach beyond r_max (envelope masked) — both sides of the cutoff."""
    from flashcart_amd import _lib
    from flashcart_amd.o3 import _ops
    code = {"affine": _lib.BASIS_CHEBYSHEV_AFFINE, "cosine": _lib.BASIS_CHEBYSHEV_COSINE,
            "bessel": _lib.BASIS_BESSEL}[basis]
    g = torch.Generator().manual_seed(l_max + 10 * code)
    n, e = 14, 80
    pos = 3.0 * torch.rand(n, 3, generator=g, dtype=torch.float64)
    idx_i = torch.sort(torch.randint(0, n, (e,), generator=g)).values
    idx_j = (idx_i + 1 + torch.randint(0, n - 1, (e,), generator=g)) % n
    shift = (torch.randint(-1, 2, (e, 3), generator=g) * 1.5).to(torch.float64) if use_shift else None
    r_max = 4.5 if use_shift else 7.0

    def gpu(p, *sv):
        return _ops.edge_geometry(p, sv[0] if sv else None, idx_i.to(DEV), idx_j.to(DEV), None, None, None, None,
                                  l_max, code, 8, 0.0, r_max, 6)

    def ref(p, *sv):
        v = p[idx_j] - p[idx_i]
        if sv:
            v = v + sv[0]
        d = v.norm(dim=-1)
        u = v / d.clamp_min(1e-4).unsqueeze(-1)
        f = O.bessel(d, 8, r_max) if basis == "bessel" else O.chebyshev(d, 8, r_max, 0.0, basis)
        return O.irreps(u, l_max), f, O.cutoff(d, r_max, 6)

    _compare(gpu, ref, [pos] + ([shift] if use_shift else []), seed=9)


@pytest.mark.parametrize("l_max,C", [(2, 16), (3, 8)])
def test_rms_norm_second_order(l_max, C):
    from flashcart_amd.o3 import _ops
    g = torch.Generator().manual_seed(l_max)
    x = torch.randn(9, (l_max + 1) ** 2 * C, generator=g, dtype=torch.float64)
    w = 1.0 + 0.3 * torch.randn(l_max + 1, C, generator=g, dtype=torch.float64)
    eps = 1e-6

    def gpu(xx, ww):
        return _ops.rms_norm(xx, ww, l_max, eps)[0]

    def ref(xx, ww):
        sd = {f"n.weights.{l}": ww[l] for l in range(l_max + 1)}
        return OM.rms_norm(sd, "n", xx, l_max, C, eps)

    _compare(gpu, ref, [x, w], seed=6)


@pytest.mark.parametrize("act", [0, 1])
def test_gate_second_order(act):
    from flashcart_amd.o3 import _ops
    g = torch.Generator().manual_seed(act)
    l_max, C, n = 2, 8, 15
    v = torch.randn(n, (l_max + 1) ** 2 * C, generator=g, dtype=torch.float64)
    p = torch.randn(n, (l_max + 1) * C, generator=g, dtype=torch.float64)

    def gpu(vv, pp):
        return _ops.gate(vv, pp, l_max, act)

    def ref(vv, pp):
        a = 1.8462285453386054 * torch.sigmoid(pp) if act else pp
        a = a.view(n, l_max + 1, C)
        rep = torch.tensor([l for l in range(l_max + 1) for _ in range(2 * l + 1)])
        return vv * a[:, rep].reshape(n, -1)

    _compare(gpu, ref, [v, p], seed=8)


# ---------------------------------------------------------------------------
# Model: parameter gradients of a force-matching loss
# ---------------------------------------------------------------------------

def _force_loss_case(model, graph, cfg, seed, w_e=1.0, w_f=10.0, rel=1e-3):
    g = torch.Generator().manual_seed(seed)
    n_graphs = int(graph.n_atoms.shape[0]) if hasattr(graph, "n_atoms") else 1
    e_ref = torch.randn(n_graphs, generator=g, dtype=torch.float64)
    f_ref = 0.1 * torch.randn(graph.positions.shape, generator=g, dtype=torch.float64)
    names = [k for k, _ in model.named_parameters()]
    want = OM.force_loss_grads(model.state_dict(), model.to_model_config(), graph.to_dict(), e_ref, f_ref, names,
                               w_e, w_f)
    m = model.to(DEV)
    m.requires_grad_(True)
    m.zero_grad(set_to_none=True)
    out = m.predict(graph.to(DEV), compute_forces=True, create_graph=True)
    loss = w_e * ((out["energy"] - e_ref.to(DEV, torch.float32)) ** 2).mean() + \
        w_f * ((out["forces"] - f_ref.to(DEV, torch.float32)) ** 2).mean()
    loss.backward()
    assert_close(loss.detach(), want["loss"], 1e-5, 0.0, "loss")
    scale = max(float(want[k].abs().max()) for k in names)
    for k, p in m.named_parameters():
        got = p.grad if p.grad is not None else torch.zeros_like(p)
        ref = want[k]
        assert_close(got, ref, 0.0, rel * max(float(ref.abs().max()), 1e-2 * scale) + 1e-9, f"d loss / d {k}")
    return out


def _model(cfg, seed):
    from tests.test_gpu_model import _model as make
    return make(cfg, seed)


def test_force_loss_water_L2():
    from flashcart_amd.data import AtomicGraph
    from flashcart_amd.data.synthetic import model_config, water_box
    numbers, pos, cell, pbc = water_box(8, seed=1)
    cfg = model_config(["H", "O"], 16, 2, avg_neighbors=20.0)
    gr = AtomicGraph.from_arrays(numbers, pos, cfg["elements"], 5.0, cell=cell, pbc=pbc)
    _force_loss_case(_model(cfg, 7), gr, cfg, seed=1)


def test_force_loss_fcc_L3():
    from flashcart_amd.data import AtomicGraph
    from flashcart_amd.data.synthetic import fcc_alloy, model_config
    numbers, pos, cell, pbc = fcc_alloy(2, 2, 2, seed=3)
    cfg = model_config(["Cu", "Ni", "Fe", "Cr"], 16, 3, avg_neighbors=42.0)
    gr = AtomicGraph.from_arrays(numbers, pos, cfg["elements"], 5.0, cell=cell, pbc=pbc)
    _force_loss_case(_model(cfg, 1234), gr, cfg, seed=2)


def test_force_loss_molecule_batch():
    from flashcart_amd.data import AtomicGraph, batch_graphs
    from flashcart_amd.data.synthetic import model_config, molecules
    mols = molecules(3, 5, 10, seed=2)
    cfg = model_config(["H", "C", "N", "O"], 8, 2, avg_neighbors=6.0)
    gr = batch_graphs([AtomicGraph.from_arrays(z, p, cfg["elements"], 5.0) for z, p in mols])
    _force_loss_case(_model(cfg, 5), gr, cfg, seed=3)


def test_create_graph_frozen_parameters():
    """create_graph with frozen parameters still runs op by op (no first-order-only fused
    backward) and gives differentiable forces: d(sum F^2)/dR matches the oracle's."""
    from flashcart_amd.data import AtomicGraph
    from flashcart_amd.data.synthetic import model_config, water_box
    numbers, pos, cell, pbc = water_box(4, seed=2)
    cfg = model_config(["H", "O"], 8, 2, avg_neighbors=20.0)
    model = _model(cfg, 3)
    gr = AtomicGraph.from_arrays(numbers, pos, cfg["elements"], 5.0, cell=cell, pbc=pbc)
    # oracle: d/dR sum(F^2) in float64
    sd = {k: v.detach().double() for k, v in model.state_dict().items()}
    gd = {k: (v.detach().cpu() if torch.is_tensor(v) else v) for k, v in gr.to_dict().items()}
    p64 = gd["positions"].double().requires_grad_(True)
    gd["positions"], gd["cell"] = p64, gd["cell"].double()
    e = O.scatter_sum(OM.node_energies(sd, model.to_model_config(), gd), gd["batch"], 1)
    (f,) = torch.autograd.grad(e.sum(), p64, create_graph=True)
    (want,) = torch.autograd.grad((f ** 2).sum(), p64)
    m = model.to(DEV)
    m.requires_grad_(False)
    from flashcart_amd.nn import fused
    with fused.disabled():  # what predict(create_graph=True) does, with the positions leaf kept
        gd = m._prepare_predict_graph(gr.to(DEV), True, False, False)
        out = m._predict_impl(gd, True, False, False, True)
    (got,) = torch.autograd.grad((out["forces"] ** 2).sum(), gd["positions"])
    assert_close(got, want, 0.0, 1e-3 * float(want.abs().max()), "d sum F^2 / dR")
