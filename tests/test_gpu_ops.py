"""GPU parity of every HIP op against the CPU oracle (float64 oracle, float32 kernels).

Tolerances: relative 2e-5 plus an absolute floor scaled by the magnitude of the
quantity (float32 accumulation over up to a few hundred terms).
"""

import math

import pytest
import torch

from oracle import ops as O
from tests.helpers import assert_close, random_csr_graph, unit_vectors

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _ops():
    from flashcart_amd.o3 import _ops
    return _ops


def _close(got, want, what, rel=2e-5):
    """float32 GPU result against a float64 reference, relative to the reference's largest entry."""
    want = want.detach().double().cpu()
    assert_close(got, want, rel, rel * max(float(want.abs().max()) if want.numel() else 0.0, 1e-30), what)


@pytest.mark.parametrize("l_max", [0, 1, 2, 3])
def test_irreps_fwd_bwd(l_max):
    ops = _ops()
    x64 = unit_vectors(1000, seed=l_max).float().double().requires_grad_(True)
    ref = O.irreps(x64, l_max)
    g = torch.randn_like(ref)
    if l_max == 0:  # the expansion is the constant 1
        ref_gx = torch.zeros_like(x64)
    else:
        (ref_gx,) = torch.autograd.grad(ref, x64, g)
    x = x64.detach().float().to(DEV).requires_grad_(True)
    out = ops.irreps_fwd(x, l_max)
    (gx,) = torch.autograd.grad(out, x, g.float().to(DEV))
    assert_close(out, ref, 1e-5, 1e-6, "irreps fwd")
    assert_close(gx, ref_gx, 1e-5, 1e-5, "irreps bwd")


@pytest.mark.parametrize("kind", ["cheb_cos", "cheb_aff", "bessel", "cutoff"])
def test_radial_fwd_bwd(kind):
    ops = _ops()
    from flashcart_amd import _lib
    torch.manual_seed(1)
    d64 = torch.empty(4096).uniform_(0.0, 6.0).double().requires_grad_(True)
    if kind == "cheb_cos":
        ref, args = O.chebyshev(d64, 8, 5.0, 0.0, "cosine"), (_lib.BASIS_CHEBYSHEV_COSINE, 8, 0.0, 5.0, 0)
    elif kind == "cheb_aff":
        ref, args = O.chebyshev(d64, 8, 5.0, 0.5, "affine"), (_lib.BASIS_CHEBYSHEV_AFFINE, 8, 0.5, 5.0, 0)
    elif kind == "bessel":
        ref, args = O.bessel(d64, 8, 5.0), (_lib.BASIS_BESSEL, 8, 0.0, 5.0, 0)
    else:
        ref, args = O.cutoff(d64, 5.0, 6), (_lib.BASIS_NONE, 1, 0.0, 5.0, 6)
    g = torch.randn_like(ref)
    (ref_gd,) = torch.autograd.grad(ref, d64, g)
    d = d64.detach().float().to(DEV).requires_grad_(True)
    feats, env = ops.radial_fwd(d, *args)
    out = env if kind == "cutoff" else feats
    (gd,) = torch.autograd.grad(out, d, g.float().to(DEV))
    assert_close(out, ref, 2e-5, 2e-5, f"{kind} fwd")
    assert_close(gd, ref_gd, 1e-4, 1e-4, f"{kind} bwd")


def _tp_case(l1, l2, lo, f1, f2, sym=False, shared=False, reduced=False, conv=True, seed=0,
             degrees=(0, 1, 5, 26), n=37):
    ops = _ops()
    torch.manual_seed(seed)
    C = max(f1, f2)
    from oracle.cartesian import enumerate_paths
    P = len(enumerate_paths(l1, l2, lo, sym))
    if conv:
        ei = random_csr_graph(n, degrees, seed=seed)
        E = ei.shape[1]
        in1 = torch.randn(n, (l1 + 1) ** 2 * f1, dtype=torch.float64)
        in2 = torch.randn(E, (l2 + 1) ** 2 * f2, dtype=torch.float64)
        items = E
    else:
        ei = None
        in1 = torch.randn(n, (l1 + 1) ** 2 * f1, dtype=torch.float64)
        in2 = in1.clone() if sym else torch.randn(n, (l2 + 1) ** 2 * f2, dtype=torch.float64)
        items = n
    w = torch.randn(P * C, dtype=torch.float64) if shared else torch.randn(items, P * C, dtype=torch.float64)
    leaves64 = [t.clone().requires_grad_(True) for t in (in1, in2, w)]
    a1, a2, aw = leaves64
    ref = O.tensor_product(a1, a1 if sym else a2, aw, ei[0] if conv else None, ei[1] if conv else None,
                           l1, l2, lo, f1, f2, sym, shared, reduced)
    g = torch.randn_like(ref)
    ref_grads = torch.autograd.grad(ref, [a1, a2, aw] if not sym else [a1, aw], g)
    leaves = [t.detach().float().to(DEV).requires_grad_(True) for t in (in1, in2, w)]
    b1, b2, bw = leaves
    meta = ops.tp_meta(l1, l2, lo, f1, f2, sym, reduced)
    out = ops.tp_fwd(b1, b1 if sym else b2, bw, ei[0].to(DEV) if conv else None, ei[1].to(DEV) if conv else None,
                     l1, l2, lo, f1, f2, sym, shared, *meta, reduced)
    grads = torch.autograd.grad(out, [b1, b2, bw] if not sym else [b1, bw], g.float().to(DEV))
    scale = float(ref.abs().max()) + 1.0
    assert_close(out, ref, 2e-5, 2e-5 * scale, "tp fwd")
    for k, (gg, rr) in enumerate(zip(grads, ref_grads)):
        s = float(rr.abs().max()) + 1.0
        assert_close(gg, rr, 2e-5, 2e-5 * s, f"tp grad {k}")


CONV_CASES = [
    (0, 3, 3, 16, 1), (2, 3, 3, 16, 1), (1, 2, 2, 8, 1), (2, 2, 2, 8, 1), (3, 3, 3, 4, 1), (0, 2, 2, 64, 1),
    (2, 3, 3, 128, 1), (1, 1, 2, 8, 8), (2, 1, 1, 1, 8),
    # 64 channels with at most 40 output rows: the backward in sender order
    (2, 2, 2, 32, 1), (2, 2, 2, 64, 1), (1, 2, 2, 64, 1), (2, 1, 2, 64, 1),
]


@pytest.mark.parametrize("case", CONV_CASES, ids=lambda c: "x".join(map(str, c)))
def test_tp_conv(case):
    _tp_case(*case, conv=True)


@pytest.mark.parametrize("case", [(2, 3, 3, 128, 1), (2, 2, 2, 64, 1), (1, 2, 2, 64, 1), (2, 2, 2, 32, 1)],
                         ids=lambda c: "x".join(map(str, c)))
def test_tp_conv_chunk_boundaries(case):
    """Receiver and sender edge counts around the backward kernels' 16-edge chunks and their
    paired edge loop (odd last edges, a last edge on a chunk's first slot, one to three chunks),
    for one edge group (128 channels) and several (32 and 64): the staged indices and the
    operand waits keep every edge's result."""
    _tp_case(*case, conv=True, seed=5, degrees=(1, 15, 16, 17, 31, 32, 33, 47), n=48)


@pytest.mark.parametrize("need", [(True, True, False), (True, False, True), (False, True, True)])
def test_tp_conv_bwd_gradient_subsets(need):
    """The interaction-layer backward asked for a subset of its gradients (the second derivative
    asks for (in1, in2) without the weights): the general kernel that then runs forms each requested
    gradient exactly as the specialised all-gradients kernel does, bit for bit."""
    ops = _ops()
    g = torch.Generator().manual_seed(7)
    l1, l2, lo, C = 2, 3, 3, 128
    ei = random_csr_graph(40, (3, 9, 17), seed=4)
    E = ei.shape[1]
    from oracle.cartesian import enumerate_paths
    P = len(enumerate_paths(l1, l2, lo, False))
    in1 = torch.randn(40, 9 * C, generator=g).to(DEV)
    in2 = torch.randn(E, 16, generator=g).to(DEV)
    w = torch.randn(E, P * C, generator=g).to(DEV)
    meta = ops.tp_meta(l1, l2, lo, C, 1, False, False)
    go = torch.randn(40, ops._tp_out_dim(l1, l2, lo, C, 1, False, False), generator=g).to(DEV)
    args = (go, in1, in2, w, ei[0].to(DEV), ei[1].to(DEV), l1, l2, lo, C, 1, False, False, *meta, False)
    full = ops.tp_bwd(*args, True, True, True)
    part = ops.tp_bwd(*args, *need)
    for k in range(3):
        if need[k]:
            assert torch.equal(part[k], full[k]), f"gradient {k}"
        else:
            assert part[k].numel() == 0


def test_tp_conv_reduced_shared():
    _tp_case(2, 2, 2, 8, 1, shared=True, reduced=True, conv=True, seed=3)


@pytest.mark.parametrize("f1", [64, 128])
def test_tp_conv_shared_weights_full_width(f1):
    """Shared weights at the interaction layer's channel counts: the per-edge-weight backward
    specialisation does not apply (it reads one weight row per edge)."""
    _tp_case(2, 3, 3, f1, 1, shared=True, conv=True, seed=5)


ROW_CASES = [
    dict(l1=3, l2=3, lo=3, f1=8, f2=8, shared=True), dict(l1=3, l2=3, lo=2, f1=8, f2=8, shared=True),
    dict(l1=3, l2=3, lo=0, f1=8, f2=8, shared=True), dict(l1=3, l2=0, lo=3, f1=8, f2=1, shared=True),
    dict(l1=3, l2=3, lo=0, f1=8, f2=8, sym=True, shared=True), dict(l1=2, l2=2, lo=0, f1=16, f2=16, sym=True,
                                                                   shared=True),
    dict(l1=2, l2=2, lo=2, f1=1, f2=8), dict(l1=2, l2=2, lo=2, f1=8, f2=8, reduced=True),
    dict(l1=3, l2=3, lo=3, f1=128, f2=128, shared=True),
]


@pytest.mark.parametrize("case", ROW_CASES, ids=lambda c: "-".join(f"{k}{v}" for k, v in c.items()))
def test_tp_rows(case):
    _tp_case(conv=False, n=300, **case)


@pytest.mark.parametrize("l1,l2,lo,comps1,shared", [(3, 3, 3, 9, True), (3, 3, 2, 16, True), (2, 2, 2, 4, False),
                                                    (3, 3, 0, 1, True)])
def test_tp_rows_accumulate(l1, l2, lo, comps1, shared):
    """fc_tp_bwd_rows_acc: input gradients of the node-wise product plus residual gradients
    (res1 over the leading comps1 components of in1, res2 over all of in2, accumulated in
    place), against the float64 oracle's vector-Jacobian product plus the residuals."""
    ops = _ops()
    torch.manual_seed(l1 + 3 * lo + comps1)
    n, C = 300, 32
    from oracle.cartesian import enumerate_paths
    P = len(enumerate_paths(l1, l2, lo, False))
    in1 = torch.randn(n, (l1 + 1) ** 2 * C, dtype=torch.float64, requires_grad=True)
    in2 = torch.randn(n, (l2 + 1) ** 2 * C, dtype=torch.float64, requires_grad=True)
    w = torch.randn(P * C, dtype=torch.float64) if shared else torch.randn(n, P * C, dtype=torch.float64)
    ref = O.tensor_product(in1, in2, w, None, None, l1, l2, lo, C, C, False, shared, False)
    g = torch.randn_like(ref)
    q1, q2 = torch.autograd.grad(ref, [in1, in2], g)
    r1, r2 = q1, q2
    res1 = torch.randn(n, comps1 * C, dtype=torch.float64)
    res2 = torch.randn(n, (l2 + 1) ** 2 * C, dtype=torch.float64)
    r1 = r1.clone()
    r1[:, : comps1 * C] += res1
    r2 = r2 + res2
    d = [t.detach().float().to(DEV) for t in (in1, in2, w, g, res1, res2)]
    res1_dev = d[4].clone()
    g1, g2 = ops.tp_bwd_rows_acc(d[3], d[0], d[1], d[2], l1, l2, lo, C, shared, res1=d[4], res2=d[5],
                                 inplace2=True)
    assert g2.data_ptr() == d[5].data_ptr(), "full-width residual must be accumulated in place"
    assert torch.equal(d[4], res1_dev), "res1 must not be modified"
    assert_close(g1, r1, 2e-5, 2e-5 * (float(r1.abs().max()) + 1.0), "rows acc grad in1")
    assert_close(g2, r2, 2e-5, 2e-5 * (float(r2.abs().max()) + 1.0), "rows acc grad in2")
    # no residuals: plain input gradients
    h1, h2 = ops.tp_bwd_rows_acc(d[3], d[0], d[1], d[2], l1, l2, lo, C, shared)
    assert_close(h1, q1, 2e-5, 2e-5 * (float(q1.abs().max()) + 1.0), "rows grad in1")
    assert_close(h2, q2, 2e-5, 2e-5 * (float(q2.abs().max()) + 1.0), "rows grad in2")


@pytest.mark.parametrize("cfg", [(0, 0, 16, 16, None), (2, 2, 32, 16, None), (3, 3, 128, 128, [3, 5, 5, 4]),
                                 (2, 3, 64, 64, None), (3, 1, 8, 24, [1, 2, 3, 1])])
def test_linear(cfg):
    ops = _ops()
    lin, lout, fin, fout, paths = cfg
    paths = paths or [1] * (lin + 1)
    torch.manual_seed(5)
    n = 333
    in_dim = sum((2 * l + 1) * fin * paths[l] for l in range(lin + 1))
    x64 = torch.randn(n, in_dim, dtype=torch.float64, requires_grad=True)
    ws64 = [torch.randn(fout, fin * paths[l], dtype=torch.float64, requires_grad=True)
            for l in range(min(lin, lout) + 1)]
    ref = O.linear(x64, ws64, lin, lout, fin, fout, paths)
    g = torch.randn_like(ref)
    ref_g = torch.autograd.grad(ref, [x64] + ws64, g)
    x = x64.detach().float().to(DEV).requires_grad_(True)
    ws = [w.detach().float().to(DEV).requires_grad_(True) for w in ws64]
    scale = [float(fin * paths[l]) ** -0.5 for l in range(min(lin, lout) + 1)]
    out = ops.linear_fwd(x, ws, lin, lout, fin, fout, paths, scale, 1.0)
    got_g = torch.autograd.grad(out, [x] + ws, g.float().to(DEV))
    assert_close(out, ref, 1e-5, 1e-4, "linear fwd")
    for k, (a, b) in enumerate(zip(got_g, ref_g)):
        assert_close(a, b, 1e-5, 1e-4 * (float(b.abs().max()) + 1), f"linear grad {k}")


@pytest.mark.parametrize("shape", [(1000, 8, 64, 1, True), (777, 64, 2176, 0, True), (500, 64, 1, 0, True),
                                   (300, 256, 64, 1, True),
                                   # no bias, K = 64: the wide-output kernel (full and partial row blocks,
                                   # and a width that is not a multiple of 64)
                                   (1000, 64, 512, 0, False), (777, 64, 2176, 0, False), (129, 64, 300, 0, False)])
def test_dense(shape):
    ops = _ops()
    n, k, m, act, with_bias = shape
    torch.manual_seed(7)
    x64 = torch.randn(n, k, dtype=torch.float64, requires_grad=True)
    w64 = torch.randn(m, k, dtype=torch.float64, requires_grad=True)
    b64 = torch.randn(m, dtype=torch.float64, requires_grad=True) if with_bias else None
    ref = O.dense(x64, w64, b64)
    if act:
        ref = O.silu(ref)
    g = torch.randn_like(ref)
    leaves64 = [x64, w64] + ([b64] if with_bias else [])
    ref_g = torch.autograd.grad(ref, leaves64, g)
    leaves = [t.detach().float().to(DEV).requires_grad_(True) for t in leaves64]
    out, _ = ops.dense_fwd(leaves[0], leaves[1], leaves[2] if with_bias else None, float(k) ** -0.5, act)
    got = torch.autograd.grad(out, leaves, g.float().to(DEV))
    assert_close(out, ref, 1e-5, 1e-4, "dense fwd")
    for i, (a, r) in enumerate(zip(got, ref_g)):
        assert_close(a, r, 1e-5, 1e-4 * (float(r.abs().max()) + 1), f"dense grad {i}")


@pytest.mark.parametrize("n,n_in,m", [(1000, 8, 512), (300, 8, 2176), (257, 40, 200), (128, 64, 256), (5, 8, 64)])
def test_radial_mlp_fused(n, n_in, m):
    """The one-pass radial MLP (8 -> 64 -> 64 -> m, rescaled SiLU) and its input gradient
    against the float64 layer-by-layer chain: partial row blocks, an output width that is
    not a multiple of 64, more inputs than one MFMA column block."""
    ops = _ops()
    gen = torch.Generator().manual_seed(n + m)
    x64 = torch.randn(n, n_in, generator=gen, dtype=torch.float64, requires_grad=True)
    w0 = torch.randn(64, n_in, generator=gen, dtype=torch.float64)
    w1 = torch.randn(64, 64, generator=gen, dtype=torch.float64)
    w2 = torch.randn(m, 64, generator=gen, dtype=torch.float64)
    ref = O.dense(O.silu(O.dense(O.silu(O.dense(x64, w0)), w1)), w2)
    g = torch.randn(ref.shape, generator=gen, dtype=torch.float64)
    (ref_gx,) = torch.autograd.grad(ref, x64, g)
    x = x64.detach().float().to(DEV)
    w0f, w1f, w2f = (t.float().to(DEV) for t in (w0, w1, w2))
    s0, s1, s2 = float(n_in) ** -0.5, 0.125, 0.125
    with torch.no_grad():
        out = ops.radial_mlp_fwd(x, w0f, s0, w1f, s1, w2f, s2)
        gh2 = ops.dense_bwd(g.float().to(DEV), x.new_empty(0), w2f, s2, 0)
        gx = ops.radial_mlp_bwd(gh2, x, w0f, s0, w1f, s1)
    assert_close(out, ref, 1e-5, 2e-5 * float(ref.abs().max()), "radial mlp fwd")
    assert_close(gx, ref_gx, 1e-5, 2e-5 * float(ref_gx.abs().max()), "radial mlp input grad")


@pytest.mark.parametrize("n,degrees", [(64, (3, 7, 12)), (300, (1, 90, 200))])
def test_edge_geometry_positions_grad(n, degrees):
    """Edge geometry forward (rows staged through LDS per 256 edges, a partial last block) and
    the position gradient's segmented sums (one wave per node; segments above 64 edges)."""
    ops = _ops()
    from flashcart_amd import _lib
    from flashcart_amd.o3._graph import build_graph
    torch.manual_seed(11)
    pos64 = (torch.rand(n, 3) * 8.0).double().requires_grad_(True)
    ei = random_csr_graph(n, degrees, seed=2)
    E = ei.shape[1]
    shift = torch.randint(-1, 2, (E, 3)).double() * 8.0
    v = pos64[ei[1]] - pos64[ei[0]] + shift
    d = v.norm(dim=-1)
    r = v / d.clamp_min(O.MIN_EDGE_LENGTH).unsqueeze(-1)
    attrs = O.irreps(r, 3)
    feats = O.chebyshev(d, 8, 5.0, 0.0, "cosine")
    env = O.cutoff(d, 5.0, 6)
    ga, gf, ge = torch.randn_like(attrs), torch.randn_like(feats), torch.randn_like(env)
    loss = (attrs * ga).sum() + (feats * gf).sum() + (env * ge).sum()
    (ref_gpos,) = torch.autograd.grad(loss, pos64)
    pos = pos64.detach().float().to(DEV).requires_grad_(True)
    g = build_graph(ei.to(DEV), n)
    a2, f2, e2 = ops.edge_geometry(pos, shift.float().to(DEV), g.idx_i, g.idx_j, None, g.rowptr, g.sender_perm,
                                   g.sender_ptr, 3, _lib.BASIS_CHEBYSHEV_COSINE, 8, 0.0, 5.0, 6)
    assert_close(a2, attrs, 1e-5, 1e-5, "edge attrs")
    assert_close(f2, feats, 1e-5, 5e-5, "edge feats")
    assert_close(e2, env, 1e-5, 1e-6, "edge env")
    loss2 = (a2 * ga.float().to(DEV)).sum() + (f2 * gf.float().to(DEV)).sum() + (e2 * ge.float().to(DEV)).sum()
    (gpos,) = torch.autograd.grad(loss2, pos)
    assert_close(gpos, ref_gpos, 1e-4, 1e-4 * (float(ref_gpos.abs().max()) + 1), "edge grad positions")


def test_segment_sum():
    ops = _ops()
    torch.manual_seed(3)
    counts = torch.tensor([0, 5, 1, 17, 0, 3])
    ptr = torch.cat([torch.zeros(1, dtype=torch.long), counts.cumsum(0)])
    index = torch.repeat_interleave(torch.arange(len(counts)), counts)
    src = torch.randn(int(counts.sum()), dtype=torch.float64)
    ref = O.scatter_sum(src, index, len(counts))
    out = ops.segment_sum(src.float().to(DEV), ptr.to(DEV), index.to(DEV))
    assert_close(out, ref, 1e-6, 1e-6, "segment sum")


@pytest.mark.parametrize("l_max,C", [(0, 128), (1, 16), (2, 128), (3, 128), (3, 40)])
def test_rms_norm(l_max, C):
    """Fused RMS norm (forward, input and gain gradients) against the oracle's
    RMSLayerNorm restatement in float64."""
    ops = _ops()
    from oracle.model import rms_norm as ref_norm
    torch.manual_seed(l_max * 7 + C)
    n = 300
    x64 = (torch.randn(n, (l_max + 1) ** 2 * C, dtype=torch.float64) * torch.rand(n, 1, dtype=torch.float64) * 3)
    x64.requires_grad_(True)
    g64 = [(1.0 + 0.3 * torch.randn(C, dtype=torch.float64)).requires_grad_(True) for _ in range(l_max + 1)]
    sd = {f"ln.weights.{l}": g64[l] for l in range(l_max + 1)}
    ref = ref_norm(sd, "ln", x64, l_max, C)
    go = torch.randn_like(ref)
    ref_g = torch.autograd.grad(ref, [x64] + g64, go)
    x = x64.detach().float().to(DEV).requires_grad_(True)
    w = torch.stack([g.detach() for g in g64]).float().to(DEV).requires_grad_(True)
    out, _ = ops.rms_norm(x, w, l_max, 1e-6)
    gx, gw = torch.autograd.grad(out, [x, w], go.float().to(DEV))
    assert_close(out, ref, 2e-5, 2e-5 * float(ref.abs().max()), "rms fwd")
    assert_close(gx, ref_g[0], 1e-4, 1e-4 * float(ref_g[0].abs().max()), "rms grad x")
    assert_close(gw, torch.stack(ref_g[1:]), 1e-4, 1e-4 * float(torch.stack(ref_g[1:]).abs().max()), "rms grad g")


@pytest.mark.parametrize("lin,lout", [(3, 3), (2, 3), (3, 1)])
def test_linear_residual(lin, lout):
    """linear_fwd / linear_bwd with a residual added in the GEMM epilogue (ranks the map
    does not produce take the residual's values); gradients pass through to the residual."""
    ops = _ops()
    torch.manual_seed(9)
    n, fin, fout = 211, 16, 16
    in_dim = (lin + 1) ** 2 * fin
    out_dim = (lout + 1) ** 2 * fout
    x64 = torch.randn(n, in_dim, dtype=torch.float64, requires_grad=True)
    r64 = torch.randn(n, out_dim, dtype=torch.float64, requires_grad=True)
    ws64 = [torch.randn(fout, fin, dtype=torch.float64) for _ in range(min(lin, lout) + 1)]
    ref = O.linear(x64, ws64, lin, lout, fin, fout) + r64
    g = torch.randn_like(ref)
    ref_g = torch.autograd.grad(ref, [x64, r64], g)
    x = x64.detach().float().to(DEV).requires_grad_(True)
    r = r64.detach().float().to(DEV).requires_grad_(True)
    ws = [w.float().to(DEV) for w in ws64]
    scale = [fin ** -0.5] * len(ws)
    out = ops.linear_fwd(x, ws, lin, lout, fin, fout, [1] * (lin + 1), scale, 1.0, r)
    got = torch.autograd.grad(out, [x, r], g.float().to(DEV))
    assert_close(out, ref, 1e-5, 1e-4, "linear+residual fwd")
    assert_close(got[0], ref_g[0], 1e-5, 1e-4 * (float(ref_g[0].abs().max()) + 1), "linear+residual grad x")
    # pass-through: exactly the float32 upstream gradient
    assert_close(got[1], g.float().double(), 0.0, 0.0, "linear+residual grad residual")
    # dgrad with an accumulated gradient: gx = go @ W * s + acc
    acc = torch.randn(n, in_dim, device=DEV)
    gx = ops.linear_bwd(g.float().to(DEV), ws, lin, lout, fin, fout, [1] * (lin + 1), scale, 1.0, acc)
    plain = ops.linear_bwd(g.float().to(DEV), ws, lin, lout, fin, fout, [1] * (lin + 1), scale, 1.0)
    assert_close(gx, plain.double() + acc.double(), 1e-6, 1e-5, "dgrad + residual")


@pytest.mark.parametrize("l_max,act", [(3, 1), (2, 0), (0, 1)])
def test_gate(l_max, act):
    """Fused rank-wise gate against the reference formula (rescaled sigmoid, index_select,
    product) in float64, with both gradients."""
    ops = _ops()
    torch.manual_seed(l_max + 10 * act)
    n, C = 257, 64
    v64 = torch.randn(n, (l_max + 1) ** 2 * C, dtype=torch.float64, requires_grad=True)
    p64 = torch.randn(n, (l_max + 1) * C, dtype=torch.float64, requires_grad=True)
    gates = 1.8462285453386054 * torch.sigmoid(p64) if act == 1 else p64
    rank = torch.cat([torch.full((2 * l + 1,), l) for l in range(l_max + 1)])
    ref = (v64.view(n, -1, C) * gates.view(n, l_max + 1, C)[:, rank]).view(n, -1)
    g = torch.randn_like(ref)
    ref_g = torch.autograd.grad(ref, [v64, p64], g)
    v = v64.detach().float().to(DEV).requires_grad_(True)
    p = p64.detach().float().to(DEV).requires_grad_(True)
    out = ops.gate(v, p, l_max, act)
    got = torch.autograd.grad(out, [v, p], g.float().to(DEV))
    assert_close(out, ref, 1e-5, 1e-6, "gate fwd")
    assert_close(got[0], ref_g[0], 1e-5, 1e-6, "gate grad values")
    assert_close(got[1], ref_g[1], 1e-5, 1e-5 * float(ref_g[1].abs().max()), "gate grad pre")


@pytest.mark.parametrize("lin,lout,fin,fout,paths,n", [
    (3, 3, 128, 128, [1, 1, 1, 1], 3000),   # several row splits per rank, 128 x 128 tiles
    (2, 2, 16, 8, [1, 3, 2], 77),           # one split, 64 x 64 tiles, partial tiles
    (3, 1, 6, 10, [1, 1, 1, 1], 150),       # widths not multiples of 4: scalar loads
    (1, 2, 64, 200, [2, 1], 1200),
])
def test_linear_wgrad(lin, lout, fin, fout, paths, n):
    """Split-K MFMA weight gradients of the equivariant map against float64 sums of
    grad_out_l^T x_l, one rank per block of (2l+1) rows per node."""
    ops = _ops()
    g = torch.Generator().manual_seed(n + fin)
    common = min(lin, lout)
    in_dim = sum((2 * l + 1) * fin * paths[l] for l in range(lin + 1))
    out_dim = sum((2 * l + 1) * fout for l in range(lout + 1))
    x = torch.randn(n, in_dim, generator=g, dtype=torch.float64)
    go = torch.randn(n, out_dim, generator=g, dtype=torch.float64)
    ws = [torch.randn(fout, fin * paths[l], generator=g).to(DEV) for l in range(common + 1)]
    scale = [0.5 + l for l in range(common + 1)]
    with torch.no_grad():
        got = ops.linear_wgrad(go.float().to(DEV), x.float().to(DEV), ws, lin, lout, fin, fout, paths, scale, 0.75,
                               [True] * (common + 1))
    io = oo = 0
    for l in range(common + 1):
        k, m = fin * paths[l], 2 * l + 1
        xl = x[:, io:io + m * k].reshape(n * m, k)
        gl = go[:, oo:oo + m * fout].reshape(n * m, fout)
        want = gl.t() @ xl * (0.75 * scale[l])
        assert_close(got[l], want, 0.0, 2e-5 * float(want.abs().max()), f"wgrad rank {l}")
        io += m * k
        oo += m * fout
    with torch.no_grad():  # a subset of ranks
        part = ops.linear_wgrad(go.float().to(DEV), x.float().to(DEV), ws, lin, lout, fin, fout, paths, scale, 0.75,
                                [l == common for l in range(common + 1)])
    assert all(p is None for p in part[:common])
    assert_close(part[common], got[common].double(), 0.0, 0.0, "subset of ranks")


@pytest.mark.parametrize("n,k,m,act,bias", [(20000, 64, 2176, 0, False), (5000, 64, 64, 1, True),
                                            (333, 8, 64, 1, True), (90, 30, 17, 0, True)])
def test_dense_wgrad(n, k, m, act, bias):
    """Dense weight (and bias) gradients with the SiLU derivative applied to grad_out
    inside the kernel, against float64."""
    ops = _ops()
    g = torch.Generator().manual_seed(n + m)
    x = torch.randn(n, k, generator=g, dtype=torch.float64)
    go = torch.randn(n, m, generator=g, dtype=torch.float64)
    pre = torch.randn(n, m, generator=g, dtype=torch.float64)
    with torch.no_grad():
        gw, gb = ops.dense_wgrad(go.float().to(DEV), pre.float().to(DEV), act, x.float().to(DEV), 0.125, True, bias)
    h = go
    if act:
        s = torch.sigmoid(pre)
        h = go * 1.6765324703310907 * s * (1 + pre * (1 - s))
    want = h.t() @ x * 0.125
    assert_close(gw, want, 0.0, 2e-5 * float(want.abs().max()), "dense wgrad")
    if bias:
        wb = h.sum(0)
        assert_close(gb, wb, 0.0, 2e-5 * float(wb.abs().max()), "dense bias grad")
    else:
        assert gb is None


@pytest.mark.parametrize("lin,lout,fin,fout,in_paths", [(3, 3, 16, 16, [3, 5, 5, 4]), (3, 1, 8, 12, None),
                                                        (1, 3, 8, 8, None), (2, 0, 4, 8, [2, 3, 1])])
def test_reference_linear_ops(lin, lout, fin, fout, in_paths):
    """torch.ops.flashcart.linear_fwd / linear_bwd / linear_dbwd called with the reference's
    arguments (metadata, scale tensor and lists of o3.LinearLayer, as its triton_linear passes
    them, src/flashcart/o3/_linear.py:860-897) against the oracle: outputs, both gradients of
    linear_bwd, and the second derivatives reached through the registered autograd chain."""
    from flashcart_amd import o3
    import flashcart_amd.o3._second_order  # noqa: F401

    torch.manual_seed(3)
    lay = o3.LinearLayer(lin, lout, fin, fout, in_paths=in_paths).to(DEV)
    n = 37
    x = torch.randn(n, lay.in_dim, device=DEV, dtype=torch.float32)
    ws = [w.detach().clone() for w in lay.weight]
    args = (lay.meta, lay.out_dim, False, "ieee", *lay.meta_lists, lay.scale)
    out = torch.ops.flashcart.linear_fwd(x, ws, *args)
    xd = x.double().cpu().requires_grad_()
    wd = [w.double().cpu().requires_grad_() for w in ws]
    ref = O.linear(xd, wd, lin, lout, fin, fout, in_paths)
    _close(out, ref, "linear_fwd")
    go = torch.randn(n, lay.out_dim, device=DEV)
    gx, gws = torch.ops.flashcart.linear_bwd(go, x, ws, True, True, False, "ieee", *lay.meta_lists, lay.scale)
    rgx, *rgw = torch.autograd.grad(ref, [xd] + wd, go.double().cpu(), create_graph=True)
    _close(gx, rgx, "linear_bwd grad_x")
    for l, (a, b) in enumerate(zip(gws, rgw)):
        _close(a, b, f"linear_bwd grad_weight[{l}]")
    # second order through the registered autograd (linear_fwd -> linear_bwd -> linear_dbwd)
    xa = x.clone().requires_grad_()
    wa = [w.clone().requires_grad_() for w in ws]
    goa = go.clone().requires_grad_()
    o = torch.ops.flashcart.linear_fwd(xa, wa, *args)
    g1 = torch.autograd.grad(o, [xa] + wa, goa, create_graph=True)
    cots = [torch.randn_like(t) for t in g1]
    s2 = sum((a * c).sum() for a, c in zip(g1, cots))
    got2 = torch.autograd.grad(s2, [goa, xa] + wa, allow_unused=True)
    god = go.double().cpu().requires_grad_()
    rg1 = torch.autograd.grad(O.linear(xd, wd, lin, lout, fin, fout, in_paths), [xd] + wd, god, create_graph=True)
    rs2 = sum((a * c.double().cpu()).sum() for a, c in zip(rg1, cots))
    want2 = torch.autograd.grad(rs2, [god, xd] + wd, allow_unused=True)
    for k, (a, b) in enumerate(zip(got2, want2)):
        b = torch.zeros_like(a).double().cpu() if b is None else b
        _close(torch.zeros_like(b) if a is None else a, b, f"linear_dbwd input {k}")
    with pytest.raises(ValueError, match="dot_input_precision"):
        torch.ops.flashcart.linear_fwd(x, ws, lay.meta, lay.out_dim, False, "bf16", *lay.meta_lists, lay.scale)


def test_irreps_dbwd_op():
    """torch.ops.flashcart.irreps_dbwd (the Eq. (1) expansion's second derivative on the GPU)
    against double autograd of the oracle's expansion, l_max 0..3."""
    from tests.helpers import unit_vectors
    import flashcart_amd.o3._second_order  # noqa: F401

    for l_max in range(4):
        u = unit_vectors(300, seed=l_max)
        g = torch.randn(300, (l_max + 1) ** 2, dtype=torch.float64)
        v = torch.randn(300, 3, dtype=torch.float64)
        d_g, d_x = torch.ops.flashcart.irreps_dbwd(g.float().to(DEV), u.float().to(DEV), v.float().to(DEV), l_max)
        if l_max == 0:  # the expansion is the constant 1: both derivatives vanish
            assert float(d_g.abs().max()) == 0.0 and float(d_x.abs().max()) == 0.0
            continue
        ud = u.clone().requires_grad_()
        gd = g.clone().requires_grad_()
        (gx,) = torch.autograd.grad(O.irreps(ud, l_max), ud, gd, create_graph=True)
        want_g, want_x = torch.autograd.grad((gx * v).sum(), [gd, ud], allow_unused=True)
        _close(d_g, want_g, f"irreps_dbwd d_grad_output l={l_max}")
        _close(d_x, torch.zeros_like(ud) if want_x is None else want_x, f"irreps_dbwd d_x l={l_max}")


def test_shift_vectors_kernel():
    """fc_shift_vectors against the tensor-op sums it replaces, bit for bit: one cell and several
    cells; the translation of -S is the exact negation of that of S; a structure index out of range
    gives NaN rows; a differentiated cell keeps the tensor ops (and its gradient)."""
    from flashcart_amd.o3 import _ops
    from flashcart_amd.utils.geometry import shift_vectors

    def torch_sums(cell, shifts, idx_i, batch):
        s = shifts.to(cell.dtype)
        c = cell[0].unsqueeze(0) if cell.shape[0] == 1 else cell[batch[idx_i]]
        return s[:, 0:1] * c[:, 0] + s[:, 1:2] * c[:, 1] + s[:, 2:3] * c[:, 2]

    g = torch.Generator().manual_seed(11)
    n_nodes, n_edges = 300, 5000
    shifts = torch.randint(-3, 4, (n_edges, 3), generator=g)
    idx_i = torch.randint(0, n_nodes, (n_edges,), generator=g)
    batch = torch.sort(torch.randint(0, 4, (n_nodes,), generator=g)).values
    for n_cells in (1, 4):
        cell = (torch.randn(n_cells, 3, 3, generator=g) * 4.0 + 7.0 * torch.eye(3)).to(DEV)
        args = (shifts.to(DEV), idx_i.to(DEV), batch.to(DEV))
        print(f"shift vectors: {n_cells} cells, {n_edges} edges", flush=True)
        got = _ops.shift_vectors(cell, args[0], args[1], args[2])
        assert torch.equal(got, torch_sums(cell, *args))
        assert torch.equal(shift_vectors(cell, args[0], args[1], args[2], antisymmetric=True), got)
        assert torch.equal(_ops.shift_vectors(cell, -args[0], args[1], args[2]), -got)
    bad = batch.clone()
    bad[int(idx_i[7])] = 9
    got = _ops.shift_vectors(cell, shifts.to(DEV), idx_i.to(DEV), bad.to(DEV))
    rows = (bad[idx_i] == 9).to(DEV)
    assert torch.isnan(got[rows]).all() and not torch.isnan(got[~rows]).any()
    assert _ops.shift_vectors(cell[:1], shifts[:0].to(DEV), None, None).shape == (0, 3)
    # a differentiated cell: tensor ops, with the cell gradient
    cg = cell.clone().requires_grad_(True)
    sv = shift_vectors(cg, shifts.to(DEV), idx_i.to(DEV), batch.to(DEV), antisymmetric=True)
    assert sv.grad_fn is not None and torch.equal(sv.detach(), torch_sums(cell, shifts.to(DEV), idx_i.to(DEV),
                                                                          batch.to(DEV)))
