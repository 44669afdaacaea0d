"""Second derivatives: autograd formulas for the first-order backward ops.

Training with a force loss differentiates F = -dE/dR once more, i.e. differentiates
every backward op of the energy graph (the reference's ``*_dbwd`` ops,
src/flashcart/o3/_tensor_product.py:1095-1096, src/flashcart/o3/_linear.py:777-778,
src/flashcart/o3/_irreps.py:201-202).

* ``tp_bwd``: the product is linear in each of (grad_out, in1, in2, weights), so the
  derivative of <c1, g1> + <c2, g2> + <cw, gw> is again a set of products of the same
  configuration with one operand replaced by a cotangent: three ``tp_fwd`` (for
  grad_out) and up to three ``tp_bwd`` calls, each a HIP kernel launch.
* ``linear_bwd`` (the dgrad GEMM) is linear in grad_out and the weights: its derivative
  is ``linear_fwd`` of the cotangent and a weight-gradient GEMM.
* ``dense_bwd``: explicit formulas with the rescaled SiLU's first and second derivative.
* ``rms_norm_bwd``, ``gate_bwd`` and ``edge_geometry_bwd``: closed-form second
  derivatives in one kernel each (``fc_rms_norm_dbwd``, ``fc_gate_dbwd`` per node,
  ``fc_edge_geometry_dbwd`` per edge).
* the standalone ``irreps_bwd`` and ``radial_bwd``: differentiate their torch
  restatements twice (``_torch_math.vjp_of_vjp``).

Importing this module registers the formulas on the ``flashcart::*`` ops.
"""

from __future__ import annotations

import torch

from flashcart_amd.o3 import _ops
from flashcart_amd.o3 import _torch_math as M

Tensor = torch.Tensor


def _live(t):
    """A cotangent that carries information (not None, not the empty stand-in tensor)."""
    return t if (t is not None and t.numel() > 0) else None


def _acc(*terms):
    out = None
    for t in terms:
        if t is None or t.numel() == 0:
            continue
        out = t if out is None else out + t
    return out


# ---------------------------------------------------------------------------
# Tensor product
# ---------------------------------------------------------------------------

def _tp_bwd_setup(ctx, inputs, output):
    (go, in1, in2, w, idx_i, idx_j, l1, l2, lo, f1, f2, sym, shared, o1, o2, osz, npl, ntot, red,
     n1, n2, nw, rowptr, sperm, sptr, alpha, pair_slot, alpha_div) = inputs
    ctx.save_for_backward(go, in1, in2, w, idx_i, idx_j, rowptr, sperm, sptr, alpha_div)
    ctx.paired = pair_slot is not None
    ctx.cfg = (int(l1), int(l2), int(lo), int(f1), int(f2), bool(sym), bool(shared), list(o1), list(o2),
               list(osz), list(npl), int(ntot), bool(red))
    ctx.alpha = float(alpha)
    ctx.computed = (bool(n1), bool(n2), bool(nw))


def _conv_bwd_specialised(cfg, conv: bool) -> bool:
    """Whether fc_tp_bwd runs a convolution of this configuration on its compile-time
    specialised kernel when the weight and in2 gradients are both requested: per-edge
    weights, one in2 channel, unreduced outputs, 32, 64 or 128 in1 channels, in2 rank >= 1,
    no symmetric product (the launcher's conditions in csrc/fc_tp_impl.h)."""
    l1, l2, lo, f1, f2, sym, shared = cfg[:7]
    red = cfg[12]
    return conv and not shared and not red and not sym and f2 == 1 and f1 in (32, 64, 128) and l2 >= 1


def _tp_dbwd(ctx, c1, c2, cw):
    """Backward of tp_bwd (reference tp_dbwd, src/flashcart/o3/_tensor_product.py:789-1093)."""
    go, in1, in2, w, ii, jj, rp, sp, sq, adiv = ctx.saved_tensors
    need = ctx.needs_input_grad
    c1 = _live(c1) if ctx.computed[0] else None
    c2 = _live(c2) if ctx.computed[1] else None
    cw = _live(cw) if ctx.computed[2] else None
    cfg, alpha = ctx.cfg, ctx.alpha
    tail = (None,) * 24
    if ctx.paired:
        raise NotImplementedError("second derivatives of a tensor product with shared pair weights (pair_slot) "
                                  "are not implemented; run without edge pairs under create_graph.")

    def fwd(a, b, ww):
        return _ops.tp_fwd(a, b, ww, ii, jj, *cfg, rp, sp, sq, alpha, None, adiv)

    def bwd(a, b, ww, n1, n2, nw):
        if not (n1 or n2 or nw):
            return None, None, None
        g1, g2, gw = _ops.tp_bwd(go, a, b, ww, ii, jj, *cfg, bool(n1), bool(n2), bool(nw), rp, sp, sq, alpha,
                                 None, adiv)
        return (g1 if n1 else None), (g2 if n2 else None), (gw if nw else None)

    d_go = None
    if need[0]:
        terms = [t for t in ((c1, in2, w), (in1, c2, w), (in1, in2, cw)) if t[0] is not None and t[1] is not None
                 and t[2] is not None]
        d_go = _acc(*[fwd(*t) for t in terms]) if terms else None
    a = bwd(c1, in2, w, False, need[2], need[3]) if c1 is not None else (None,) * 3
    # the in2 gradient of the second product is not needed; asking for it anyway lets an
    # interaction-layer convolution take the kernel specialised for (in1, in2, weight) gradients
    b = bwd(in1, c2, w, need[1], _conv_bwd_specialised(cfg, ii is not None) and bool(need[3]), need[3]) \
        if c2 is not None else (None,) * 3
    b = (b[0], None, b[2])
    c = bwd(in1, in2, cw, need[1], need[2], False) if cw is not None else (None,) * 3
    d_in1 = _acc(b[0], c[0]) if need[1] else None
    d_in2 = _acc(a[1], c[1]) if need[2] else None
    d_w = _acc(a[2], b[2]) if need[3] else None
    return (d_go, d_in1, d_in2, d_w) + tail


_ops._register_autograd(_ops.tp_bwd, _tp_dbwd, _tp_bwd_setup)


# ---------------------------------------------------------------------------
# Equivariant linear map
# ---------------------------------------------------------------------------

def _linear_bwd_setup(ctx, inputs, output):
    go, w0, w1, w2, w3, w4, in_l_max, out_l_max, fin, fout, in_paths, scale, alpha, residual = inputs
    ws = _ops._wlist(w0, w1, w2, w3, w4)
    ctx.save_for_backward(go, *ws)
    ctx.cfg = (int(in_l_max), int(out_l_max), int(fin), int(fout), list(in_paths), list(scale))
    ctx.alpha = float(alpha)


def _linear_dbwd(ctx, c):
    """Backward of linear_bwd (reference linear_dbwd, src/flashcart/o3/_linear.py:540-760):
    gx_l = a s_l go_l W_l, so d/d go = linear_fwd(c) and d/dW_l = a s_l go_l^T c_l."""
    go, *weights = ctx.saved_tensors
    in_l_max, out_l_max, fin, fout, in_paths, scale = ctx.cfg
    need = ctx.needs_input_grad
    d_go = None
    if need[0]:
        d_go = _ops.linear_fwd(c, weights, in_l_max, out_l_max, fin, fout, in_paths, scale, ctx.alpha)
    d_ws = [None] * _ops._lib.MAX_RANKS
    if any(need[1:1 + _ops._lib.MAX_RANKS]):
        d_ws = _ops.linear_wgrad(go, c, weights, in_l_max, out_l_max, fin, fout, in_paths, scale, ctx.alpha,
                                 [bool(need[1 + l]) for l in range(len(weights))])
        d_ws = d_ws + [None] * (_ops._lib.MAX_RANKS - len(d_ws))
    i_res = 8 + _ops._lib.MAX_RANKS
    d_res = c if len(need) > i_res and need[i_res] else None
    return (d_go, *d_ws) + (None,) * 7 + (d_res,)


_ops._register_autograd(_ops.linear_bwd_op, _linear_dbwd, _linear_bwd_setup)


# ---------------------------------------------------------------------------
# Dense layer
# ---------------------------------------------------------------------------

def _dense_bwd_setup(ctx, inputs, output):
    go, pre, weight, scale, act = inputs
    ctx.save_for_backward(go, pre, weight)
    ctx.scale = float(scale)
    ctx.act = int(act)


def _dense_dbwd(ctx, c):
    """gx = s * h @ W with h = go * f'(pre) (h = go without activation):
    dh = s * c @ W^T, d go = dh * f'(pre), d pre = dh * go * f''(pre), dW = s * h^T @ c."""
    go, pre, w = ctx.saved_tensors
    need = ctx.needs_input_grad
    m, k = w.shape
    c2 = c.reshape(-1, k)
    go2 = go.reshape(-1, m)
    d_go = d_pre = d_w = None
    dh = None
    if need[0] or (ctx.act and need[1]):
        dh, _ = _ops.dense_fwd(c2, w, None, ctx.scale, 0)
    if ctx.act:
        p2 = pre.reshape(-1, m)
        if not torch.is_grad_enabled() and (need[0] or need[1]):  # one elementwise pass for both
            d_go, d_pre = _ops.silu_grad_mix(dh, p2, b=go2, need1=bool(need[0]), need2=bool(need[1]))
            d_go = d_go.reshape(go.shape) if d_go is not None else None
            d_pre = d_pre.reshape(pre.shape) if d_pre is not None else None
        else:
            if need[0]:
                d_go = (dh * M.silu_grad(p2)).reshape(go.shape)
            if need[1]:
                d_pre = (dh * go2 * M.silu_grad2(p2)).reshape(pre.shape)
    elif need[0]:
        d_go = dh.reshape(go.shape)
    if need[2]:  # s * h^T c with h = go * act'(pre)
        d_w, _ = _ops.dense_wgrad(go2, pre.reshape(-1, m) if ctx.act else None, ctx.act, c2, ctx.scale, True,
                                  False)
    return d_go, d_pre, d_w, None, None


_ops._register_autograd(_ops.dense_bwd, _dense_dbwd, _dense_bwd_setup)


# ---------------------------------------------------------------------------
# Eq. (1) expansion and radial basis
# ---------------------------------------------------------------------------

def _irreps_bwd_setup(ctx, inputs, output):
    g, x, l_max = inputs
    ctx.save_for_backward(g, x)
    ctx.l_max = int(l_max)


def _irreps_dbwd(ctx, c):
    """Backward of irreps_bwd: the irreps_dbwd op (reference src/flashcart/o3/_irreps.py:146-199)."""
    g, x = ctx.saved_tensors
    need = ctx.needs_input_grad
    if c is None or not (need[0] or need[1]):
        return None, None, None
    d_g, d_x = _ops.irreps_dbwd(g, x, c, ctx.l_max)
    return (d_g if need[0] else None), (d_x if need[1] else None), None


_ops._register_autograd(_ops.irreps_bwd, _irreps_dbwd, _irreps_bwd_setup)


def _radial_bwd_setup(ctx, inputs, output):
    d, g_feats, g_env, basis, n_radial, r_min, r_max, poly_order = inputs
    ctx.save_for_backward(d, g_feats, g_env)
    ctx.cfg = (int(basis), int(n_radial), float(r_min), float(r_max), int(poly_order))


def _radial_dbwd(ctx, c):
    d, gf, ge = ctx.saved_tensors
    basis, n_radial, r_min, r_max, poly_order = ctx.cfg
    need = ctx.needs_input_grad
    gf = _live(gf) if basis != _ops._lib.BASIS_NONE else None
    ge = _live(ge) if poly_order > 0 else None

    def fn(dd):
        return (M.radial_basis(dd, basis, n_radial, r_min, r_max) if gf is not None else None,
                M.envelope(dd, r_max, poly_order) if ge is not None else None)

    gp, gg = M.vjp_of_vjp(fn, [d], [0], [gf, ge], [c], [need[0]], [need[1], need[2]])
    return (gp[0], gg[0], gg[1]) + (None,) * 5


_ops._register_autograd(_ops.radial_bwd, _radial_dbwd, _radial_bwd_setup)


# ---------------------------------------------------------------------------
# Fused edge geometry
# ---------------------------------------------------------------------------

def _edge_bwd_setup(ctx, inputs, output):
    (g_attrs, g_feats, g_env, positions, shift_vec, idx_i, idx_j, vectors, rowptr, sperm, sptr) = inputs[:11]
    ctx.save_for_backward(g_attrs, g_feats, g_env, positions, shift_vec, idx_i, idx_j, vectors, rowptr, sperm, sptr)
    ctx.cfg = tuple(inputs[11:17])
    ctx.computed_pos = bool(inputs[17]) and positions is not None


def _edge_dbwd(ctx, c_pos, c_vec):
    """gvec = d<g, geometry(v)>/dv and gpos = its scatter onto the atoms (v = R_j - R_i + shift),
    so <c_pos, gpos> + <c_vec, gvec> = <c_vec + c_pos[j] - c_pos[i], gvec>: one per-edge
    kernel (``fc_edge_geometry_dbwd``) for the Hessian-vector product and the gradients of
    the upstream gradients, and the node scatter of the first-order backward for positions."""
    _no_third("the edge geometry")
    g_attrs, g_feats, g_env, positions, shift_vec, idx_i, idx_j, vectors, rowptr, sperm, sptr = ctx.saved_tensors
    l_max, basis, n_radial, r_min, r_max, poly_order = ctx.cfg
    need = ctx.needs_input_grad
    L = _ops._lib
    cv = _live(c_vec)
    cp = _live(c_pos) if ctx.computed_pos else None
    if cp is not None:
        ii, jj = idx_i.to(torch.int64), idx_j.to(torch.int64)
        cv = _acc(cv, cp.index_select(0, jj) - cp.index_select(0, ii))
    if cv is None:
        return (None,) * 18
    gs = [_live(g_attrs), _live(g_feats) if basis != L.BASIS_NONE else None,
          _live(g_env) if poly_order > 0 else None]
    gs = [L.contig(name, t) if t is not None else None for name, t in zip(("g_attrs", "g_feats", "g_env"), gs)]
    E = idx_i.shape[0]
    ref = cv
    d_ga = ref.new_empty(E, (l_max + 1) ** 2) if need[0] else None
    d_gf = ref.new_empty(E, n_radial) if (need[1] and basis != L.BASIS_NONE) else None
    d_ge = ref.new_empty(E) if (need[2] and poly_order > 0) else None
    need_v = need[3] or need[4] or need[7]
    hv = ref.new_empty(E, 3) if need_v else None
    pos = L.contig("positions", positions) if positions is not None else None
    sv = L.contig("shift_vec", shift_vec) if shift_vec is not None else None
    vec = L.contig("vectors", vectors) if vectors is not None else None
    desc = _ops._edge_desc(l_max, basis, n_radial, r_min, r_max, poly_order)
    # converted copies stay referenced until the launch has read their addresses
    ii32, jj32, cvc = _ops._i32("idx_i", idx_i), _ops._i32("idx_j", idx_j), L.contig("cotangent", cv)
    _ops._lib_call("fc_edge_geometry_dbwd", desc, E, L.ptr(pos), L.ptr(sv), ii32.data_ptr(), jj32.data_ptr(),
                   L.ptr(vec), *(L.ptr(t) for t in gs), cvc.data_ptr(), L.ptr(d_ga), L.ptr(d_gf), L.ptr(d_ge),
                   L.ptr(hv), L.stream_of(cvc))
    d_pos = d_shift = d_vec = None
    if hv is not None:
        if need[3] and positions is not None:
            d_pos = _ops.edge_grad_to_nodes(hv, positions.shape[0], idx_i, idx_j, rowptr, sperm, sptr)
        if need[4] and shift_vec is not None:
            d_shift = hv
        if need[7] and vectors is not None:
            d_vec = hv
    return (d_ga, d_gf, d_ge, d_pos, d_shift, None, None, d_vec) + (None,) * 10


_ops._register_autograd(_ops.edge_geometry_bwd, _edge_dbwd, _edge_bwd_setup)


# ---------------------------------------------------------------------------
# RMS norm and gate
# ---------------------------------------------------------------------------

def _rms_bwd_setup(ctx, inputs, output):
    go, x, weight, scale, l_max = inputs
    ctx.save_for_backward(go, x, weight, scale)
    ctx.l_max = int(l_max)


def _no_third(name: str) -> None:
    if torch.is_grad_enabled():
        raise NotImplementedError(f"third derivatives of {name} are not provided "
                                  "(a second-order backward was run with create_graph=True).")


def _rms_dbwd(ctx, c):
    """Backward of rms_norm_bwd: one node-wise kernel (``fc_rms_norm_dbwd``) for the
    gradients with respect to grad_out and x and each node's share of the gain gradient."""
    _no_third("the RMS norm")
    go, x, weight, scale = ctx.saved_tensors
    need = ctx.needs_input_grad
    if c is None or not any(need[:3]):
        return None, None, None, None, None
    n, C, l_max = x.shape[0], weight.shape[-1], ctx.l_max
    g = _ops._lib.contig("grad_out", go)
    xx = _ops._lib.contig("x", x)
    cc = _ops._lib.contig("cotangent", c)
    w = _ops._lib.contig("weight", weight)
    sc = _ops._lib.contig("scale", scale)
    d_go = torch.empty_like(xx) if need[0] else None
    d_x = torch.empty_like(xx) if need[1] else None
    part = xx.new_empty(n, l_max + 1, C) if need[2] else None
    _ops._lib_call("fc_rms_norm_dbwd", n, l_max, C, g.data_ptr(), xx.data_ptr(), w.data_ptr(), sc.data_ptr(),
                   cc.data_ptr(), _ops._lib.ptr(d_go), _ops._lib.ptr(d_x), _ops._lib.ptr(part),
                   _ops._lib.stream_of(xx))
    return d_go, d_x, (part.sum(0) if part is not None else None), None, None


_ops._register_autograd(_ops.rms_norm_bwd, _rms_dbwd, _rms_bwd_setup)


def _gate_bwd_setup(ctx, inputs, output):
    go, values, pre, l_max, act, need_values, need_pre = inputs
    ctx.save_for_backward(go, values, pre)
    ctx.cfg = (int(l_max), int(act))
    ctx.computed = (bool(need_values), bool(need_pre))


def _gate_dbwd(ctx, c_values, c_pre):
    """Backward of gate_bwd: one elementwise kernel (``fc_gate_dbwd``)."""
    _no_third("the gate")
    go, values, pre = ctx.saved_tensors
    l_max, act = ctx.cfg
    need = ctx.needs_input_grad
    cv = _live(c_values) if ctx.computed[0] else None
    cp = _live(c_pre) if ctx.computed[1] else None
    if (cv is None and cp is None) or not any(need[:3]):
        return None, None, None, None, None, None, None
    L = _ops._lib
    g = L.contig("grad_out", go)
    v = L.contig("values", values)
    p = L.contig("pre", pre)
    cv = L.contig("cot_values", cv) if cv is not None else None
    cp = L.contig("cot_pre", cp) if cp is not None else None
    d_go = torch.empty_like(g) if need[0] else None
    d_v = torch.empty_like(v) if need[1] else None
    d_p = torch.empty_like(p) if need[2] else None
    C = p.shape[-1] // (l_max + 1)
    _ops._lib_call("fc_gate_dbwd", v.shape[0], l_max, C, g.data_ptr(), v.data_ptr(), p.data_ptr(), int(act),
                   L.ptr(cv), L.ptr(cp), L.ptr(d_go), L.ptr(d_v), L.ptr(d_p), L.stream_of(v))
    return d_go, d_v, d_p, None, None, None, None


_ops._register_autograd(_ops.gate_bwd, _gate_dbwd, _gate_bwd_setup)
