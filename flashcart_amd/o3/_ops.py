"""PyTorch custom operators backed by the HIP C ABI (``torch.ops.flashcart.*``).

Op names follow the reference's registered operators
(src/flashcart/o3/_tensor_product.py:332,588; src/flashcart/o3/_irreps.py:84,117;
src/flashcart/o3/_linear.py:328,457) so call sites read the same. Each op has a
shape-only fake implementation (for torch.compile / meta tracing) and a registered
autograd formula whose backward is another HIP op. The backward ops' own autograd
formulas (second derivatives, for training with force losses) are registered by
``flashcart_amd.o3._second_order``, imported at the end of this module.

Every implementation checks that its tensors are float32 on a ROCm device and
raises otherwise; there is no CPU path.
"""

from __future__ import annotations

import contextlib
from typing import List, Optional, Tuple

import torch

from flashcart_amd import _lib
from flashcart_amd.codegen.cartesian import count_output_paths
from flashcart_amd.o3 import _torch_math

Tensor = torch.Tensor


# MFMA entry points of the library and the algorithmic FLOPs of one call, from its arguments:
# equivariant maps sum 2 n (2l+1) (C_in paths_l) C_out over the ranks both sides have; dense layers
# 2 n k m; the pair-sum GEMM 2 P m k (after the pair sum); the radial MLP kernels count each layer
# they run (the backward recomputes the two hidden layers, then multiplies back through both).
def _linear_flops(args):
    d, n = args[0], int(args[1])
    lm = min(d.in_l_max, d.out_l_max)
    return sum(2.0 * n * (2 * l + 1) * d.in_features * d.in_paths[l] * d.out_features for l in range(lm + 1))


def _linear_shape(args):
    d, n = args[0], int(args[1])
    lm = min(d.in_l_max, d.out_l_max)
    ks = [d.in_features * d.in_paths[l] for l in range(lm + 1)]
    return f"rows n(2l+1), n={n}, l<={lm}, K per rank={ks}, N={d.out_features}"


def _dense_shape(a):
    return f"M={int(a[0])}, K={int(a[1])}, N={int(a[2])}"


_MFMA_CALLS = {
    "fc_linear_fwd": ("equivariant_linear", _linear_flops, _linear_shape),
    "fc_linear_dgrad": ("equivariant_linear", _linear_flops, _linear_shape),
    "fc_linear_wgrad": ("equivariant_linear", _linear_flops, _linear_shape),
    "fc_dense_fwd": ("dense", lambda a: 2.0 * a[0] * a[1] * a[2], _dense_shape),
    "fc_dense_dgrad": ("dense", lambda a: 2.0 * a[0] * a[1] * a[2], _dense_shape),
    "fc_dense_wgrad": ("dense", lambda a: 2.0 * a[0] * a[1] * a[2], _dense_shape),
    "fc_dense_fwd_pairsum": ("dense", lambda a: 2.0 * a[0] * a[1] * a[2],
                             lambda a: f"pairs={int(a[0])}, K={int(a[1])} (summed row pair), N={int(a[2])}"),
    "fc_radial_mlp_fwd": ("radial_mlp", lambda a: 2.0 * a[0] * (a[1] * 64 + 64 * 64 + 64 * a[7]),
                          lambda a: f"rows={int(a[0])}, {int(a[1])}->64->64->{int(a[7])}"),
    "fc_radial_mlp_hidden_fwd": ("radial_mlp", lambda a: 2.0 * a[0] * (a[1] * 64 + 64 * 64),
                                 lambda a: f"rows={int(a[0])}, {int(a[1])}->64->64"),
    "fc_radial_mlp_bwd": ("radial_mlp", lambda a: 2.0 * a[0] * (2 * a[1] * 64 + 2 * 64 * 64),
                          lambda a: f"rows={int(a[0])}, 64->64->{int(a[1])} (hidden layers recomputed)"),
    "fc_radial_mlp_bwd_pairsum": ("radial_mlp", lambda a: 2.0 * a[0] * (2 * a[1] * 64 + 2 * 64 * 64),
                                  lambda a: f"pairs={int(a[0])}, 64->64->{int(a[1])} (hidden layers recomputed)"),
}
_mfma_record: Optional[list] = None


@contextlib.contextmanager
def mfma_timer():
    """Within the context, every launch of an MFMA kernel family of the library (equivariant
    linear maps, dense layers, radial MLP) is bracketed by HIP events on the stream it runs on,
    and (name, group, flops, start event, end event, shape) is appended to the yielded list: the
    in-step MFMA time and achieved FLOP/s of the linear maps (bench.py). Not during graph capture."""
    global _mfma_record
    prev, rec = _mfma_record, []
    _mfma_record = rec
    try:
        yield rec
    finally:
        _mfma_record = prev


def _lib_call(name: str, *args) -> None:
    lib = _lib.load()
    rec = _mfma_record
    if rec is not None and name in _MFMA_CALLS and not torch.cuda.is_current_stream_capturing():
        group, flops, shape = _MFMA_CALLS[name]
        stream = torch.cuda.current_stream()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        _lib.check(getattr(lib, name)(*args), name)
        e1.record(stream)
        rec.append((name, group, float(flops(args)), e0, e1, shape(args)))
        return
    _lib.check(getattr(lib, name)(*args), name)


def _i32(name: str, t: Optional[Tensor]) -> Optional[Tensor]:
    if t is None:
        return None
    if not t.is_cuda:
        raise RuntimeError(f"`{name}` must be on a ROCm device, got {t.device}.")
    if t.dtype != torch.int32:
        t = t.to(torch.int32)
    return t.contiguous()


def _tp_out_dim(in1_l_max, in2_l_max, out_l_max, in1_features, in2_features, symmetric, reduced) -> int:
    counts, _ = count_output_paths(in1_l_max, in2_l_max, out_l_max, symmetric)
    c = max(in1_features, in2_features)
    return sum((2 * l + 1) * (min(n, 1) if reduced else n) * c for l, n in enumerate(counts))


_META_LEN = 4  # ranks 0..3 compiled into the library


def tp_meta(in1_l_max: int, in2_l_max: int, out_l_max: int, in1_features: int, in2_features: int,
            symmetric_product: bool, reduce_paths: bool):
    """Layout lists of the reference's ``tp_fwd`` schema for the standard feature layout.

    Returns ``(in1_offs, in2_offs, out_sizes, n_paths_per_l, n_total_paths)``, each list
    padded with zeros to one entry per compiled rank, as the reference builds them
    (src/flashcart/o3/_tensor_product.py:51-72,1158-1164).
    """
    counts, total = count_output_paths(in1_l_max, in2_l_max, out_l_max, symmetric_product)
    c = max(in1_features, in2_features)

    def offs(l_max, f):
        return [l * l * f if l <= l_max else 0 for l in range(_META_LEN)]

    n_paths = [int(counts[l]) if l < len(counts) else 0 for l in range(_META_LEN)]
    sizes = [((2 * l + 1) * c if n > 0 else 0) if reduce_paths else n * (2 * l + 1) * c
             for l, n in enumerate(n_paths)]
    return offs(in1_l_max, in1_features), offs(in2_l_max, in2_features), sizes, n_paths, int(total)


# Engine queries used to narrow needs_input_grad; without them (another torch build) every
# statically required gradient is computed, which is correct, only slower.
_current_node = getattr(torch._C, "_current_autograd_node", None)
if not hasattr(torch._C, "_will_engine_execute_node"):
    _current_node = None


def param_alias(t: Optional[Tensor]) -> Optional[Tensor]:
    """A parameter as an op input: a view of it while autograd records, so that the backward
    can ask the engine whether the current pass needs the parameter's gradient (it cannot
    for the leaf itself inside ``autograd.grad``). No copy; the kernels read the same memory."""
    if t is not None and t.is_leaf and t.requires_grad and torch.is_grad_enabled():
        return t.view_as(t)
    return t


def _register_autograd(op, backward, setup_context) -> None:
    """``op.register_autograd`` with ``ctx.needs_input_grad`` narrowed, while the backward
    runs, to the inputs the running backward pass will actually use.

    The static flags say which inputs require grad; a pass such as
    ``autograd.grad(E, positions)`` (forces) needs none of the parameter gradients, so the
    weight-gradient GEMMs are skipped there. A gradient the pass does not use is dropped by
    the engine anyway, so returning None for it changes no result. The engine cannot answer
    for a leaf inside ``autograd.grad``; such an input keeps its static flag, which is why
    parameters are handed to the ops through ``param_alias``."""
    def setup(ctx, inputs, output):
        ctx.tensor_inputs = tuple(torch.is_tensor(a) for a in inputs)
        setup_context(ctx, inputs, output)

    def used(node) -> bool:
        if node is None:
            return False
        try:
            return bool(torch._C._will_engine_execute_node(node))
        except RuntimeError:  # a leaf's accumulator during autograd.grad: unknown
            return True

    def bwd(ctx, *grads):
        static = ctx.needs_input_grad
        node = _current_node() if _current_node is not None else None
        mask = ctx.tensor_inputs
        if node is not None and len(node.next_functions) == sum(mask):
            edges = iter(node.next_functions)
            need = []
            for k, is_tensor in enumerate(mask):
                nxt = next(edges)[0] if is_tensor else None
                need.append(bool(k < len(static) and static[k] and used(nxt)))
            ctx.needs_input_grad = tuple(need[:len(static)])
        try:
            return backward(ctx, *grads)
        finally:
            ctx.needs_input_grad = static

    op.register_autograd(bwd, setup_context=setup)


def _check_tp_meta(cfg, in1_offs, in2_offs, out_sizes, n_paths_per_l, n_total_paths) -> None:
    """The kernels implement the standard contiguous layout only; reject any other."""
    want = tp_meta(*cfg)
    got = (list(in1_offs), list(in2_offs), list(out_sizes), list(n_paths_per_l), int(n_total_paths))
    names = ("in1_offs", "in2_offs", "out_sizes", "n_paths_per_l", "n_total_paths")
    for name, g, w in zip(names, got, want):
        if isinstance(w, list):
            g = g + [0] * max(0, len(w) - len(g))
            if g[:len(w)] != w or any(v != 0 for v in g[len(w):]):
                raise ValueError(f"{name}={got[names.index(name)]} does not describe the standard layout {w}.")
        elif g != w:
            raise ValueError(f"{name}={g} does not match the configuration ({w}).")


# ---------------------------------------------------------------------------
# Eq. (1) expansion
# ---------------------------------------------------------------------------

@torch.library.custom_op("flashcart::irreps_fwd", mutates_args=())
def irreps_fwd(x: Tensor, l_max: int) -> Tensor:
    x = _lib.contig("x", x)
    out = x.new_empty(x.shape[0], (l_max + 1) ** 2)
    _lib_call("fc_irreps_fwd", x.shape[0], l_max, x.data_ptr(), out.data_ptr(), _lib.stream_of(x))
    return out


@irreps_fwd.register_fake
def _(x, l_max):
    return x.new_empty(x.shape[0], (l_max + 1) ** 2)


@torch.library.custom_op("flashcart::irreps_bwd", mutates_args=())
def irreps_bwd(grad_output: Tensor, x: Tensor, l_max: int) -> Tensor:
    g = _lib.contig("grad_output", grad_output)
    x = _lib.contig("x", x)
    gx = torch.empty_like(x)
    _lib_call("fc_irreps_bwd", x.shape[0], l_max, g.data_ptr(), x.data_ptr(), gx.data_ptr(), _lib.stream_of(x))
    return gx


@irreps_bwd.register_fake
def _(grad_output, x, l_max):
    return torch.empty_like(x)


@torch.library.custom_op("flashcart::irreps_dbwd", mutates_args=())
def irreps_dbwd(grad_output: Tensor, x: Tensor, v: Tensor, l_max: int) -> Tuple[Tensor, Tensor]:
    """Backward of irreps_bwd along v (reference flashcart::irreps_dbwd, o3/_irreps.py:146-176):
    (d grad_output = J(x) v, d x = sum_a grad_output_a H_a(x) v)."""
    x = _lib.contig("x", x)
    g = _lib.contig("grad_output", grad_output)
    vv = _lib.contig("v", v)
    d_g = x.new_empty(x.shape[0], (l_max + 1) ** 2)
    d_x = torch.empty_like(x)
    _lib_call("fc_irreps_dbwd", x.shape[0], l_max, g.data_ptr(), x.data_ptr(), vv.data_ptr(), d_g.data_ptr(),
              d_x.data_ptr(), _lib.stream_of(x))
    return d_g, d_x


@irreps_dbwd.register_fake
def _(grad_output, x, v, l_max):
    return x.new_empty(x.shape[0], (l_max + 1) ** 2), torch.empty_like(x)


def _irreps_setup(ctx, inputs, output):
    x, l_max = inputs
    ctx.save_for_backward(x)
    ctx.l_max = int(l_max)


def _irreps_backward(ctx, grad):
    (x,) = ctx.saved_tensors
    if not ctx.needs_input_grad[0]:
        return None, None
    return irreps_bwd(grad, x, ctx.l_max), None


_register_autograd(irreps_fwd, _irreps_backward, _irreps_setup)


# ---------------------------------------------------------------------------
# Radial basis and cutoff envelope
# ---------------------------------------------------------------------------

@torch.library.custom_op("flashcart::radial_fwd", mutates_args=())
def radial_fwd(d: Tensor, basis: int, n_radial: int, r_min: float, r_max: float, poly_order: int) -> Tuple[Tensor, Tensor]:
    """(feats (n, n_radial) or empty when basis is NONE, env (n,) or empty when poly_order == 0)."""
    d = _lib.contig("distances", d)
    n = d.shape[0]
    feats = d.new_empty(n, n_radial) if basis != _lib.BASIS_NONE else d.new_empty(0)
    env = d.new_empty(n) if poly_order > 0 else d.new_empty(0)
    desc = _lib.radial_desc(basis, n_radial, r_min, r_max, poly_order)
    _lib_call("fc_radial_fwd", desc, n, d.data_ptr(), _lib.ptr(feats) if feats.numel() else None,
              _lib.ptr(env) if env.numel() else None, _lib.stream_of(d))
    return feats, env


@radial_fwd.register_fake
def _(d, basis, n_radial, r_min, r_max, poly_order):
    n = d.shape[0]
    return (d.new_empty(n, n_radial) if basis != _lib.BASIS_NONE else d.new_empty(0),
            d.new_empty(n) if poly_order > 0 else d.new_empty(0))


@torch.library.custom_op("flashcart::radial_bwd", mutates_args=())
def radial_bwd(d: Tensor, g_feats: Optional[Tensor], g_env: Optional[Tensor], basis: int, n_radial: int,
               r_min: float, r_max: float, poly_order: int) -> Tensor:
    d = _lib.contig("distances", d)
    gf = _lib.contig("grad_feats", g_feats) if g_feats is not None and basis != _lib.BASIS_NONE else None
    ge = _lib.contig("grad_env", g_env) if g_env is not None and poly_order > 0 else None
    gd = torch.empty_like(d)
    desc = _lib.radial_desc(basis, n_radial, r_min, r_max, poly_order)
    _lib_call("fc_radial_bwd", desc, d.shape[0], d.data_ptr(), _lib.ptr(gf), _lib.ptr(ge), gd.data_ptr(),
              _lib.stream_of(d))
    return gd


@radial_bwd.register_fake
def _(d, g_feats, g_env, basis, n_radial, r_min, r_max, poly_order):
    return torch.empty_like(d)


def _radial_setup(ctx, inputs, output):
    d, basis, n_radial, r_min, r_max, poly_order = inputs
    ctx.save_for_backward(d)
    ctx.cfg = (int(basis), int(n_radial), float(r_min), float(r_max), int(poly_order))


def _radial_backward(ctx, g_feats, g_env):
    (d,) = ctx.saved_tensors
    if not ctx.needs_input_grad[0]:
        return (None,) * 6
    basis, n_radial, r_min, r_max, poly_order = ctx.cfg
    gf = g_feats if (g_feats is not None and g_feats.numel()) else None
    ge = g_env if (g_env is not None and g_env.numel()) else None
    return (radial_bwd(d, gf, ge, basis, n_radial, r_min, r_max, poly_order),) + (None,) * 5


_register_autograd(radial_fwd, _radial_backward, _radial_setup)


# ---------------------------------------------------------------------------
# Fused edge geometry (edge vectors -> expansion, radial basis, envelope)
# ---------------------------------------------------------------------------

def _edge_desc(l_max, basis, n_radial, r_min, r_max, poly_order):
    return _lib.EdgeDesc(int(l_max), _lib.radial_desc(basis, n_radial, r_min, r_max, poly_order))


def shift_vectors(cell: Tensor, shifts: Tensor, idx_i: Optional[Tensor], batch: Optional[Tensor]) -> Tensor:
    """Translation S . cell[batch[idx_i]] of every edge (``fc_shift_vectors``; reference
    ``utils/geometry.py:52``): each product and sum rounded on its own, so -S gives exactly the
    negated translation. No gradient: for a cell that is differentiated, form it with tensor ops.
    ``idx_i`` and ``batch`` are read only for several cells."""
    c = _lib.contig("cell", cell)
    if c.dim() != 3 or tuple(c.shape[1:]) != (3, 3):
        raise ValueError(f"cell must be (n_cells, 3, 3), got {tuple(c.shape)}.")
    if not shifts.is_cuda or shifts.device != c.device:
        raise RuntimeError(f"`shifts` must be on {c.device}, got {shifts.device}.")
    if shifts.dim() != 2 or shifts.shape[1] != 3:
        raise ValueError(f"shifts must be (n_edges, 3), got {tuple(shifts.shape)}.")
    sh = shifts if shifts.dtype == torch.int64 else shifts.to(torch.int64)
    sh = sh.contiguous()
    n_cells = int(c.shape[0])
    ii = _i32("idx_i", idx_i) if n_cells > 1 else None
    bb = _i32("batch", batch) if n_cells > 1 else None
    if n_cells > 1 and (ii is None or bb is None or ii.shape[0] != sh.shape[0]):
        raise ValueError("several cells need idx_i (one per edge) and batch.")
    out = torch.empty(sh.shape[0], 3, dtype=torch.float32, device=c.device)
    _lib_call("fc_shift_vectors", sh.shape[0], n_cells, sh.data_ptr(), c.data_ptr(), _lib.ptr(ii),
              _lib.ptr(bb), 0 if bb is None else bb.shape[0], out.data_ptr(), _lib.stream_of(c))
    return out


@torch.library.custom_op("flashcart::edge_geometry", mutates_args=())
def edge_geometry(positions: Optional[Tensor], shift_vec: Optional[Tensor], idx_i: Tensor, idx_j: Tensor,
                  vectors: Optional[Tensor], rowptr: Optional[Tensor], sender_perm: Optional[Tensor],
                  sender_ptr: Optional[Tensor], l_max: int, basis: int, n_radial: int, r_min: float, r_max: float,
                  poly_order: int) -> Tuple[Tensor, Tensor, Tensor]:
    """(edge_attrs (E, (l_max+1)^2), radial feats (E, n_radial), envelope (E,))."""
    ii = _i32("idx_i", idx_i)
    jj = _i32("idx_j", idx_j)
    pos = _lib.contig("positions", positions) if positions is not None else None
    sv = _lib.contig("shift_vec", shift_vec) if shift_vec is not None else None
    vec = _lib.contig("vectors", vectors) if vectors is not None else None
    ref = pos if pos is not None else vec
    if ref is None:
        raise ValueError("edge_geometry needs positions or vectors.")
    E = ii.shape[0]
    attrs = _lib.rows_empty(ref, E, (l_max + 1) ** 2)
    feats = _lib.rows_empty(ref, E, n_radial) if basis != _lib.BASIS_NONE else ref.new_empty(0)
    env = _lib.rows_empty(ref, E) if poly_order > 0 else ref.new_empty(0)
    desc = _edge_desc(l_max, basis, n_radial, r_min, r_max, poly_order)
    _lib_call("fc_edge_geometry_fwd", desc, E, _lib.ptr(pos), _lib.ptr(sv), ii.data_ptr(), jj.data_ptr(),
              _lib.ptr(vec), attrs.data_ptr(), _lib.ptr(feats) if feats.numel() else None,
              _lib.ptr(env) if env.numel() else None, _lib.stream_of(ref))
    return attrs, feats, env


@edge_geometry.register_fake
def _(positions, shift_vec, idx_i, idx_j, vectors, rowptr, sender_perm, sender_ptr, l_max, basis, n_radial, r_min,
      r_max, poly_order):
    ref = positions if positions is not None else vectors
    E = idx_i.shape[0]
    return (ref.new_empty(E, (l_max + 1) ** 2),
            ref.new_empty(E, n_radial) if basis != _lib.BASIS_NONE else ref.new_empty(0),
            ref.new_empty(E) if poly_order > 0 else ref.new_empty(0))


@torch.library.custom_op("flashcart::edge_geometry_bwd", mutates_args=())
def edge_geometry_bwd(g_attrs: Optional[Tensor], g_feats: Optional[Tensor], g_env: Optional[Tensor],
                      positions: Optional[Tensor], shift_vec: Optional[Tensor], idx_i: Tensor, idx_j: Tensor,
                      vectors: Optional[Tensor], rowptr: Optional[Tensor], sender_perm: Optional[Tensor],
                      sender_ptr: Optional[Tensor], l_max: int, basis: int, n_radial: int, r_min: float,
                      r_max: float, poly_order: int, need_positions: bool) -> Tuple[Tensor, Tensor]:
    """(grad_positions (N, 3) or empty, grad_vec (E, 3))."""
    ii = _i32("idx_i", idx_i)
    jj = _i32("idx_j", idx_j)
    pos = _lib.contig("positions", positions) if positions is not None else None
    sv = _lib.contig("shift_vec", shift_vec) if shift_vec is not None else None
    vec = _lib.contig("vectors", vectors) if vectors is not None else None
    ref = pos if pos is not None else vec
    ga = _lib.contig("grad_attrs", g_attrs) if g_attrs is not None else None
    gf = _lib.contig("grad_feats", g_feats) if (g_feats is not None and basis != _lib.BASIS_NONE) else None
    ge = _lib.contig("grad_env", g_env) if (g_env is not None and poly_order > 0) else None
    E = ii.shape[0]
    gvec = _lib.rows_empty(ref, E, 3)
    desc = _edge_desc(l_max, basis, n_radial, r_min, r_max, poly_order)
    stream = _lib.stream_of(ref)
    _lib_call("fc_edge_geometry_bwd", desc, E, _lib.ptr(pos), _lib.ptr(sv), ii.data_ptr(), jj.data_ptr(),
              _lib.ptr(vec), _lib.ptr(ga), _lib.ptr(gf), _lib.ptr(ge), gvec.data_ptr(), stream)
    if not need_positions or pos is None:
        return ref.new_empty(0), gvec
    return edge_grad_to_nodes(gvec, pos.shape[0], idx_i, idx_j, rowptr, sender_perm, sender_ptr), gvec


def edge_grad_to_nodes(gvec: Tensor, n_nodes: int, idx_i: Tensor, idx_j: Tensor, rowptr: Optional[Tensor],
                       sender_perm: Optional[Tensor], sender_ptr: Optional[Tensor]) -> Tensor:
    """Gradient of the positions from that of the edge vectors v = R_j - R_i (+ shift):
    sender sums minus receiver sums, as segmented sums in a fixed order (``fc_edge_grad_to_nodes``)."""
    if rowptr is None or sender_perm is None or sender_ptr is None:
        from flashcart_amd.o3._graph import build_graph
        gcsr = build_graph(torch.stack([idx_i, idx_j]), n_nodes, check_sorted=False)
        rowptr, sender_perm, sender_ptr = gcsr.rowptr, gcsr.sender_perm, gcsr.sender_ptr
    gv = _lib.contig("grad_vec", gvec)
    # int32 copies stay referenced until the launch has read their addresses
    jj, rp, sp, sq = (_i32("idx_j", idx_j), _i32("rowptr", rowptr), _i32("sender_perm", sender_perm),
                      _i32("sender_ptr", sender_ptr))
    gpos = gv.new_empty(n_nodes, 3)
    csr = _lib.csr_struct(n_nodes, jj.shape[0], jj, rp, sp, sq, n_nodes)
    _lib_call("fc_edge_grad_to_nodes", csr, gv.data_ptr(), gpos.data_ptr(), _lib.stream_of(gv))
    return gpos


@edge_geometry_bwd.register_fake
def _(g_attrs, g_feats, g_env, positions, shift_vec, idx_i, idx_j, vectors, rowptr, sender_perm, sender_ptr,
      l_max, basis, n_radial, r_min, r_max, poly_order, need_positions):
    ref = positions if positions is not None else vectors
    gp = ref.new_empty(positions.shape[0], 3) if (need_positions and positions is not None) else ref.new_empty(0)
    return gp, ref.new_empty(idx_i.shape[0], 3)


def _edge_setup(ctx, inputs, output):
    positions, shift_vec, idx_i, idx_j, vectors, rowptr, sender_perm, sender_ptr = inputs[:8]
    ctx.cfg = tuple(inputs[8:])
    ctx.save_for_backward(positions, shift_vec, idx_i, idx_j, vectors, rowptr, sender_perm, sender_ptr)


def _edge_backward(ctx, g_attrs, g_feats, g_env):
    positions, shift_vec, idx_i, idx_j, vectors, rowptr, sender_perm, sender_ptr = ctx.saved_tensors
    need_pos = ctx.needs_input_grad[0]
    need_shift = ctx.needs_input_grad[1]
    need_vec = ctx.needs_input_grad[4]
    if not (need_pos or need_shift or need_vec):
        return (None,) * 14
    gpos, gvec = edge_geometry_bwd(
        g_attrs, g_feats if (g_feats is not None and g_feats.numel()) else None,
        g_env if (g_env is not None and g_env.numel()) else None,
        positions, shift_vec, idx_i, idx_j, vectors, rowptr, sender_perm, sender_ptr, *ctx.cfg, bool(need_pos))
    return ((gpos if need_pos else None), (gvec if need_shift else None), None, None,
            (gvec if need_vec else None)) + (None,) * 9


_register_autograd(edge_geometry, _edge_backward, _edge_setup)


# ---------------------------------------------------------------------------
# Tensor product
# ---------------------------------------------------------------------------

def _alpha_div(t: Optional[Tensor]) -> Optional[Tensor]:
    """The divisor tensor of a tensor product: one float32 element on the device (contiguous)."""
    if t is None:
        return None
    if t.numel() != 1:
        raise ValueError(f"alpha_div must hold one element, got shape {tuple(t.shape)}.")
    return _lib.contig("alpha_div", t.detach().reshape(1))


def _tp_csr(in1: Tensor, idx_i: Tensor, idx_j: Tensor, rowptr: Optional[Tensor], sender_perm: Optional[Tensor],
            sender_ptr: Optional[Tensor], need_senders: bool, pair_slot: Optional[Tensor] = None,
            receivers: bool = False):
    """``receivers``: also pass each edge's receiver (``fc_csr.idx_i``), which lets the backward of a
    64-channel convolution run in sender order."""
    n = in1.shape[0]
    jj = _i32("idx_j", idx_j)
    if rowptr is None or (need_senders and (sender_perm is None or sender_ptr is None)):
        from flashcart_amd.o3._graph import build_graph
        g = build_graph(torch.stack([idx_i.to(torch.int64), idx_j.to(torch.int64)]), n)
        rowptr, sender_perm, sender_ptr = g.rowptr, g.sender_perm, g.sender_ptr
    rp = _i32("rowptr", rowptr)
    sp = _i32("sender_perm", sender_perm)
    sq = _i32("sender_ptr", sender_ptr)
    if rp.shape[0] != n + 1:
        raise ValueError(f"rowptr must have in1.shape[0] + 1 = {n + 1} entries, got {rp.shape[0]}.")
    ps = _i32("pair_slot", pair_slot)
    if ps is not None and ps.shape[0] != jj.shape[0]:
        raise ValueError(f"pair_slot must have one entry per edge ({jj.shape[0]}), got {ps.shape[0]}.")
    ii = _i32("idx_i", idx_i) if receivers else None
    keep = (jj, rp, sp, sq, ps, ii)
    return _lib.csr_struct(n, jj.shape[0], jj, rp, sp, sq, n, ps, ii), keep


def _check_tp_inputs(in1, in2, weights, idx_i, idx_j, in1_l_max, in2_l_max, out_l_max, in1_features,
                     in2_features, symmetric_product, shared_weights, paired=False):
    conv = idx_i is not None and idx_j is not None
    c = max(in1_features, in2_features)
    _, n_paths = count_output_paths(in1_l_max, in2_l_max, out_l_max, symmetric_product)
    if in1.shape[-1] != (in1_l_max + 1) ** 2 * in1_features or in2.shape[-1] != (in2_l_max + 1) ** 2 * in2_features:
        raise ValueError("tensor-product input widths do not match the configuration.")
    items = idx_i.shape[0] if conv else in1.shape[0]
    if conv:
        if in2.shape[0] != items or idx_j.shape[0] != items:
            raise ValueError("in2, idx_i and idx_j must have one row per edge.")
    elif in2.shape[0] != in1.shape[0]:
        raise ValueError("idx_i and idx_j must be provided when in1 and in2 have different batch sizes. "
                         f"Got in1_batch={in1.shape[0]}, in2_batch={in2.shape[0]}.")
    if paired and (shared_weights or not conv or items % 2):
        raise ValueError("pair_slot needs a convolution with per-edge weights over an even number of edges.")
    w_rows = items // 2 if paired else items
    if shared_weights:
        if weights.dim() != 1 or weights.shape[0] != n_paths * c:
            raise ValueError(f"Shared weights must be 1D of size {n_paths * c}, got {tuple(weights.shape)}.")
    elif weights.dim() != 2 or weights.shape[0] != w_rows or weights.shape[1] != n_paths * c:
        raise ValueError(f"Non-shared weights must have shape ({w_rows}, {n_paths * c}), got {tuple(weights.shape)}.")
    return conv


@torch.library.custom_op("flashcart::tp_fwd", mutates_args=())
def tp_fwd(in1: Tensor, in2: Tensor, weights: Tensor, idx_i: Optional[Tensor], idx_j: Optional[Tensor],
           in1_l_max: int, in2_l_max: int, out_l_max: int, in1_features: int, in2_features: int,
           symmetric_product: bool, shared_weights: bool, in1_offs: List[int], in2_offs: List[int],
           out_sizes: List[int], n_paths_per_l: List[int], n_total_paths: int, reduce_paths: bool = False,
           rowptr: Optional[Tensor] = None, sender_perm: Optional[Tensor] = None,
           sender_ptr: Optional[Tensor] = None, alpha: float = 1.0, pair_slot: Optional[Tensor] = None,
           alpha_div: Optional[Tensor] = None) -> Tensor:
    """Reference schema (src/flashcart/o3/_tensor_product.py:332-352) plus optional CSR
    arrays (``rowptr``, ``sender_perm``, ``sender_ptr``, see ``o3._graph``), ``alpha``,
    a scale applied to the output, ``pair_slot`` (``o3._graph.EdgePairs.slot``): the two
    edges of a pair read one weight row, so ``weights`` holds E / 2 rows, and ``alpha_div``, a
    one-element device tensor s: the output is then scaled by alpha / s, s read on the device
    (the interaction layers' ``aggregated / sqrt_avg_neighbors``, reference
    ``nn/layers.py:368``, without a host copy of the buffer)."""
    _check_tp_meta((in1_l_max, in2_l_max, out_l_max, in1_features, in2_features, symmetric_product, reduce_paths),
                   in1_offs, in2_offs, out_sizes, n_paths_per_l, n_total_paths)
    conv = _check_tp_inputs(in1, in2, weights, idx_i, idx_j, in1_l_max, in2_l_max, out_l_max, in1_features,
                            in2_features, symmetric_product, shared_weights, pair_slot is not None)
    in1 = _lib.contig("in1", in1)
    in2 = _lib.contig("in2", in2)
    w = _lib.contig("weights", weights)
    desc = _lib.tp_desc(in1_l_max, in2_l_max, out_l_max, in1_features, in2_features, symmetric_product,
                        shared_weights, reduce_paths, _alpha_div(alpha_div))
    out = in1.new_empty(in1.shape[0], _tp_out_dim(in1_l_max, in2_l_max, out_l_max, in1_features, in2_features,
                                                  symmetric_product, reduce_paths))
    csr, keep = (None, None)
    if conv:
        csr, keep = _tp_csr(in1, idx_i, idx_j, rowptr, sender_perm, sender_ptr, need_senders=False,
                            pair_slot=pair_slot)
    _lib_call("fc_tp_fwd", desc, csr, in1.shape[0], in1.data_ptr(), in2.data_ptr(), w.data_ptr(), float(alpha),
              out.data_ptr(), _lib.stream_of(in1))
    return out


@tp_fwd.register_fake
def _(in1, in2, weights, idx_i, idx_j, in1_l_max, in2_l_max, out_l_max, in1_features, in2_features,
      symmetric_product, shared_weights, in1_offs, in2_offs, out_sizes, n_paths_per_l, n_total_paths,
      reduce_paths=False, rowptr=None, sender_perm=None, sender_ptr=None, alpha=1.0, pair_slot=None,
      alpha_div=None):
    return in1.new_empty(in1.shape[0], _tp_out_dim(in1_l_max, in2_l_max, out_l_max, in1_features, in2_features,
                                                   symmetric_product, reduce_paths))


@torch.library.custom_op("flashcart::tp_bwd", mutates_args=())
def tp_bwd(grad_out: Tensor, in1: Tensor, in2: Tensor, weights: Tensor, idx_i: Optional[Tensor],
           idx_j: Optional[Tensor], in1_l_max: int, in2_l_max: int, out_l_max: int, in1_features: int,
           in2_features: int, symmetric_product: bool, shared_weights: bool, in1_offs: List[int],
           in2_offs: List[int], out_sizes: List[int], n_paths_per_l: List[int], n_total_paths: int,
           reduce_paths: bool, need_grad_in1: bool, need_grad_in2: bool, need_grad_weights: bool,
           rowptr: Optional[Tensor] = None, sender_perm: Optional[Tensor] = None,
           sender_ptr: Optional[Tensor] = None, alpha: float = 1.0,
           pair_slot: Optional[Tensor] = None, alpha_div: Optional[Tensor] = None) -> Tuple[Tensor, Tensor, Tensor]:
    """Gradients wrt (in1, in2, weights); unrequested ones are returned as empty (0,) tensors.

    Reference schema (src/flashcart/o3/_tensor_product.py:588-611) plus the optional
    CSR arrays, ``alpha``, ``pair_slot`` and ``alpha_div`` of ``tp_fwd``. With ``pair_slot`` the weight
    gradient has one row per edge (edge order); the sum of a pair's two rows is the gradient
    of the pair's weight row."""
    _check_tp_meta((in1_l_max, in2_l_max, out_l_max, in1_features, in2_features, symmetric_product, reduce_paths),
                   in1_offs, in2_offs, out_sizes, n_paths_per_l, n_total_paths)
    conv = idx_i is not None and idx_j is not None
    go = _lib.contig("grad_out", grad_out)
    in1 = _lib.contig("in1", in1)
    in2 = _lib.contig("in2", in2)
    w = _lib.contig("weights", weights)
    desc = _lib.tp_desc(in1_l_max, in2_l_max, out_l_max, in1_features, in2_features, symmetric_product,
                        shared_weights, reduce_paths, _alpha_div(alpha_div))
    csr, keep = (None, None)
    if conv:
        sender_order = (need_grad_in1 and need_grad_in2 and need_grad_weights and not shared_weights
                        and in2_features == 1 and in1_features == 64)
        csr, keep = _tp_csr(in1, idx_i, idx_j, rowptr, sender_perm, sender_ptr, need_senders=need_grad_in1,
                            pair_slot=pair_slot, receivers=sender_order)
    elif pair_slot is not None:
        raise ValueError("pair_slot needs a convolution (idx_i, idx_j).")
    g1 = _lib.rows_empty(in1, *in1.shape) if need_grad_in1 else in1.new_empty(0)
    g2 = _lib.rows_empty(in2, *in2.shape) if need_grad_in2 else in2.new_empty(0)
    gw_rows = 2 * w.shape[0] if pair_slot is not None else w.shape[0]  # per edge either way
    gw = _lib.rows_empty(w, gw_rows, *w.shape[1:]) if need_grad_weights else w.new_empty(0)
    lib = _lib.load()
    n_ws = lib.fc_tp_bwd_workspace(desc, csr, in1.shape[0], int(need_grad_in1), int(need_grad_weights))
    if n_ws < 0:
        _lib.check(-n_ws, "fc_tp_bwd_workspace")
    ws = _lib.rows_empty(in1, max(int(n_ws), 1))
    _lib_call("fc_tp_bwd", desc, csr, in1.shape[0], go.data_ptr(), in1.data_ptr(), in2.data_ptr(), w.data_ptr(),
              float(alpha), g1.data_ptr() if need_grad_in1 else None, g2.data_ptr() if need_grad_in2 else None,
              gw.data_ptr() if need_grad_weights else None, ws.data_ptr(), int(n_ws), _lib.stream_of(in1))
    return g1, g2, gw


@tp_bwd.register_fake
def _(grad_out, in1, in2, weights, idx_i, idx_j, in1_l_max, in2_l_max, out_l_max, in1_features, in2_features,
      symmetric_product, shared_weights, in1_offs, in2_offs, out_sizes, n_paths_per_l, n_total_paths,
      reduce_paths, need_grad_in1, need_grad_in2, need_grad_weights, rowptr=None, sender_perm=None,
      sender_ptr=None, alpha=1.0, pair_slot=None, alpha_div=None):
    gw_rows = 2 * weights.shape[0] if pair_slot is not None else weights.shape[0]
    return (torch.empty_like(in1) if need_grad_in1 else in1.new_empty(0),
            torch.empty_like(in2) if need_grad_in2 else in2.new_empty(0),
            weights.new_empty(gw_rows, *weights.shape[1:]) if need_grad_weights else weights.new_empty(0))


def _tp_setup(ctx, inputs, output):
    (in1, in2, weights, idx_i, idx_j, l1, l2, lo, f1, f2, sym, shared, o1, o2, osz, npl, ntot, red,
     rowptr, sperm, sptr, alpha, pair_slot, alpha_div) = inputs
    ctx.save_for_backward(in1, in2, weights, idx_i, idx_j, rowptr, sperm, sptr, pair_slot, alpha_div)
    ctx.cfg = (int(l1), int(l2), int(lo), int(f1), int(f2), bool(sym), bool(shared), list(o1), list(o2),
               list(osz), list(npl), int(ntot), bool(red))
    ctx.alpha = float(alpha)


def _tp_backward(ctx, grad):
    in1, in2, weights, idx_i, idx_j, rowptr, sperm, sptr, pair_slot, alpha_div = ctx.saved_tensors
    n1, n2, nw = ctx.needs_input_grad[0], ctx.needs_input_grad[1], ctx.needs_input_grad[2]
    none_tail = (None,) * 21
    if not (n1 or n2 or nw):
        return (None, None, None) + none_tail
    g1, g2, gw = tp_bwd(grad, in1, in2, weights, idx_i, idx_j, *ctx.cfg, bool(n1), bool(n2), bool(nw),
                        rowptr, sperm, sptr, ctx.alpha, pair_slot, alpha_div)
    if nw and pair_slot is not None:  # both edges of a pair read its weight row (two terms: order-free)
        gw = gw.new_zeros(weights.shape).index_add_(0, (pair_slot // 2).long(), gw)
    return (g1 if n1 else None, g2 if n2 else None, gw if nw else None) + none_tail


_register_autograd(tp_fwd, _tp_backward, _tp_setup)


def tp_bwd_rows_acc(grad_out: Tensor, in1: Tensor, in2: Tensor, weights: Tensor, in1_l_max: int, in2_l_max: int,
                    out_l_max: int, features: int, shared_weights: bool, res1: Optional[Tensor] = None,
                    res2: Optional[Tensor] = None, alpha: float = 1.0, inplace1: bool = False,
                    inplace2: bool = False) -> Tuple[Tensor, Tensor]:
    """(pad(res1) + dL/d in1, pad(res2) + dL/d in2) of a node-wise product with per-path
    outputs and in1_features == in2_features (``fc_tp_bwd_rows_acc``; outside autograd).

    ``res1`` / ``res2`` hold gradients of the leading rank blocks of in1 / in2 from other
    consumers (any whole number of components per row, zero above). With ``inplace1`` /
    ``inplace2``, a residual as wide as its operand is accumulated into and returned."""
    go = _lib.contig("grad_out", grad_out)
    in1 = _lib.contig("in1", in1)
    in2 = _lib.contig("in2", in2)
    w = _lib.contig("weights", weights)
    C = int(features)

    def prep(name, res, like, l_max, inplace):
        full = (l_max + 1) ** 2
        if res is None:
            return None, 0, torch.empty_like(like)
        res = _lib.contig(name, res)
        comps = res.shape[-1] // C
        if res.dim() != 2 or res.shape[0] != like.shape[0] or comps * C != res.shape[-1] or comps > full:
            raise RuntimeError(f"{name} of shape {tuple(res.shape)} does not match an operand of shape "
                               f"{tuple(like.shape)} with {C} channels.")
        return res, comps, (res if inplace and comps == full else torch.empty_like(like))

    r1, c1, g1 = prep("res1", res1, in1, in1_l_max, inplace1)
    r2, c2, g2 = prep("res2", res2, in2, in2_l_max, inplace2)
    desc = _lib.tp_desc(in1_l_max, in2_l_max, out_l_max, C, C, False, shared_weights, False)
    _lib_call("fc_tp_bwd_rows_acc", desc, in1.shape[0], go.data_ptr(), in1.data_ptr(), in2.data_ptr(), w.data_ptr(),
              float(alpha), _lib.ptr(r1), int(c1), _lib.ptr(r2), int(c2), g1.data_ptr(), g2.data_ptr(),
              _lib.stream_of(in1))
    return g1, g2


# ---------------------------------------------------------------------------
# Equivariant linear map
# ---------------------------------------------------------------------------

def _linear_dims(in_l_max, out_l_max, in_features, out_features, in_paths):
    in_dim = sum((2 * l + 1) * in_features * in_paths[l] for l in range(in_l_max + 1))
    out_dim = sum((2 * l + 1) * out_features for l in range(out_l_max + 1))
    return in_dim, out_dim


def _wlist(w0, w1, w2, w3, w4) -> List[Tensor]:
    return [w for w in (w0, w1, w2, w3, w4) if w is not None]


def _lin_dtype(t: Tensor) -> torch.dtype:
    """Arithmetic type of a linear-map call: float64 tensors take the ``fc_linear_*_f64`` entry
    points (float64 accumulation, as the reference's use_fp64), every other dtype must be float32."""
    return torch.float64 if t.dtype == torch.float64 else torch.float32


def _lin_name(name: str, dt: torch.dtype) -> str:
    return name + "_f64" if dt == torch.float64 else name


def _pad_ranks(weights):
    """The weights in the ops' MAX_RANKS slots (ranks 0..4), None past the last rank."""
    ws = list(weights) + [None] * (_lib.MAX_RANKS - len(weights))
    if len(ws) != _lib.MAX_RANKS:
        raise ValueError(f"at most {_lib.MAX_RANKS} rank blocks (l <= {_lib.MAX_RANKS - 1}) are supported.")
    return ws


@torch.library.custom_op("flashcart::equiv_linear_fwd", mutates_args=())
def linear_fwd_op(x: Tensor, w0: Tensor, w1: Optional[Tensor], w2: Optional[Tensor], w3: Optional[Tensor],
                  w4: Optional[Tensor], in_l_max: int, out_l_max: int, in_features: int, out_features: int, in_paths: List[int],
                  scale: List[float], alpha: float = 1.0, residual: Optional[Tensor] = None) -> Tensor:
    """out = linear(x) (+ residual, a tensor of the output's shape added in the GEMM epilogue): the
    build's own layers call this op (the reference-schema ``flashcart::linear_fwd`` is below)."""
    in_dim, out_dim = _linear_dims(in_l_max, out_l_max, in_features, out_features, in_paths)
    if x.shape[-1] != in_dim:
        raise RuntimeError(f"Incorrect last dimension for x. Expected {in_dim}, got {x.shape[-1]}.")
    dt = _lin_dtype(x)
    x = _lib.contig("x", x, dt)
    ws = [_lib.contig(f"weight[{l}]", w, dt) for l, w in enumerate(_wlist(w0, w1, w2, w3, w4))]
    out = x.new_empty(x.shape[0], out_dim)
    r = _check_residual(residual, out)
    desc = _lib.linear_desc(in_l_max, out_l_max, in_features, out_features, in_paths, ws, scale)
    _lib_call(_lin_name("fc_linear_fwd", dt), desc, x.shape[0], x.data_ptr(), float(alpha), _lib.ptr(r), out.data_ptr(),
              _lib.stream_of(x))
    return out


@linear_fwd_op.register_fake
def _(x, w0, w1, w2, w3, w4, in_l_max, out_l_max, in_features, out_features, in_paths, scale, alpha=1.0,
      residual=None):
    _, out_dim = _linear_dims(in_l_max, out_l_max, in_features, out_features, in_paths)
    return x.new_empty(x.shape[0], out_dim)


@torch.library.custom_op("flashcart::equiv_linear_dgrad", mutates_args=())
def linear_bwd_op(grad_out: Tensor, w0: Tensor, w1: Optional[Tensor], w2: Optional[Tensor], w3: Optional[Tensor],
                  w4: Optional[Tensor], in_l_max: int, out_l_max: int, in_features: int, out_features: int, in_paths: List[int],
                  scale: List[float], alpha: float = 1.0, residual: Optional[Tensor] = None) -> Tensor:
    """Input gradient of linear_fwd (the MFMA dgrad), plus ``residual`` when given."""
    in_dim, _ = _linear_dims(in_l_max, out_l_max, in_features, out_features, in_paths)
    dt = _lin_dtype(grad_out)
    go = _lib.contig("grad_out", grad_out, dt)
    ws = [_lib.contig(f"weight[{l}]", w, dt) for l, w in enumerate(_wlist(w0, w1, w2, w3, w4))]
    gx = go.new_empty(go.shape[0], in_dim)
    r = _check_residual(residual, gx)
    desc = _lib.linear_desc(in_l_max, out_l_max, in_features, out_features, in_paths, ws, scale)
    _lib_call(_lin_name("fc_linear_dgrad", dt), desc, go.shape[0], go.data_ptr(), float(alpha), _lib.ptr(r), gx.data_ptr(),
              _lib.stream_of(go))
    return gx


@linear_bwd_op.register_fake
def _(grad_out, w0, w1, w2, w3, w4, in_l_max, out_l_max, in_features, out_features, in_paths, scale, alpha=1.0,
      residual=None):
    in_dim, _ = _linear_dims(in_l_max, out_l_max, in_features, out_features, in_paths)
    return grad_out.new_empty(grad_out.shape[0], in_dim)


def linear_fwd(x: Tensor, weights: List[Tensor], in_l_max: int, out_l_max: int, in_features: int,
               out_features: int, in_paths: List[int], scale: List[float], alpha: float = 1.0,
               residual: Optional[Tensor] = None) -> Tensor:
    """out_l = alpha * scale_l * x_l @ W_l^T for every shared rank (torch.ops.flashcart.equiv_linear_fwd),
    plus ``residual`` (same shape as the output) when given."""
    return linear_fwd_op(x, *_pad_ranks(weights), in_l_max, out_l_max, in_features, out_features, list(in_paths),
                         [float(s) for s in scale], float(alpha), residual)


def linear_bwd(grad_out: Tensor, weights: List[Tensor], in_l_max: int, out_l_max: int, in_features: int,
               out_features: int, in_paths: List[int], scale: List[float], alpha: float = 1.0,
               residual: Optional[Tensor] = None) -> Tensor:
    return linear_bwd_op(grad_out, *_pad_ranks(weights), in_l_max, out_l_max, in_features, out_features,
                         list(in_paths), [float(s) for s in scale], float(alpha), residual)


def _check_residual(residual: Optional[Tensor], out: Tensor) -> Optional[Tensor]:
    if residual is None:
        return None
    if residual.shape != out.shape:
        raise RuntimeError(f"residual shape {tuple(residual.shape)} != output shape {tuple(out.shape)}.")
    return _lib.contig("residual", residual, out.dtype)


def _linear_setup(ctx, inputs, output):
    x, w0, w1, w2, w3, w4, in_l_max, out_l_max, in_features, out_features, in_paths, scale, alpha, residual = inputs
    ws = _wlist(w0, w1, w2, w3, w4)
    ctx.save_for_backward(x, *ws)
    ctx.cfg = (int(in_l_max), int(out_l_max), int(in_features), int(out_features), list(in_paths), list(scale))
    ctx.alpha = float(alpha)


def _linear_backward(ctx, grad):
    x, *weights = ctx.saved_tensors
    in_l_max, out_l_max, fin, fout, in_paths, scale = ctx.cfg
    need = ctx.needs_input_grad
    gx = None
    if need[0]:
        gx = linear_bwd(grad, weights, in_l_max, out_l_max, fin, fout, in_paths, scale, ctx.alpha)
    gws = [None] * _lib.MAX_RANKS
    if any(need[1:1 + _lib.MAX_RANKS]):  # parameter gradients (training)
        gws = linear_wgrad(grad, x, weights, in_l_max, out_l_max, fin, fout, in_paths, scale, ctx.alpha,
                           [bool(need[1 + l]) for l in range(len(weights))])
        gws = gws + [None] * (_lib.MAX_RANKS - len(gws))
    # trailing arguments left at their defaults are not part of needs_input_grad
    i_res = 8 + _lib.MAX_RANKS  # x, the weight slots, 7 configuration arguments, residual
    g_res = grad if len(need) > i_res and need[i_res] else None
    return (gx, *gws) + (None,) * 7 + (g_res,)


_register_autograd(linear_fwd_op, _linear_backward, _linear_setup)


def linear_wgrad(grad_out: Tensor, x: Tensor, weights: List[Tensor], in_l_max: int, out_l_max: int,
                 in_features: int, out_features: int, in_paths: List[int], scale: List[float], alpha: float,
                 need: List[bool]) -> List[Optional[Tensor]]:
    """dW_l = alpha * scale_l * sum over (node, component) rows of grad_out_l^T x_l for every rank
    with ``need[l]`` (``fc_linear_wgrad``: split-K MFMA over the rows read in place).

    Under grad mode (a backward with create_graph) the same sums are formed with torch
    matmuls instead, so that they stay differentiable."""
    common = min(in_l_max, out_l_max)
    if torch.is_grad_enabled():
        n = x.shape[0]
        outs: List[Optional[Tensor]] = []
        in_off = out_off = 0
        for l in range(common + 1):
            k = in_features * in_paths[l]
            m = 2 * l + 1
            if need[l]:
                xl = x[:, in_off:in_off + m * k].reshape(n * m, k)
                gl = grad_out[:, out_off:out_off + m * out_features].reshape(n * m, out_features)
                outs.append((gl.t() @ xl) * (scale[l] * alpha))
            else:
                outs.append(None)
            in_off += m * k
            out_off += m * out_features
        return outs
    dt = _lin_dtype(grad_out)
    go = _lib.contig("grad_out", grad_out, dt)
    xx = _lib.contig("x", x, dt)
    ws = [_lib.contig(f"weight[{l}]", w, dt) for l, w in enumerate(weights)]
    outs = [torch.empty_like(ws[l]) if (l <= common and need[l]) else None for l in range(len(ws))]
    desc = _lib.linear_desc(in_l_max, out_l_max, in_features, out_features, in_paths, ws, scale)
    lib = _lib.load()
    n = go.shape[0]
    ptrs = (_lib.c_vp * _lib.MAX_RANKS)(*([o.data_ptr() if o is not None else None for o in outs] +
                                          [None] * (_lib.MAX_RANKS - len(outs))))
    ws_name = "fc_linear_wgrad_f64_workspace" if dt == torch.float64 else "fc_linear_wgrad_workspace"
    n_ws = getattr(lib, ws_name)(desc, n, ptrs)
    if n_ws < 0:
        _lib.check(-n_ws, ws_name)
    buf = go.new_empty(max(int(n_ws), 1))
    _lib_call(_lin_name("fc_linear_wgrad", dt), desc, n, go.data_ptr(), xx.data_ptr(), float(alpha), ptrs, buf.data_ptr(),
              int(n_ws), _lib.stream_of(go))
    return outs



# ---------------------------------------------------------------------------
# The reference's linear ops, same names and schemas (src/flashcart/o3/_linear.py:328-385,
# :457-538, :571-699, autograd chain :777-778), on the same MFMA kernels
# ---------------------------------------------------------------------------

_PRECISIONS = ("ieee", "tf32", "tf32x3")
def _scale_values(scale: Tensor, n: int) -> List[float]:
    """Host copy of the per-rank scale tensor (one small device-to-host copy per call of the
    reference-schema ops; the build's own layers keep their scales on the host)."""
    if scale.numel() < n:
        raise RuntimeError(f"Expected {n} scales, got {scale.numel()}.")
    return [float(v) for v in scale.detach().reshape(-1)[:n].cpu()]


def _ref_linear_layout(x: Tensor, weights: List[Tensor], use_fp64: bool, dot_input_precision: str,
                       in_offsets, out_offsets, weight_offsets, m_values, f_in_values, f_out_values, out_size=None):
    """The descriptor of the reference's metadata lists (make_linear_metadata, _linear.py:113-166):
    rank l of n active ranks has 2l+1 components, f_in_values[l] input columns (channels x paths)
    and f_out_values[l] = out_features outputs; returns (n, in_active_end, out_l_max, desc args)."""
    if dot_input_precision not in _PRECISIONS:
        raise ValueError(f"dot_input_precision must be one of {_PRECISIONS}. Provided: {dot_input_precision!r}.")
    n = len(in_offsets)
    lists = (out_offsets, weight_offsets, m_values, f_in_values, f_out_values)
    if any(len(v) != n for v in lists) or n > _lib.MAX_RANKS:
        raise RuntimeError(f"linear metadata lists must have one entry per active rank (at most {_lib.MAX_RANKS}).")
    if len(weights) < n:
        raise RuntimeError(f"Expected at least {n} weight tensors, got {len(weights)}.")
    fout = int(f_out_values[0]) if n else 1
    i_off = o_off = w_off = 0
    for l in range(n):
        if (int(m_values[l]) != 2 * l + 1 or int(in_offsets[l]) != i_off or int(out_offsets[l]) != o_off
                or int(weight_offsets[l]) != w_off or int(f_out_values[l]) != fout):
            raise ValueError("linear metadata does not describe the standard layout (make_linear_metadata).")
        if tuple(weights[l].shape) != (fout, int(f_in_values[l])):
            raise RuntimeError(f"Weight[{l}] shape mismatch: expected ({fout}, {int(f_in_values[l])}), "
                               f"got {tuple(weights[l].shape)}.")
        i_off += (2 * l + 1) * int(f_in_values[l])
        o_off += (2 * l + 1) * fout
        w_off += fout * int(f_in_values[l])
    if x.shape[-1] < i_off:
        raise RuntimeError(f"Incorrect last dimension for x. Expected at least {i_off}, got {x.shape[-1]}.")
    out_l_max = n - 1
    if out_size is not None:
        r = int(round((int(out_size) / max(fout, 1)) ** 0.5)) - 1
        if r < n - 1 or (r + 1) ** 2 * fout != int(out_size):
            raise ValueError(f"out_size={out_size} is not (out_l_max+1)^2 * {fout} for out_l_max >= {n - 1}.")
        out_l_max = r
    return n, i_off, out_l_max, fout


def _widen(use_fp64: bool, *tensors):
    """use_fp64 with float32 tensors (float64 accumulation, the reference's USE_FP64 kernels):
    the tensors (lists of tensors too) as float64 copies, the map runs in float64 and its results
    are rounded back to the inputs' dtype; otherwise the tensors unchanged."""
    if not use_fp64:
        return tensors
    return tuple([t.double() for t in v] if isinstance(v, (list, tuple)) else
                 (v.double() if v.dtype == torch.float32 else v) for v in tensors)


def _narrow(t, dtype):
    if isinstance(t, (list, tuple)):
        return [v.to(dtype) for v in t]
    return t.to(dtype)


def _ref_desc(n, out_l_max, fout, f_in_values, weights, scale):
    return _lib.linear_desc(n - 1, out_l_max, 1, fout, [int(v) for v in f_in_values[:n]], weights[:n],
                            _scale_values(scale, n))


@torch.library.custom_op("flashcart::linear_fwd", mutates_args=())
def linear_fwd_ref(x: Tensor, weights: List[Tensor], meta: Tensor, out_size: int, use_fp64: bool,
                   dot_input_precision: str, in_offsets: List[int], out_offsets: List[int],
                   weight_offsets: List[int], m_values: List[int], f_in_values: List[int],
                   f_out_values: List[int], scale: Tensor) -> Tensor:
    """out_l = scale_l * x_l @ W_l^T for the active ranks, zeros above (the reference's op;
    ``meta`` holds the same columns as the lists and is not read)."""
    dt0 = x.dtype
    x, weights = _widen(use_fp64, x, weights)
    n, in_end, out_l_max, fout = _ref_linear_layout(x, weights, use_fp64, dot_input_precision, in_offsets,
                                                    out_offsets, weight_offsets, m_values, f_in_values,
                                                    f_out_values, out_size)
    dt = _lin_dtype(x)
    x = _lib.contig("x", x, dt)
    if n == 0:
        return x.new_zeros(x.shape[0], int(out_size), dtype=dt0)
    if x.shape[1] != in_end:  # input ranks above the output's: not read
        x = x[:, :in_end].contiguous()
    ws = [_lib.contig(f"weight[{l}]", w, dt) for l, w in enumerate(weights[:n])]
    out = x.new_empty(x.shape[0], int(out_size))
    _lib_call(_lin_name("fc_linear_fwd", dt), _ref_desc(n, out_l_max, fout, f_in_values, ws, scale), x.shape[0],
              x.data_ptr(), 1.0, None, out.data_ptr(), _lib.stream_of(x))
    return _narrow(out, dt0)


@linear_fwd_ref.register_fake
def _(x, weights, meta, out_size, use_fp64, dot_input_precision, in_offsets, out_offsets, weight_offsets, m_values,
      f_in_values, f_out_values, scale):
    return x.new_empty(x.shape[0], int(out_size))


def _ref_grad_x(grad_out, x, ws, n, in_end, fout, f_in_values, scale):
    """scale_l * go_l @ W_l into the active input columns, zeros beyond."""
    dt = _lin_dtype(grad_out)
    go = _lib.contig("grad_out", grad_out, dt)
    out_l_max = int(round((go.shape[1] / fout) ** 0.5)) - 1
    gx = go.new_empty(go.shape[0], in_end)
    _lib_call(_lin_name("fc_linear_dgrad", dt), _ref_desc(n, out_l_max, fout, f_in_values, ws, scale), go.shape[0],
              go.data_ptr(), 1.0, None, gx.data_ptr(), _lib.stream_of(go))
    if x.shape[1] != in_end:
        gx = torch.cat([gx, gx.new_zeros(gx.shape[0], x.shape[1] - in_end)], dim=1)
    return gx


def _ref_grad_w(grad_out, b, ws, n, in_end, fout, f_in_values, scale):
    """scale_l * sum over rows of go_l^T b_l for every active rank (split-K MFMA)."""
    b = _lib.contig("x", b, _lin_dtype(b))
    if b.shape[1] != in_end:
        b = b[:, :in_end].contiguous()
    out_l_max = int(round((grad_out.shape[1] / fout) ** 0.5)) - 1
    with torch.no_grad():
        return linear_wgrad(grad_out, b, ws, n - 1, out_l_max, 1, fout, [int(v) for v in f_in_values[:n]],
                            _scale_values(scale, n), 1.0, [True] * n)


@torch.library.custom_op("flashcart::linear_bwd", mutates_args=())
def linear_bwd_ref(grad_out: Tensor, x: Tensor, weights: List[Tensor], need_x: bool, need_weight: bool,
                   use_fp64: bool, dot_input_precision: str, in_offsets: List[int], out_offsets: List[int],
                   weight_offsets: List[int], m_values: List[int], f_in_values: List[int],
                   f_out_values: List[int], scale: Tensor) -> Tuple[Tensor, List[Tensor]]:
    """(grad_x, grad_weights) of linear_fwd, empty (0,) tensors for the unrequested ones."""
    if use_fp64 and x.dtype != torch.float64:
        gx, gws = linear_bwd_ref_impl(*_widen(True, grad_out, x, weights), need_x, need_weight, True,
                                      dot_input_precision, in_offsets, out_offsets, weight_offsets, m_values,
                                      f_in_values, f_out_values, scale)
        return _narrow(gx, x.dtype), [g.to(w.dtype) for g, w in zip(gws, weights)]
    return linear_bwd_ref_impl(grad_out, x, weights, need_x, need_weight, use_fp64, dot_input_precision, in_offsets,
                               out_offsets, weight_offsets, m_values, f_in_values, f_out_values, scale)


def linear_bwd_ref_impl(grad_out, x, weights, need_x, need_weight, use_fp64, dot_input_precision, in_offsets,
                        out_offsets, weight_offsets, m_values, f_in_values, f_out_values, scale):
    n, in_end, _, fout = _ref_linear_layout(x, weights, use_fp64, dot_input_precision, in_offsets, out_offsets,
                                            weight_offsets, m_values, f_in_values, f_out_values)
    if n == 0 or not (need_x or need_weight):
        gx = torch.zeros_like(x) if need_x else x.new_empty((0,))
        gws = [torch.zeros_like(w) for w in weights] if need_weight else [w.new_empty(0) for w in weights]
        return gx, gws
    ws = [_lib.contig(f"weight[{l}]", w, _lin_dtype(x)) for l, w in enumerate(weights[:n])]
    gx = _ref_grad_x(grad_out, x, ws, n, in_end, fout, f_in_values, scale) if need_x else x.new_empty((0,))
    if need_weight:
        gws = _ref_grad_w(grad_out, x, ws, n, in_end, fout, f_in_values, scale)
        gws = gws + [torch.zeros_like(w) for w in weights[n:]]
    else:
        gws = [w.new_empty(0) for w in weights]
    return gx, gws


@linear_bwd_ref.register_fake
def _(grad_out, x, weights, need_x, need_weight, use_fp64, dot_input_precision, in_offsets, out_offsets,
      weight_offsets, m_values, f_in_values, f_out_values, scale):
    gx = torch.empty_like(x) if need_x else x.new_empty((0,))
    return gx, [torch.empty_like(w) if need_weight else w.new_empty(0) for w in weights]


@torch.library.custom_op("flashcart::linear_dbwd", mutates_args=())
def linear_dbwd_ref(grad_out: Tensor, x: Tensor, weights: List[Tensor], v_grad_x: Tensor,
                    v_grad_weight: List[Tensor], use_fp64: bool, dot_input_precision: str, need_d_grad_out: bool,
                    need_d_x: bool, need_d_weight: bool, has_v_grad_x: bool, has_v_grad_weight: bool,
                    in_offsets: List[int], out_offsets: List[int], weight_offsets: List[int], m_values: List[int],
                    f_in_values: List[int], f_out_values: List[int],
                    scale: Tensor) -> Tuple[Tensor, Tensor, List[Tensor]]:
    """Backward of linear_bwd along cotangents (v_grad_x, v_grad_weight):
    d grad_out_l = s_l (v_gx_l W_l^T + x_l v_gW_l^T), d x_l = s_l go_l v_gW_l, d W_l = s_l go_l^T v_gx_l."""
    args = (need_d_grad_out, need_d_x, need_d_weight, has_v_grad_x, has_v_grad_weight, in_offsets, out_offsets,
            weight_offsets, m_values, f_in_values, f_out_values, scale)
    if use_fp64 and x.dtype != torch.float64:
        go64, x64, w64, vgx64, vgw64 = _widen(True, grad_out, x, weights, v_grad_x, v_grad_weight)
        d_go, d_x, d_ws = linear_dbwd_ref_impl(go64, x64, w64, vgx64, vgw64, True, dot_input_precision, *args)
        return _narrow(d_go, grad_out.dtype), _narrow(d_x, x.dtype), [d.to(w.dtype) for d, w in zip(d_ws, weights)]
    return linear_dbwd_ref_impl(grad_out, x, weights, v_grad_x, v_grad_weight, use_fp64, dot_input_precision, *args)


def linear_dbwd_ref_impl(grad_out, x, weights, v_grad_x, v_grad_weight, use_fp64, dot_input_precision,
                         need_d_grad_out, need_d_x, need_d_weight, has_v_grad_x, has_v_grad_weight, in_offsets,
                         out_offsets, weight_offsets, m_values, f_in_values, f_out_values, scale):
    n, in_end, _, fout = _ref_linear_layout(x, weights, use_fp64, dot_input_precision, in_offsets, out_offsets,
                                            weight_offsets, m_values, f_in_values, f_out_values)
    dt = _lin_dtype(x)
    go = _lib.contig("grad_out", grad_out, dt)
    ws = [_lib.contig(f"weight[{l}]", w, dt) for l, w in enumerate(weights[:n])]
    vws = [_lib.contig(f"v_grad_weight[{l}]", v, dt) for l, v in enumerate(v_grad_weight[:n])] \
        if has_v_grad_weight else []
    out_l_max = int(round((go.shape[1] / max(fout, 1)) ** 0.5)) - 1

    def fwd(inp, mats, residual=None):
        a = _lib.contig("input", inp, dt)
        if a.shape[1] != in_end:
            a = a[:, :in_end].contiguous()
        out = a.new_empty(a.shape[0], go.shape[1])
        _lib_call(_lin_name("fc_linear_fwd", dt), _ref_desc(n, out_l_max, fout, f_in_values, mats, scale),
                  a.shape[0], a.data_ptr(), 1.0, _lib.ptr(residual), out.data_ptr(), _lib.stream_of(a))
        return out

    if not need_d_grad_out:
        d_go = go.new_empty((0,))
    elif n == 0 or not (has_v_grad_x or has_v_grad_weight):
        d_go = torch.zeros_like(go)
    else:
        d_go = fwd(x, vws) if has_v_grad_weight else None
        if has_v_grad_x:
            d_go = fwd(v_grad_x, ws, d_go)
    if not need_d_x:
        d_x = x.new_empty((0,))
    elif n == 0 or not has_v_grad_weight:
        d_x = torch.zeros_like(x)
    else:
        d_x = _ref_grad_x(go, x, vws, n, in_end, fout, f_in_values, scale)
    if not need_d_weight:
        d_ws = [w.new_empty(0) for w in weights]
    elif n == 0 or not has_v_grad_x:
        d_ws = [torch.zeros_like(w) for w in weights]
    else:
        d_ws = _ref_grad_w(go, v_grad_x, ws, n, in_end, fout, f_in_values, scale) + \
            [torch.zeros_like(w) for w in weights[n:]]
    return d_go, d_x, d_ws


@linear_dbwd_ref.register_fake
def _(grad_out, x, weights, v_grad_x, v_grad_weight, use_fp64, dot_input_precision, need_d_grad_out, need_d_x,
      need_d_weight, has_v_grad_x, has_v_grad_weight, in_offsets, out_offsets, weight_offsets, m_values,
      f_in_values, f_out_values, scale):
    return (torch.empty_like(grad_out) if need_d_grad_out else grad_out.new_empty((0,)),
            torch.empty_like(x) if need_d_x else x.new_empty((0,)),
            [torch.empty_like(w) if need_d_weight else w.new_empty(0) for w in weights])


_REF_LIN_META = ("in_offsets", "out_offsets", "weight_offsets", "m_values", "f_in_values", "f_out_values")


def _linear_ref_setup(ctx, inputs, output):
    (x, weights, meta, out_size, use_fp64, prec, *lists, scale) = inputs
    ctx.save_for_backward(x, *weights, scale)
    ctx.opts = (bool(use_fp64), prec)
    ctx.lists = [list(v) for v in lists]


def _linear_ref_backward(ctx, grad_out):
    """The reference's linear_bwd (o3/_linear.py:409-455): one linear_bwd op call for the
    gradients that are needed."""
    x, *weights, scale = ctx.saved_tensors
    need_x, need_w = bool(ctx.needs_input_grad[0]), bool(ctx.needs_input_grad[1])
    if not (need_x or need_w):
        return (None,) * 13
    gx, gws = torch.ops.flashcart.linear_bwd(grad_out, x, weights, need_x, need_w, *ctx.opts, *ctx.lists, scale)
    return (gx if need_x else None, gws if need_w else None) + (None,) * 11


def _linear_bwd_ref_setup(ctx, inputs, output):
    (go, x, weights, need_x, need_w, use_fp64, prec, *lists, scale) = inputs
    ctx.set_materialize_grads(False)
    ctx.save_for_backward(go, x, *weights, scale)
    ctx.need_out = (bool(need_x), bool(need_w))
    ctx.opts = (bool(use_fp64), prec)
    ctx.lists = [list(v) for v in lists]


def _linear_bwd_ref_backward(ctx, v_gx, v_gws):
    """The reference's linear_dbwd autograd (o3/_linear.py:700-760)."""
    go, x, *weights, scale = ctx.saved_tensors
    need = ctx.needs_input_grad
    nd_go, nd_x, nd_w = bool(need[0]), bool(need[1]), bool(need[2])
    if not (nd_go or nd_x or nd_w):
        return (None,) * 14
    has_gx = v_gx is not None and v_gx.numel() != 0 and ctx.need_out[0]
    has_gw = v_gws is not None and any(v is not None and v.numel() != 0 for v in v_gws) and ctx.need_out[1]
    vgx = v_gx if has_gx else x.new_empty((0,))
    vgw = [(v if v is not None and v.numel() != 0 else torch.zeros_like(w)) for v, w in zip(v_gws, weights)] \
        if has_gw else [w.new_empty(0) for w in weights]
    d_go, d_x, d_ws = torch.ops.flashcart.linear_dbwd(go, x, weights, vgx, vgw, *ctx.opts, nd_go, nd_x, nd_w,
                                                        has_gx, has_gw, *ctx.lists, scale)
    return (d_go if nd_go else None, d_x if nd_x else None, d_ws if nd_w else None) + (None,) * 11


linear_fwd_ref.register_autograd(_linear_ref_backward, setup_context=_linear_ref_setup)
linear_bwd_ref.register_autograd(_linear_bwd_ref_backward, setup_context=_linear_bwd_ref_setup)


# ---------------------------------------------------------------------------
# Dense layer with optional rescaled-SiLU epilogue (radial / readout MLPs)
# ---------------------------------------------------------------------------

@torch.library.custom_op("flashcart::dense_fwd", mutates_args=())
def dense_fwd(x: Tensor, weight: Tensor, bias: Optional[Tensor], scale: float, act: int) -> Tuple[Tensor, Tensor]:
    """(activated output, pre-activation (empty when act == 0))."""
    x = _lib.contig("x", x)
    w = _lib.contig("weight", weight)
    b = _lib.contig("bias", bias) if bias is not None else None
    m, k = w.shape
    if x.shape[-1] != k:
        raise RuntimeError(f"Incorrect last dimension for x. Expected {k}, got {x.shape[-1]}.")
    lead = x.shape[:-1]
    x2 = x.reshape(-1, k)
    out = _lib.rows_empty(x, x2.shape[0], m)
    pre = _lib.rows_empty(x, x2.shape[0], m) if act else x.new_empty(0)
    _lib_call("fc_dense_fwd", x2.shape[0], k, m, x2.data_ptr(), w.data_ptr(), float(scale), _lib.ptr(b), int(act),
              pre.data_ptr() if act else None, out.data_ptr(), _lib.stream_of(x))
    return out.reshape(*lead, m), (pre.reshape(*lead, m) if act else pre)


@dense_fwd.register_fake
def _(x, weight, bias, scale, act):
    m = weight.shape[0]
    return x.new_empty(*x.shape[:-1], m), (x.new_empty(*x.shape[:-1], m) if act else x.new_empty(0))


@torch.library.custom_op("flashcart::dense_bwd", mutates_args=())
def dense_bwd(grad_out: Tensor, pre: Tensor, weight: Tensor, scale: float, act: int) -> Tensor:
    go = _lib.contig("grad_out", grad_out)
    w = _lib.contig("weight", weight)
    m, k = w.shape
    lead = go.shape[:-1]
    go2 = go.reshape(-1, m)
    gx = _lib.rows_empty(go, go2.shape[0], k)
    if act == 0:
        # gx = go @ (W s): the forward kernel with the transposed weight as its (k, m) matrix, whose
        # operands both stage through LDS as 128-bit rows (the radial output layer's input
        # gradient, K = P x C = 2,176 -> 64, runs 6% faster this way than on the k-major path)
        wt = w.t().contiguous()  # (k, m): a few microseconds for the radial output layer's 2,176 x 64
        _lib_call("fc_dense_fwd", go2.shape[0], m, k, go2.data_ptr(), wt.data_ptr(), float(scale), None, 0, None,
                  gx.data_ptr(), _lib.stream_of(go))
        return gx.reshape(*lead, k)
    pr = _lib.contig("pre", pre).reshape(-1, m)
    _lib_call("fc_dense_dgrad", go2.shape[0], k, m, go2.data_ptr(), _lib.ptr(pr), w.data_ptr(), float(scale),
              int(act), gx.data_ptr(), _lib.stream_of(go))
    return gx.reshape(*lead, k)


@dense_bwd.register_fake
def _(grad_out, pre, weight, scale, act):
    return grad_out.new_empty(*grad_out.shape[:-1], weight.shape[1])


def dense_bwd_pairs(grad: Tensor, weight: Tensor, scale: float, rows_lo: Optional[Tensor] = None,
                    rows_hi: Optional[Tensor] = None) -> Tensor:
    """Input gradient of a bias-free linear layer whose output rows are shared by pairs of
    consumers: gx[p] = scale (g_lo[p] + g_hi[p]) W, with g_lo / g_hi rows rows_lo[p] / rows_hi[p]
    of ``grad`` (an edge-order gradient and the pairs' edges), or rows 2p / 2p + 1 without them.
    One GEMM that adds the two rows as its operands are read (``fc_dense_fwd_pairsum``): the
    MFMA work of P rows."""
    go = _lib.contig("grad", grad)
    w = _lib.contig("weight", weight)
    m, k = w.shape
    gathered = rows_lo is not None
    if go.dim() != 2 or go.shape[1] != m or (not gathered and go.shape[0] % 2):
        raise RuntimeError(f"grad must be (E, {m}) (pair-major (2P, {m}) without row indices), got {tuple(go.shape)}.")
    lo, hi = (_i32("rows_lo", rows_lo), _i32("rows_hi", rows_hi)) if gathered else (None, None)
    n_pairs = lo.shape[0] if gathered else go.shape[0] // 2
    wt = w.t().contiguous()  # (k, m): the forward kernel's (N, K) weight
    gx = _lib.rows_empty(go, n_pairs, k)
    if m % 32 == 0 and k <= 64 and k % 4 == 0 and go.data_ptr() % 16 == 0:
        _lib_call("fc_dense_fwd_pairsum", n_pairs, m, k, go.data_ptr(), _lib.ptr(lo), _lib.ptr(hi), wt.data_ptr(),
                  float(scale), gx.data_ptr(), _lib.stream_of(go))
        return gx
    # other widths: the pair sum formed first, then the plain GEMM
    s = go[lo.long()] + go[hi.long()] if gathered else go.view(n_pairs, 2, m).sum(1)
    _lib_call("fc_dense_fwd", n_pairs, m, k, s.data_ptr(), wt.data_ptr(), float(scale), None, 0, None, gx.data_ptr(),
              _lib.stream_of(go))
    return gx


class _PairInputs(torch.autograd.Function):
    """x[p] = feats[pair_edge[p]] * env[pair_edge[p]]: the radial-MLP input of each edge pair
    (``fc_pair_inputs_fwd``); backward per edge, the lower edge of each pair taking the pair's
    gradient (``fc_pair_inputs_bwd``). First-order only."""

    @staticmethod
    def forward(ctx, feats: Tensor, env: Tensor, pair_edge: Tensor, pair_slot: Tensor) -> Tensor:
        f = _lib.contig("feats", feats)
        en = _lib.contig("env", env)
        pe = _i32("pair_edge", pair_edge)
        width = f.shape[-1]
        x = _lib.rows_empty(f, pe.shape[0], width)
        _lib_call("fc_pair_inputs_fwd", pe.shape[0], width, pe.data_ptr(), f.data_ptr(), en.data_ptr(), x.data_ptr(),
                  _lib.stream_of(f))
        ctx.save_for_backward(f, en, _i32("pair_slot", pair_slot))
        return x

    @staticmethod
    @torch.autograd.function.once_differentiable
    def backward(ctx, gx: Tensor):
        f, en, slot = ctx.saved_tensors
        nf, ne = ctx.needs_input_grad[0], ctx.needs_input_grad[1]
        if not (nf or ne):
            return None, None, None, None
        gxc = _lib.contig("grad", gx)
        g_f = _lib.rows_empty(f, *f.shape) if nf else None
        g_e = _lib.rows_empty(en, *en.shape) if ne else None
        _lib_call("fc_pair_inputs_bwd", f.shape[0], f.shape[-1], slot.data_ptr(), f.data_ptr(), en.data_ptr(),
                  gxc.data_ptr(), _lib.ptr(g_f), _lib.ptr(g_e), _lib.stream_of(f))
        return g_f, g_e, None, None


def pair_inputs(feats: Tensor, env: Tensor, pair_edge: Tensor, pair_slot: Tensor) -> Tensor:
    """Radial-MLP inputs feats * env of the lower edge of each pair (``o3._graph.EdgePairs``)."""
    return _PairInputs.apply(feats, env, pair_edge, pair_slot)


def _dense_setup(ctx, inputs, output):
    x, weight, bias, scale, act = inputs
    ctx.save_for_backward(x, weight, output[1])
    ctx.scale = float(scale)
    ctx.act = int(act)
    ctx.has_bias = bias is not None
    # an unused output's gradient arrives as None rather than a zero tensor
    ctx.set_materialize_grads(False)


def _dense_backward(ctx, grad, grad_pre):
    """Gradients from the activated output and, when a second derivative has been taken
    through a ``dense_bwd`` that read it, from the pre-activation output."""
    x, weight, pre = ctx.saved_tensors
    if not ctx.act or (grad_pre is not None and grad_pre.numel() == 0):
        grad_pre = None
    if grad is None and grad_pre is None:
        return None, None, None, None, None
    m = weight.shape[0]
    gx = gw = gb = None
    if ctx.needs_input_grad[0]:
        if grad is not None:
            gx = dense_bwd(grad, pre, weight, ctx.scale, ctx.act)
        if grad_pre is not None:
            gp = dense_bwd(grad_pre, pre, weight, ctx.scale, 0)
            gx = gp if gx is None else gx + gp
    if ctx.needs_input_grad[1] or (ctx.has_bias and ctx.needs_input_grad[2]):  # parameter gradients (training)
        if grad_pre is None:  # act'(pre) is applied inside the weight-gradient kernel
            g, act = grad, ctx.act
        else:
            if grad is None:
                g = grad_pre
            elif torch.is_grad_enabled():
                g = grad * _torch_math.silu_grad(pre) + grad_pre
            else:
                g, _ = silu_grad_mix(grad, pre, add=grad_pre)
            act = 0
        gw, gb = dense_wgrad(g, pre, act, x, ctx.scale, bool(ctx.needs_input_grad[1]),
                             bool(ctx.has_bias and ctx.needs_input_grad[2]))
    return gx, gw, gb, None, None


_register_autograd(dense_fwd, _dense_backward, _dense_setup)


def _radial_mlp_check(x: Tensor, w0: Tensor, w1: Tensor) -> int:
    n_in = w0.shape[1]
    if w0.dim() != 2 or w0.shape[0] != 64 or not 1 <= n_in <= 64 or tuple(w1.shape) != (64, 64):
        raise RuntimeError(f"radial MLP needs hidden widths 64, 64 and at most 64 inputs; got W0 {tuple(w0.shape)}, "
                           f"W1 {tuple(w1.shape)}.")
    if x.shape[-1] != n_in:
        raise RuntimeError(f"Incorrect last dimension for x. Expected {n_in}, got {x.shape[-1]}.")
    return n_in


@torch.library.custom_op("flashcart::radial_mlp_fwd", mutates_args=())
def radial_mlp_fwd(x: Tensor, w0: Tensor, s0: float, w1: Tensor, s1: float, w2: Tensor, s2: float) -> Tensor:
    """s2 silu(s1 silu(s0 x W0^T) W1^T) W2^T in one pass (``fc_radial_mlp_fwd``); the hidden
    activations are not returned (the backward recomputes them)."""
    x = _lib.contig("x", x)
    w0, w1, w2 = _lib.contig("w0", w0), _lib.contig("w1", w1), _lib.contig("w2", w2)
    n_in = _radial_mlp_check(x, w0, w1)
    if w2.dim() != 2 or w2.shape[1] != 64:
        raise RuntimeError(f"W2 must be (m, 64), got {tuple(w2.shape)}.")
    m = w2.shape[0]
    x2 = x.reshape(-1, n_in)
    out = _lib.rows_empty(x, x2.shape[0], m)
    _lib_call("fc_radial_mlp_fwd", x2.shape[0], n_in, x2.data_ptr(), w0.data_ptr(), float(s0), w1.data_ptr(),
              float(s1), m, w2.data_ptr(), float(s2), out.data_ptr(), _lib.stream_of(x))
    return out.reshape(*x.shape[:-1], m)


@radial_mlp_fwd.register_fake
def _(x, w0, s0, w1, s1, w2, s2):
    return x.new_empty(*x.shape[:-1], w2.shape[0])


def radial_mlp_bwd_pairsum(grad_h2: Tensor, x: Tensor, w0: Tensor, s0: float, w1: Tensor, s1: float) -> Tensor:
    """``radial_mlp_bwd`` with dL/dh2 given as two rows per row of x (2n, 64), summed
    (``fc_radial_mlp_bwd_pairsum``)."""
    x = _lib.contig("x", x)
    w0, w1 = _lib.contig("w0", w0), _lib.contig("w1", w1)
    gh = _lib.contig("grad_h2", grad_h2)
    n_in = _radial_mlp_check(x, w0, w1)
    x2 = x.reshape(-1, n_in)
    if gh.numel() != 2 * x2.shape[0] * 64:
        raise RuntimeError(f"grad_h2 must hold {2 * x2.shape[0]} rows of 64, got {tuple(gh.shape)}.")
    gx = _lib.rows_empty(x2, *x2.shape)
    _lib_call("fc_radial_mlp_bwd_pairsum", x2.shape[0], n_in, x2.data_ptr(), w0.data_ptr(), float(s0), w1.data_ptr(),
              float(s1), gh.data_ptr(), gx.data_ptr(), _lib.stream_of(x))
    return gx.reshape(x.shape)


@torch.library.custom_op("flashcart::radial_mlp_bwd", mutates_args=())
def radial_mlp_bwd(grad_h2: Tensor, x: Tensor, w0: Tensor, s0: float, w1: Tensor, s1: float) -> Tensor:
    """dL/dx of the radial MLP's hidden part from dL/dh2 (``fc_radial_mlp_bwd``)."""
    x = _lib.contig("x", x)
    w0, w1 = _lib.contig("w0", w0), _lib.contig("w1", w1)
    gh = _lib.contig("grad_h2", grad_h2)
    n_in = _radial_mlp_check(x, w0, w1)
    x2 = x.reshape(-1, n_in)
    if gh.numel() != x2.shape[0] * 64:
        raise RuntimeError(f"grad_h2 must hold {x2.shape[0]} rows of 64, got {tuple(gh.shape)}.")
    gx = _lib.rows_empty(x2, *x2.shape)
    _lib_call("fc_radial_mlp_bwd", x2.shape[0], n_in, x2.data_ptr(), w0.data_ptr(), float(s0), w1.data_ptr(),
              float(s1), gh.data_ptr(), gx.data_ptr(), _lib.stream_of(x))
    return gx.reshape(x.shape)


@radial_mlp_bwd.register_fake
def _(grad_h2, x, w0, s0, w1, s1):
    return torch.empty_like(x)


def radial_mlp_hidden_fwd(x: Tensor, w0: Tensor, s0: float, w1: Tensor, s1: float) -> Tensor:
    """h2 = silu(s1 silu(s0 x W0^T) W1^T) (n, 64): the radial MLP without its output layer
    (``fc_radial_mlp_hidden_fwd``)."""
    x = _lib.contig("x", x)
    w0, w1 = _lib.contig("w0", w0), _lib.contig("w1", w1)
    n_in = _radial_mlp_check(x, w0, w1)
    x2 = x.reshape(-1, n_in)
    h = _lib.rows_empty(x2, x2.shape[0], 64)
    _lib_call("fc_radial_mlp_hidden_fwd", x2.shape[0], n_in, x2.data_ptr(), w0.data_ptr(), float(s0), w1.data_ptr(),
              float(s1), h.data_ptr(), _lib.stream_of(x))
    return h


def species_density_fwd(csr, l_max: int, y_l_max: int, n_species: int, edge_species: Tensor, h: Tensor,
                        y: Tensor, n_nodes: int) -> Tensor:
    """dens[i, (l, m), Z, k] = sum over the receiver's edges of species-Z senders of h[pair, k] y[e, (l, m)]
    (``fc_species_density_fwd``; ``csr`` a CSR struct carrying the edge pairing)."""
    zj = _i32("edge_species", edge_species)
    hh, yy = _lib.contig("h", h), _lib.contig("y", y)
    dens = _lib.rows_empty(hh, n_nodes, (l_max + 1) ** 2 * n_species * 64)
    _lib_call("fc_species_density_fwd", csr, int(l_max), int(y_l_max), int(n_species), zj.data_ptr(), hh.data_ptr(),
              yy.data_ptr(), dens.data_ptr(), _lib.stream_of(hh))
    return dens


def species_density_bwd(csr, l_max: int, y_l_max: int, n_species: int, edge_species: Tensor, h: Tensor, y: Tensor,
                        g_dens: Tensor) -> Tuple[Tensor, Tensor]:
    """(dL/dh per edge, pair-major rows; dL/dy) of ``species_density_fwd`` (``fc_species_density_bwd``)."""
    zj = _i32("edge_species", edge_species)
    hh, yy, gd = _lib.contig("h", h), _lib.contig("y", y), _lib.contig("g_dens", g_dens)
    n_edges = yy.shape[0]
    g_h = _lib.rows_empty(hh, n_edges, 64)
    g_y = _lib.rows_empty(yy, n_edges, yy.shape[1])
    _lib_call("fc_species_density_bwd", csr, int(l_max), int(y_l_max), int(n_species), zj.data_ptr(), hh.data_ptr(),
              yy.data_ptr(), gd.data_ptr(), g_h.data_ptr(), g_y.data_ptr(), _lib.stream_of(hh))
    return g_h, g_y


def species_maps(table: Tensor, w_first: Tensor, s_first: float, alpha_div: Tensor, w_second: List[Tensor],
                 w_radial: Tensor) -> List[Tensor]:
    """Per rank l < len(w_second): maps[l][o, Z * nh + k] = sum_c w_second[l][o, c] x[Z, c]
    w_radial[l * c_mid + c, k] with x = s_first * table @ w_first^T / alpha_div (``fc_species_maps``,
    one launch; alpha_div a one-element device tensor)."""
    tb, wf, wr = _lib.contig("table", table), _lib.contig("w_first", w_first), _lib.contig("w_radial", w_radial)
    ws = [_lib.contig(f"w_second[{l}]", w) for l, w in enumerate(w_second)]
    div = _lib.contig("alpha_div", alpha_div.detach().reshape(-1)[:1])
    n_sp, c_in = tb.shape
    c_mid, nh, c_out, n = wf.shape[0], wr.shape[1], ws[0].shape[0], len(ws)
    if wf.shape[1] != c_in or wr.shape[0] < n * c_mid or any(tuple(w.shape) != (c_out, c_mid) for w in ws):
        raise RuntimeError("species_maps: inconsistent shapes.")
    out = tb.new_empty(n, c_out, n_sp * nh)
    mats = [out[l] for l in range(n)]
    wp = (_lib.c_vp * _lib.MAX_RANKS)(*([w.data_ptr() for w in ws] + [None] * (_lib.MAX_RANKS - n)))
    mp = (_lib.c_vp * _lib.MAX_RANKS)(*([m.data_ptr() for m in mats] + [None] * (_lib.MAX_RANKS - n)))
    _lib_call("fc_species_maps", int(n_sp), int(c_in), int(c_mid), int(c_out), int(nh), int(n), tb.data_ptr(),
              wf.data_ptr(), float(s_first), div.data_ptr(), wp, wr.data_ptr(), mp, _lib.stream_of(tb))
    return mats


def silu_grad_mix(a: Tensor, pre: Tensor, add: Optional[Tensor] = None, b: Optional[Tensor] = None,
                  need1: bool = True, need2: bool = False) -> Tuple[Optional[Tensor], Optional[Tensor]]:
    """(a * f'(pre) + add, a * b * f''(pre)) for the rescaled SiLU f, the requested ones, in one
    elementwise pass (``fc_silu_grad_mix``). Not differentiable: callers use it outside grad mode
    (the torch statements in ``_torch_math`` otherwise)."""
    ac = _lib.contig("a", a)
    pc = _lib.contig("pre", pre)
    dc = _lib.contig("add", add) if add is not None else None
    bc = _lib.contig("b", b) if need2 else None
    for name, t in (("pre", pc), ("add", dc), ("b", bc)):
        if t is not None and t.shape != ac.shape:
            raise RuntimeError(f"silu_grad_mix: {name} {tuple(t.shape)} does not match a {tuple(ac.shape)}.")
    o1 = torch.empty_like(ac) if need1 else None
    o2 = torch.empty_like(ac) if need2 else None
    _lib_call("fc_silu_grad_mix", ac.numel(), ac.data_ptr(), _lib.ptr(bc), pc.data_ptr(), _lib.ptr(dc), _lib.ptr(o1),
              _lib.ptr(o2), _lib.stream_of(ac))
    return o1, o2


def dense_wgrad(grad_out: Tensor, pre: Optional[Tensor], act: int, x: Tensor, scale: float, need_weight: bool,
                need_bias: bool) -> Tuple[Optional[Tensor], Optional[Tensor]]:
    """(scale * g^T x, column sums of g) with g = grad_out * act'(pre) (act 1) or grad_out
    (``fc_dense_wgrad``); torch matmuls under grad mode, so that the result stays differentiable."""
    if not (need_weight or need_bias):
        return None, None
    m, k = grad_out.shape[-1], x.shape[-1]
    if torch.is_grad_enabled():
        g2 = (grad_out * _torch_math.silu_grad(pre) if act else grad_out).reshape(-1, m)
        gw = (g2.t() @ x.reshape(-1, k)) * scale if need_weight else None
        return gw, (g2.sum(0) if need_bias else None)
    go = _lib.contig("grad_out", grad_out).reshape(-1, m)
    xx = _lib.contig("x", x).reshape(-1, k)
    pr = _lib.contig("pre", pre).reshape(-1, m) if act else None
    n = go.shape[0]
    gw = go.new_empty(m, k)
    gb = go.new_empty(m) if need_bias else None
    lib = _lib.load()
    n_ws = lib.fc_dense_wgrad_workspace(n, k, m, int(need_bias))
    if n_ws < 0:
        _lib.check(-n_ws, "fc_dense_wgrad_workspace")
    buf = _lib.rows_empty(go, max(int(n_ws), 1))
    _lib_call("fc_dense_wgrad", n, k, m, go.data_ptr(), _lib.ptr(pr), int(act), xx.data_ptr(), float(scale),
              gw.data_ptr(), _lib.ptr(gb), buf.data_ptr(), int(n_ws), _lib.stream_of(go))
    return (gw if need_weight else None), gb


# ---------------------------------------------------------------------------
# Segment sum over contiguous sorted segments (per-graph energies)
# ---------------------------------------------------------------------------

@torch.library.custom_op("flashcart::segment_sum", mutates_args=())
def segment_sum(src: Tensor, ptr: Tensor, index: Tensor) -> Tensor:
    """dst[s] = sum(src[ptr[s]:ptr[s+1]]); ``index`` (row -> segment) is used by the backward."""
    s = _lib.contig("src", src)
    p = _i32("ptr", ptr)
    n_seg = p.shape[0] - 1
    width = 1 if s.dim() == 1 else int(s[0].numel()) if s.shape[0] else int(torch.Size(s.shape[1:]).numel())
    dst = s.new_empty((n_seg,) + tuple(s.shape[1:]))
    _lib_call("fc_segment_sum", n_seg, width, s.data_ptr(), None, p.data_ptr(), dst.data_ptr(), _lib.stream_of(s))
    return dst


@segment_sum.register_fake
def _(src, ptr, index):
    return src.new_empty((ptr.shape[0] - 1,) + tuple(src.shape[1:]))


def _seg_setup(ctx, inputs, output):
    src, ptr, index = inputs
    ctx.save_for_backward(index)


def _seg_backward(ctx, grad):
    (index,) = ctx.saved_tensors
    return grad.index_select(0, index.to(torch.int64)), None, None


_register_autograd(segment_sum, _seg_backward, _seg_setup)


# ---------------------------------------------------------------------------
# Invariant RMS normalisation
# ---------------------------------------------------------------------------

@torch.library.custom_op("flashcart::rms_norm", mutates_args=())
def rms_norm(x: Tensor, weight: Tensor, l_max: int, eps: float) -> Tuple[Tensor, Tensor]:
    """(out, scale): out_l = x_l * (m + eps)^-1/2 * weight[l] with m the per-node mean of the
    rank-weighted invariants (reference src/flashcart/nn/layers.py:494-528, no centering)."""
    x = _lib.contig("x", x)
    w = _lib.contig("weight", weight)
    n = x.shape[0]
    C = w.shape[-1]
    if w.shape != (l_max + 1, C) or x.shape[-1] != (l_max + 1) ** 2 * C:
        raise RuntimeError(f"rms_norm: weight {tuple(w.shape)} / x {tuple(x.shape)} do not match l_max={l_max}.")
    out = torch.empty_like(x)
    scale = x.new_empty(n)
    _lib_call("fc_rms_norm_fwd", n, l_max, C, x.data_ptr(), w.data_ptr(), float(eps), out.data_ptr(),
              scale.data_ptr(), _lib.stream_of(x))
    return out, scale


@rms_norm.register_fake
def _(x, weight, l_max, eps):
    return torch.empty_like(x), x.new_empty(x.shape[0])


@torch.library.custom_op("flashcart::rms_norm_bwd", mutates_args=())
def rms_norm_bwd(grad_out: Tensor, x: Tensor, weight: Tensor, scale: Tensor, l_max: int) -> Tensor:
    go = _lib.contig("grad_out", grad_out)
    x = _lib.contig("x", x)
    w = _lib.contig("weight", weight)
    s = _lib.contig("scale", scale)
    gx = torch.empty_like(x)
    _lib_call("fc_rms_norm_bwd", x.shape[0], l_max, w.shape[-1], go.data_ptr(), x.data_ptr(), w.data_ptr(),
              s.data_ptr(), gx.data_ptr(), _lib.stream_of(x))
    return gx


@rms_norm_bwd.register_fake
def _(grad_out, x, weight, scale, l_max):
    return torch.empty_like(x)


def _rms_setup(ctx, inputs, output):
    x, weight, l_max, eps = inputs
    ctx.save_for_backward(x, weight, output[1])
    ctx.l_max = int(l_max)
    ctx.set_materialize_grads(False)


def _rms_backward(ctx, grad_out, grad_scale):
    """Gradients from the normalised output and, when a second derivative has been taken
    through an expression that read the saved scale, from the scale output."""
    x, weight, scale = ctx.saved_tensors
    if grad_out is None:
        grad_out = torch.zeros_like(x)
    gx = rms_norm_bwd(grad_out, x, weight, scale, ctx.l_max) if ctx.needs_input_grad[0] else None
    if gx is not None and grad_scale is not None:
        # s = (m(x) + eps)^-1/2: ds/dx = -s^3/2 dm/dx, differentiated through the torch statement
        from flashcart_amd.o3 import _torch_math as M
        with torch.enable_grad():
            xx = x if x.requires_grad else x.detach().requires_grad_(True)
            m = M.rms_mean(xx, ctx.l_max, weight.shape[-1])
            (gm,) = torch.autograd.grad(m, xx, grad_scale * (-0.5) * scale.pow(3),
                                        create_graph=torch.is_grad_enabled())
        gx = gx + gm
    gw = None
    if ctx.needs_input_grad[1]:  # d/dg_l[c] = sum_{n,a} grad_out * x * s (parameter training only)
        n, C = x.shape[0], weight.shape[-1]
        # node sum first, over the contiguous rows (a strided per-rank slice summed over nodes
        # and components is a slow reduction), then the components of each rank
        per_comp = (grad_out * x * scale.unsqueeze(-1)).view(n, -1).sum(0).view(-1, C)
        gw = torch.stack([per_comp[l * l:(l + 1) ** 2].sum(0) for l in range(ctx.l_max + 1)])
    return gx, gw, None, None


_register_autograd(rms_norm, _rms_backward, _rms_setup)


# ---------------------------------------------------------------------------
# Rank-wise gating
# ---------------------------------------------------------------------------

@torch.library.custom_op("flashcart::gate", mutates_args=())
def gate(values: Tensor, pre: Tensor, l_max: int, act: int) -> Tensor:
    """values[n, (l, a), c] * act(pre[n, l, c]); act 0 identity, 1 rescaled sigmoid
    (reference src/flashcart/nn/layers.py:609-635)."""
    v = _lib.contig("values", values)
    p = _lib.contig("pre", pre)
    n = v.shape[0]
    C = p.shape[-1] // (l_max + 1)
    if v.shape[-1] != (l_max + 1) ** 2 * C or p.shape[-1] != (l_max + 1) * C or p.shape[0] != n:
        raise RuntimeError(f"gate: values {tuple(v.shape)} / pre {tuple(p.shape)} do not match l_max={l_max}.")
    out = torch.empty_like(v)
    _lib_call("fc_gate_fwd", n, l_max, C, v.data_ptr(), p.data_ptr(), int(act), out.data_ptr(), _lib.stream_of(v))
    return out


@gate.register_fake
def _(values, pre, l_max, act):
    return torch.empty_like(values)


@torch.library.custom_op("flashcart::gate_bwd", mutates_args=())
def gate_bwd(grad_out: Tensor, values: Tensor, pre: Tensor, l_max: int, act: int, need_values: bool,
             need_pre: bool) -> Tuple[Tensor, Tensor]:
    go = _lib.contig("grad_out", grad_out)
    v = _lib.contig("values", values)
    p = _lib.contig("pre", pre)
    gv = torch.empty_like(v) if need_values else v.new_empty(0)
    gp = torch.empty_like(p) if need_pre else p.new_empty(0)
    C = p.shape[-1] // (l_max + 1)
    _lib_call("fc_gate_bwd", v.shape[0], l_max, C, go.data_ptr(), v.data_ptr(), p.data_ptr(), int(act),
              gv.data_ptr() if need_values else None, gp.data_ptr() if need_pre else None, _lib.stream_of(v))
    return gv, gp


@gate_bwd.register_fake
def _(grad_out, values, pre, l_max, act, need_values, need_pre):
    return (torch.empty_like(values) if need_values else values.new_empty(0),
            torch.empty_like(pre) if need_pre else pre.new_empty(0))


def _gate_setup(ctx, inputs, output):
    values, pre, l_max, act = inputs
    ctx.save_for_backward(values, pre)
    ctx.cfg = (int(l_max), int(act))


def _gate_backward(ctx, grad):
    values, pre = ctx.saved_tensors
    nv, np_ = ctx.needs_input_grad[0], ctx.needs_input_grad[1]
    if not (nv or np_):
        return None, None, None, None
    gv, gp = gate_bwd(grad, values, pre, *ctx.cfg, bool(nv), bool(np_))
    return (gv if nv else None), (gp if np_ else None), None, None


_register_autograd(gate, _gate_backward, _gate_setup)


# second derivatives: autograd formulas of the backward ops above
from flashcart_amd.o3 import _second_order  # noqa: E402,F401
