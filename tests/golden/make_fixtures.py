"""Writes the golden fixtures of tests/golden/ from the reference's own modules.

Runs only in the build container, where the reference is mounted read-only at
/root/reference (it never travels to the GPU box; the committed .npz files do):

    python tests/golden/make_fixtures.py            # all fixtures
    python tests/golden/make_fixtures.py potential_default

Every fixture is produced by the reference's own code on CPU in float64:
``flashcart.o3`` (TensorProduct, LinearLayer, Irreps), ``flashcart.nn`` (InteractionLayer,
RMSLayerNorm, EquivariantGatedLayer, ProductLayer, EnergyReadoutLayer, ChebyshevBasis,
PolynomialCutoff), ``flashcart.utils.geometry.get_edge_vectors`` and
``flashcart.model.atomistic.AtomisticModel.predict`` (forces and stress). The Triton path
is off (``use_triton=False``), so the reference's CPU PyTorch ops run; their generated
modules are written to a temporary ``FLASHCART_CACHE_DIR``.

``flashcart.model.flashcart`` imports ``lightning.fabric``, which is not installed here, so
``FlashCartPotential`` itself cannot be imported. ``_Potential`` below is an
``AtomisticModel`` that builds the reference's layer objects in the order of
``FlashCartPotential.__init__`` (src/flashcart/model/flashcart.py:151-221) and chains them as
its ``forward`` does (:249-317); no module is stubbed or replaced.

A fixture is one .npz of named arrays:
  meta        JSON string: the constructor arguments and the kind of fixture
  sd/<key>    state dict the outputs were computed with (float64 parameters)
  init/<key>  (potentials) the float32 state dict drawn by torch.manual_seed(1234)
  in/<name>   inputs; out/<name> outputs
  cot/<name>  cotangents; grad/<name>, pgrad/<key> vector-Jacobian products for them
"""

from __future__ import annotations

import json
import os
import sys
import tempfile

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
REF_SRC = "/root/reference/src"


def _import_reference():
    if not os.path.isdir(REF_SRC):
        raise SystemExit(f"{REF_SRC} not found: fixtures are written in the build container only")
    os.environ["FLASHCART_CACHE_DIR"] = tempfile.mkdtemp(prefix="flashcart_codegen_")
    sys.path.insert(0, REF_SRC)
    import importlib.util

    import flashcart.nn as fnn
    from flashcart import o3
    from flashcart.utils.geometry import get_edge_vectors, uses_periodic_shifts
    from flashcart.utils.torch_geometric.data import Data

    # flashcart/model/__init__.py imports flashcart.model.flashcart (and with it lightning), so
    # the reference's atomistic.py is executed from its own file, outside that package initializer.
    path = os.path.join(REF_SRC, "flashcart", "model", "atomistic.py")
    spec = importlib.util.spec_from_file_location("_reference_atomistic", path)
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return o3, fnn, mod.AtomisticModel, Data, get_edge_vectors, uses_periodic_shifts


o3, fnn, AtomisticModel, Data, get_edge_vectors, uses_periodic_shifts = _import_reference()
from flashcart.nn import layers as NNL  # noqa: E402  (after the reference path is on sys.path)
from flashcart.nn.radial import ChebyshevBasis, PolynomialCutoff  # noqa: E402

F64 = torch.float64


# ----------------------------------------------------------------------------- helpers

def _np(t: torch.Tensor) -> np.ndarray:
    return t.detach().cpu().numpy()


def _perturb(module: torch.nn.Module, gen: torch.Generator, scale: float = 0.4) -> None:
    """Add N(0, scale^2) to every floating parameter, so that zero- or one-initialised
    parameters (gated output maps, path deltas, norm gains) take part in the result."""
    with torch.no_grad():
        for p in module.parameters():
            p.add_(scale * torch.randn(p.shape, generator=gen, dtype=p.dtype))


def _vjp(outputs, inputs, params, gen):
    """Cotangents for the outputs, and the gradients of <outputs, cotangents> w.r.t.
    the inputs and parameters."""
    cots = [torch.randn(o.shape, generator=gen, dtype=o.dtype) for o in outputs]
    named = list(params)
    leaves = list(inputs) + [p for _, p in named]
    grads = torch.autograd.grad(outputs, leaves, cots, allow_unused=True)
    gin = [g if g is not None else torch.zeros_like(x) for g, x in zip(grads[:len(inputs)], inputs)]
    gp = {k: (g if g is not None else torch.zeros_like(p)) for (k, p), g in zip(named, grads[len(inputs):])}
    return cots, gin, gp


def _save(name: str, meta: dict, sd: dict, ins: dict, outs: dict, cots: dict = None, grads: dict = None,
          pgrads: dict = None, init: dict = None) -> None:
    arrays = {"meta": np.array(json.dumps(meta, sort_keys=True))}
    for prefix, d in (("sd", sd), ("in", ins), ("out", outs), ("cot", cots), ("grad", grads),
                      ("pgrad", pgrads), ("init", init)):
        for k, v in (d or {}).items():
            arrays[f"{prefix}/{k}"] = _np(v) if torch.is_tensor(v) else np.asarray(v)
    path = os.path.join(HERE, f"{name}.npz")
    np.savez_compressed(path, **arrays)
    print(f"wrote {os.path.relpath(path)} ({os.path.getsize(path) / 1024:.1f} KiB, {len(arrays)} arrays)")


def _unit(n, gen):
    v = torch.randn(n, 3, generator=gen, dtype=F64)
    return v / v.norm(dim=-1, keepdim=True)


def _csr_edges(n_nodes, degrees, gen):
    """Receiver-sorted edges; receiver i gets degrees[i % len(degrees)] random senders != i."""
    ii, jj = [], []
    for i in range(n_nodes):
        for _ in range(degrees[i % len(degrees)]):
            j = int(torch.randint(0, n_nodes - 1, (1,), generator=gen))
            ii.append(i)
            jj.append(j if j < i else j + 1)
    return torch.tensor([ii, jj], dtype=torch.long)


def _edge_inputs(n_edges, l_max, n_radial, r_max, gen, mapping="cosine"):
    """Edge attributes, radial features and envelope from the reference's own modules."""
    u = _unit(n_edges, gen)
    d = 0.6 + (r_max - 0.4) * torch.rand(n_edges, generator=gen, dtype=F64)
    attrs = o3.Irreps(l_max).forward_normalized(u)
    feats = ChebyshevBasis(n_radial, r_max=r_max, r_min=0.0, mapping=mapping).to(F64)(d)
    env = PolynomialCutoff(r_max, poly_order=6).to(F64)(d)
    return attrs, feats, env


def _pairs(pos: np.ndarray, cell: np.ndarray, pbc, r: float):
    """Brute-force neighbour pairs (i, j, S) with |pos[j] - pos[i] + S.cell| < r, self pairs with
    S = 0 dropped, ordered by (i, j, S) (reference data/neighbors.py:120-143 semantics)."""
    reach = []
    for a in range(3):
        if pbc[a]:
            other = np.cross(cell[(a + 1) % 3], cell[(a + 2) % 3])
            spacing = abs(np.dot(cell[a], other)) / np.linalg.norm(other)
            reach.append(int(np.ceil(r / spacing)) + 1)
        else:
            reach.append(0)
    out = []
    n = pos.shape[0]
    for sx in range(-reach[0], reach[0] + 1):
        for sy in range(-reach[1], reach[1] + 1):
            for sz in range(-reach[2], reach[2] + 1):
                s = np.array([sx, sy, sz])
                off = s @ cell
                d = np.linalg.norm(pos[None, :, :] - pos[:, None, :] + off, axis=-1)
                for i, j in zip(*np.nonzero(d < r)):
                    if i == j and not s.any():
                        continue
                    out.append((int(i), int(j), sx, sy, sz))
    out.sort()
    arr = np.array(out, dtype=np.int64).reshape(-1, 5)
    return arr[:, :2].T.copy(), arr[:, 2:].astype(np.int64)


def _graph(structs, r_max):
    """Batched graph dict of a list of (numbers->types, positions, cell, pbc)."""
    ei, sh, pos, cells, batch, types, n_atoms, off = [], [], [], [], [], [], [], 0
    for g, (t, p, c, pbc) in enumerate(structs):
        e, s = _pairs(p, c, pbc, r_max)
        ei.append(e + off)
        sh.append(s)
        pos.append(p)
        cells.append(c)
        batch.append(np.full(len(t), g))
        types.append(t)
        n_atoms.append(len(t))
        off += len(t)
    return dict(edge_index=torch.tensor(np.concatenate(ei, 1)), shifts=torch.tensor(np.concatenate(sh, 0)),
                positions=torch.tensor(np.concatenate(pos, 0), dtype=F64), cell=torch.tensor(np.stack(cells), dtype=F64),
                batch=torch.tensor(np.concatenate(batch)), atom_types=torch.tensor(np.concatenate(types)),
                n_atoms=torch.tensor(n_atoms), pbc=torch.tensor(np.stack([s[3] for s in structs])))


def _state(module):
    return {k: v for k, v in module.state_dict().items()}


def _params(module):
    return [(k, p) for k, p in module.named_parameters()]


# ----------------------------------------------------------------------------- o3 fixtures

def fx_tp(name, gen, l1, l2, lo, f1, f2, conv=False, sym=False, shared=False, reduced=False, rows=6,
          degrees=(3, 0, 5, 1, 4, 2)):
    """TensorProduct forward and VJP (o3/tensor_product.py:84-155): output and weight layout,
    path order (canonical, then swapped), broadcast of single-feature operands, the conv
    gather by idx_j and scatter to idx_i."""
    tp = o3.TensorProduct(l1, l2, lo, f1, f2, symmetric_product=sym, shared_weights=shared,
                          reduce_paths=reduced).to(F64)
    C = max(f1, f2)
    in1 = torch.randn(rows, (l1 + 1) ** 2 * f1, generator=gen, dtype=F64)
    if conv:
        ei = _csr_edges(rows, degrees, gen)
        n2 = ei.shape[1]
    else:
        ei = None
        n2 = rows
    if f2 == 1:
        in2 = o3.Irreps(l2).forward_normalized(_unit(n2, gen))
    else:
        in2 = in1.clone() if sym else torch.randn(n2, (l2 + 1) ** 2 * f2, generator=gen, dtype=F64)
    P = tp.n_total_paths
    w = torch.randn((P * C,) if shared else (n2, P * C), generator=gen, dtype=F64)
    ins = [in1.requires_grad_(), w.requires_grad_()]
    if not sym:
        ins.insert(1, in2.requires_grad_())
        out = tp(in1, in2, w, ei[0] if conv else None, ei[1] if conv else None)
    else:
        out = tp(in1, in1, w)
    cots, g, _ = _vjp([out], ins, [], gen)
    meta = dict(kind="tp", in1_l_max=l1, in2_l_max=l2, out_l_max=lo, in1_features=f1, in2_features=f2,
                symmetric_product=sym, shared_weights=shared, reduce_paths=reduced, conv=conv,
                out_paths=list(tp.out_paths), n_total_paths=P)
    ins_d = {"in1": in1, "weights": w}
    grads = {"in1": g[0], "weights": g[-1]}
    if not sym:
        ins_d["in2"] = in2
        grads["in2"] = g[1]
    if conv:
        ins_d["edge_index"] = ei
    _save(name, meta, {}, ins_d, {"out": out}, {"out": cots[0]}, grads)


def fx_linear(name, gen, lin, lout, fin, fout, in_paths=None, rows=7):
    """o3.LinearLayer (o3/linear.py:88-128): per-rank maps, K index path*C + f inside a
    TP-output block, scale (C_in*paths_l)^-1/2, zero output ranks above min(in, out)."""
    torch.manual_seed(7)
    lay = o3.LinearLayer(lin, lout, fin, fout, in_paths=in_paths).to(F64)
    paths = in_paths or [1] * (lin + 1)
    x = torch.randn(rows, sum((2 * l + 1) * fin * paths[l] for l in range(lin + 1)), generator=gen,
                    dtype=F64).requires_grad_()
    out = lay(x)
    cots, g, gp = _vjp([out], [x], _params(lay), gen)
    meta = dict(kind="linear", in_l_max=lin, out_l_max=lout, in_features=fin, out_features=fout,
                in_paths=in_paths)
    _save(name, meta, _state(lay), {"x": x}, {"out": out}, {"out": cots[0]}, {"x": g[0]}, gp)


# ----------------------------------------------------------------------------- nn fixtures

def fx_interaction(name, gen, lin, L, C=4, hidden=(8, 8), n_elements=None, ef=None, avg=7.3):
    """InteractionLayer forward + VJP (nn/layers.py:310-379) with skip connection and RMS norm."""
    torch.manual_seed(11)
    lay = NNL.InteractionLayer(lin, L, L, C, C, n_radial=8, hidden_radial=list(hidden), n_elements=n_elements,
                             element_features=ef, avg_neighbors=avg, use_sc=True, use_layer_norm=True).to(F64)
    _perturb(lay, gen)
    n = 7
    ei = _csr_edges(n, (3, 5, 0, 2, 6, 4, 1), gen)
    attrs, feats, env = _edge_inputs(ei.shape[1], L, 8, 5.0, gen)
    x = torch.randn(n, (lin + 1) ** 2 * C, generator=gen, dtype=F64)
    types = torch.randint(0, n_elements or 1, (n,), generator=gen)
    ins = [t.requires_grad_() for t in (x, attrs, feats, env)]
    out = lay(x, attrs, feats, ei, env, atom_types=types if n_elements else None)
    cots, g, gp = _vjp([out], ins, _params(lay), gen)
    meta = dict(kind="interaction", in1_l_max=lin, in2_l_max=L, out_l_max=L, in1_features=C, out_features=C,
                n_radial=8, hidden_radial=list(hidden), n_elements=n_elements, element_features=ef,
                avg_neighbors=avg, use_sc=True, use_layer_norm=True)
    _save(name, meta, _state(lay),
          {"node_feats": x, "edge_attrs": attrs, "edge_feats": feats, "envelope": env, "edge_index": ei,
           "atom_types": types},
          {"out": out}, {"out": cots[0]},
          {"node_feats": g[0], "edge_attrs": g[1], "edge_feats": g[2], "envelope": g[3]}, gp)


def fx_rms(name, gen, l_max, C):
    """RMSLayerNorm (nn/layers.py:494-528), eps 1e-6 as the model builds it."""
    lay = NNL.RMSLayerNorm(l_max, C, eps=1.0e-6).to(F64)
    _perturb(lay, gen)
    x = torch.randn(9, (l_max + 1) ** 2 * C, generator=gen, dtype=F64).requires_grad_()
    out = lay(x)
    cots, g, gp = _vjp([out], [x], _params(lay), gen)
    _save(name, dict(kind="rms_norm", l_max=l_max, n_features=C, eps=1.0e-6), _state(lay), {"x": x},
          {"out": out}, {"out": cots[0]}, {"x": g[0]}, gp)


def fx_gated(name, gen, l_max, C, act):
    """EquivariantGatedLayer (nn/layers.py:609-635); the zero-initialised output map is perturbed."""
    torch.manual_seed(13)
    lay = NNL.EquivariantGatedLayer(l_max, C, C, gate_activation=act, gate_bias=True).to(F64)
    _perturb(lay, gen)
    x = torch.randn(8, (l_max + 1) ** 2 * C, generator=gen, dtype=F64).requires_grad_()
    out = lay(x)
    cots, g, gp = _vjp([out], [x], _params(lay), gen)
    _save(name, dict(kind="gated", l_max=l_max, in_features=C, gate_activation=act, gate_bias=True),
          _state(lay), {"x": x}, {"out": out}, {"out": cots[0]}, {"x": g[0]}, gp)


def fx_product(name, gen, L_in, L_out, C, corr, reduced, n_elements=None):
    """ProductLayer (nn/layers.py:949-995) with skip connection and RMS norm."""
    torch.manual_seed(17)
    lay = NNL.ProductLayer(L_in, L_out, C, n_elements=n_elements, correlation=corr, path_reduced=reduced,
                         use_sc=True, use_layer_norm=True).to(F64)
    _perturb(lay, gen, 0.3)
    n = 8
    x = torch.randn(n, (L_in + 1) ** 2 * C, generator=gen, dtype=F64).requires_grad_()
    types = torch.randint(0, n_elements or 1, (n,), generator=gen)
    out = lay(x, types if n_elements else None)
    cots, g, gp = _vjp([out], [x], _params(lay), gen)
    _save(name, dict(kind="product", in_l_max=L_in, out_l_max=L_out, in_features=C, correlation=corr,
                     path_reduced=reduced, n_elements=n_elements, use_sc=True, use_layer_norm=True),
          _state(lay), {"x": x, "atom_types": types}, {"out": out}, {"out": cots[0]}, {"x": g[0]}, gp)


def fx_readout(name, gen, C, n_layers, hidden):
    """EnergyReadoutLayer (nn/layers.py:1045-1063): MLP on the first C columns of every layer."""
    torch.manual_seed(19)
    lay = NNL.EnergyReadoutLayer(C, n_layers, hidden_readout=list(hidden)).to(F64)
    xs = [torch.randn(6, C * (2 * k + 1), generator=gen, dtype=F64).requires_grad_() for k in range(n_layers)]
    out = lay(xs)
    cots, g, gp = _vjp([out], xs, _params(lay), gen)
    _save(name, dict(kind="readout", in_features=C, n_layers=n_layers, hidden_readout=list(hidden)), _state(lay),
          {f"x{k}": x for k, x in enumerate(xs)}, {"out": out}, {"out": cots[0]},
          {f"x{k}": gk for k, gk in enumerate(g)}, gp)


# ----------------------------------------------------------------------------- potential fixtures

class _Potential(AtomisticModel):
    """The module tree of FlashCartPotential (src/flashcart/model/flashcart.py:92-221) built from
    the reference's layer classes in its construction order (so a seed draws the same initial
    parameters under the same state-dict keys), and its forward (:249-317) without the LAMMPS
    exchange branch."""

    def __init__(self, elements, r_max, r_min=0.0, n_hidden_feats=32, l_max_hidden_feats=1, l_max_edge_attrs=3,
                 n_radial=8, n_interactions=2, correlation=3, path_reduced_product=True,
                 element_agnostic_interaction=True, element_agnostic_product=True, n_element_interaction_features=16,
                 nonlinearity=False, gate_activation="silu", gate_bias=True, layer_norm=False, hidden_radial=None,
                 hidden_readout=None, radial_mapping="affine", cutoff_poly_order=6, avg_neighbors=None, **_):
        super().__init__()
        C, Lh, Le = n_hidden_feats, l_max_hidden_feats, l_max_edge_attrs
        self.n_hidden_feats = C
        self.nonlinearity = nonlinearity
        self.element_agnostic_interaction = element_agnostic_interaction
        self.element_agnostic_product = element_agnostic_product
        hidden_radial = [64, 64] if hidden_radial is None else list(hidden_radial)
        hidden_readout = [64, 64] if hidden_readout is None else list(hidden_readout)
        avg = 1.0 if avg_neighbors is None else float(avg_neighbors)
        self.embedding = torch.nn.Embedding(len(elements), C)
        self.radial_basis = ChebyshevBasis(n_radial, r_max=r_max, r_min=r_min, mapping=radial_mapping)
        self.cutoff_fn = PolynomialCutoff(r_max, poly_order=cutoff_poly_order)
        self.irreps = o3.Irreps(Le)
        prod_out = [Lh if k < n_interactions - 1 else 0 for k in range(n_interactions)]
        int_in = [0 if k == 0 else Lh for k in range(n_interactions)]
        self.use_products = correlation > 1
        int_out = [Le] * n_interactions if self.use_products else prod_out
        self.interactions = torch.nn.ModuleList([
            NNL.InteractionLayer(in1_l_max=a, in2_l_max=Le, out_l_max=b, in1_features=C, out_features=C,
                               n_radial=n_radial, hidden_radial=hidden_radial,
                               n_elements=None if element_agnostic_interaction else len(elements),
                               element_features=n_element_interaction_features, avg_neighbors=avg, use_sc=True,
                               use_layer_norm=layer_norm)
            for a, b in zip(int_in, int_out)])
        self.products = torch.nn.ModuleList([
            NNL.ProductLayer(in_l_max=Le, out_l_max=p, in_features=C,
                           n_elements=None if element_agnostic_product else len(elements), correlation=correlation,
                           path_reduced=path_reduced_product, use_sc=True, use_layer_norm=layer_norm)
            for p in prod_out] if self.use_products else [])
        if nonlinearity:
            self.nonlinearities = torch.nn.ModuleList([
                NNL.EquivariantGatedLayer(l_max=b, in_features=C, hidden_features=C, gate_activation=gate_activation,
                                        gate_bias=gate_bias) for b in int_out])
        self.readout = NNL.EnergyReadoutLayer(C, n_interactions, hidden_readout=hidden_readout)
        self.scale_shift = NNL.ScaleShiftEnergyLayer(len(elements))

    def forward(self, graph):
        ei, batch, types = graph["edge_index"], graph["batch"], graph["atom_types"]
        use_shifts = graph.get("use_shifts", True)
        if not isinstance(use_shifts, bool):
            use_shifts = uses_periodic_shifts(use_shifts)
        vectors = get_edge_vectors(graph["positions"], graph["cell"], graph["shifts"], ei, batch,
                                   use_shifts=use_shifts)
        d = vectors.norm(dim=-1)
        u = vectors / d.clamp_min(1.0e-4).unsqueeze(-1)
        attrs = self.irreps.forward_normalized(u)
        feats = self.radial_basis(d)
        env = self.cutoff_fn(d)
        x = self.embedding(types)
        outs = []
        for k, inter in enumerate(self.interactions):
            y = inter(x, attrs, feats, ei, env, atom_types=types if not self.element_agnostic_interaction else None)
            if self.nonlinearity:
                y = self.nonlinearities[k](y)
            if self.use_products:
                x = self.products[k](y, None if self.element_agnostic_product else types)
            else:
                x = y
            outs.append(x[:, : self.n_hidden_feats])
        return self.scale_shift(self.readout(outs), types)


def fx_potential(name, cfg, structs, gen, stress=True):
    """Energies, site energies, forces and (periodic) stress of the potential through the
    reference's AtomisticModel.predict (model/atomistic.py:75-156,276-340), plus the initial
    state dict of torch.manual_seed(1234) (float32, default dtype, as constructed)."""
    torch.manual_seed(1234)
    model = _Potential(**cfg)
    init = {k: v.clone() for k, v in model.state_dict().items()}
    model = model.to(F64)
    _perturb(model, gen, 0.3)
    with torch.no_grad():  # the per-element scales are buffers: make them differ from 1 too
        model.scale_shift.scales.copy_(1.0 + 0.3 * torch.randn(len(cfg["elements"]), generator=gen, dtype=F64))
    g = _graph(structs, cfg["r_max"])
    data = Data(**{k: v for k, v in g.items()})
    out = model.predict(data, compute_forces=True, compute_stress=stress)
    outs = {"node_energies": out["node_energies"], "energy": out["energy"], "forces": out["forces"]}
    if stress:
        outs["stress"] = out["stress"]
    meta = dict(kind="potential", config=cfg, stress=stress)
    _save(name, meta, _state(model), g, outs, init=init)


def _fcc(n, a, gen, jitter=0.1):
    basis = np.array([[0, 0, 0], [0.5, 0.5, 0], [0.5, 0, 0.5], [0, 0.5, 0.5]])
    grid = np.stack(np.meshgrid(*[np.arange(n)] * 3, indexing="ij"), -1).reshape(-1, 3)
    pos = ((grid[:, None, :] + basis[None]) * a).reshape(-1, 3)
    pos = pos + jitter * torch.randn(pos.shape, generator=gen, dtype=F64).numpy()
    return pos, np.diag([n * a] * 3)


def _molecule(n, gen):
    pos = [np.zeros(3)]
    while len(pos) < n:
        v = torch.randn(3, generator=gen, dtype=F64).numpy()
        step = pos[-1] + v / np.linalg.norm(v) * (1.0 + 0.5 * float(torch.rand(1, generator=gen)))
        if np.min(np.linalg.norm(np.array(pos) - step, axis=1)) > 0.9:
            pos.append(step)
    return np.array(pos)


def _default_cfg(elements, C, L, **kw):
    """The packaged default architecture (configs/default.yaml:27-49) with small MLP widths."""
    cfg = dict(elements=list(elements), r_max=5.0, r_min=0.0, n_hidden_feats=C, l_max_hidden_feats=2,
               l_max_edge_attrs=L, n_radial=8, n_interactions=2, correlation=3, path_reduced_product=False,
               element_agnostic_interaction=True, element_agnostic_product=True, n_element_interaction_features=16,
               nonlinearity=True, gate_activation="sigmoid", gate_bias=True, layer_norm=True, hidden_radial=[16, 16],
               hidden_readout=[16, 16], radial_mapping="cosine", cutoff_poly_order=6, avg_neighbors=21.5)
    cfg.update(kw)
    return cfg


def _all(gen_seed: int = 20240601):
    def G(k):
        return torch.Generator().manual_seed(gen_seed + k)

    jobs = {}
    # o3: the layouts and path orders the model runs through
    jobs["tp_conv_2x3_3"] = lambda: fx_tp("tp_conv_2x3_3", G(1), 2, 3, 3, 4, 1, conv=True)
    jobs["tp_conv_0x3_3"] = lambda: fx_tp("tp_conv_0x3_3", G(2), 0, 3, 3, 4, 1, conv=True)
    jobs["tp_conv_1x2_2"] = lambda: fx_tp("tp_conv_1x2_2", G(3), 1, 2, 2, 3, 1, conv=True)
    jobs["tp_rows_3x3_3"] = lambda: fx_tp("tp_rows_3x3_3", G(4), 3, 3, 3, 4, 4, shared=True)
    jobs["tp_rows_3x3_2_reduced"] = lambda: fx_tp("tp_rows_3x3_2_reduced", G(5), 3, 3, 2, 4, 4, shared=True,
                                                  reduced=True)
    jobs["tp_rows_3x3_3_perrow"] = lambda: fx_tp("tp_rows_3x3_3_perrow", G(6), 3, 3, 3, 4, 4)
    jobs["tp_rows_3x0_3"] = lambda: fx_tp("tp_rows_3x0_3", G(7), 3, 0, 3, 4, 1, shared=True)
    jobs["tp_sym_3x3_0"] = lambda: fx_tp("tp_sym_3x3_0", G(8), 3, 3, 0, 4, 4, sym=True, shared=True)
    jobs["linear_inpaths"] = lambda: fx_linear("linear_inpaths", G(9), 3, 3, 4, 5, in_paths=[3, 5, 5, 4])
    jobs["linear_up"] = lambda: fx_linear("linear_up", G(10), 1, 3, 4, 3)
    jobs["linear_down"] = lambda: fx_linear("linear_down", G(11), 3, 0, 3, 4)
    # nn layers
    jobs["interaction_l0"] = lambda: fx_interaction("interaction_l0", G(12), 0, 3)
    jobs["interaction_l2"] = lambda: fx_interaction("interaction_l2", G(13), 2, 3)
    jobs["interaction_elem"] = lambda: fx_interaction("interaction_elem", G(14), 1, 2, n_elements=3, ef=2)
    jobs["rms_norm_l3"] = lambda: fx_rms("rms_norm_l3", G(15), 3, 4)
    jobs["gated_sigmoid"] = lambda: fx_gated("gated_sigmoid", G(16), 3, 4, "sigmoid")
    jobs["gated_silu"] = lambda: fx_gated("gated_silu", G(17), 2, 4, "silu")
    jobs["product_full"] = lambda: fx_product("product_full", G(18), 3, 2, 4, 3, False)
    jobs["product_full_out0"] = lambda: fx_product("product_full_out0", G(19), 3, 0, 4, 3, False)
    jobs["product_reduced"] = lambda: fx_product("product_reduced", G(20), 3, 2, 4, 3, True)
    jobs["product_elem"] = lambda: fx_product("product_elem", G(21), 2, 1, 4, 3, False, n_elements=3)
    jobs["product_elem_reduced"] = lambda: fx_product("product_elem_reduced", G(22), 2, 0, 4, 2, True, n_elements=3)
    jobs["readout"] = lambda: fx_readout("readout", G(23), 4, 3, (8, 8))

    # potentials
    def pot_default():
        g = G(30)
        pos, cell = _fcc(2, 3.6, g)
        types = torch.randint(0, 4, (pos.shape[0],), generator=g).numpy()
        fx_potential("potential_default", _default_cfg(["Cu", "Ni", "Fe", "Cr"], 8, 3),
                     [(types, pos, cell, np.array([True] * 3))], g)

    def pot_elem():
        g = G(31)
        structs = []
        for n in (6, 9):
            structs.append((torch.randint(0, 4, (n,), generator=g).numpy(), _molecule(n, g), np.zeros((3, 3)),
                            np.array([False] * 3)))
        cfg = _default_cfg(["H", "C", "N", "O"], 6, 2, l_max_hidden_feats=1, path_reduced_product=True,
                           element_agnostic_interaction=False, element_agnostic_product=False,
                           n_element_interaction_features=3, gate_activation="silu", avg_neighbors=4.7)
        fx_potential("potential_elem", cfg, structs, g, stress=False)

    def pot_plain():
        g = G(32)
        cell = np.array([[6.0, 0.0, 0.0], [1.5, 6.2, 0.0], [0.7, 1.1, 5.8]])
        frac = torch.rand(14, 3, generator=g, dtype=F64).numpy()
        types = torch.randint(0, 2, (14,), generator=g).numpy()
        cfg = _default_cfg(["H", "O"], 4, 2, l_max_hidden_feats=1, n_interactions=3, correlation=1,
                           nonlinearity=False, layer_norm=False, radial_mapping="affine", r_max=4.0,
                           avg_neighbors=9.0)
        fx_potential("potential_plain", cfg, [(types, frac @ cell, cell, np.array([True] * 3))], g)

    jobs["potential_default"] = pot_default
    jobs["potential_elem"] = pot_elem
    jobs["potential_plain"] = pot_plain
    return jobs


if __name__ == "__main__":
    torch.set_num_threads(min(8, os.cpu_count() or 1))
    jobs = _all()
    names = sys.argv[1:] or list(jobs)
    for n in names:
        jobs[n]()
