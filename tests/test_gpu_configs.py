"""GPU parity on the benchmark configurations' own inputs (2, 3, 5).

* cfg 1 — standalone tensor product 2 x 2 -> 2, 32 channels, single-channel in2,
  E = 4096 edges (512 receivers x 8 in-edges, senders uniform != receiver), forward
  and gradients of in1, in2, weights; plus the node-wise (dense) variant on E rows.
* cfg 2 — expansion l <= 3 + Bessel(8, r_max 5) + polynomial cutoff (p = 6) of
  200,000 vectors with d ~ U[0.8, 5.0], directions uniform on the sphere; forward and
  the gradient of a random projection with respect to the vectors.
* cfg 3 — 512 water molecules (1536 atoms) in a periodic box, C = 64, L = 2, two
  layers: energy and forces against the float64 oracle on the whole system.
* cfg 5 — 512 ragged molecules (20-50 atoms, C/H/N/O), C = 64, L = 2: the full batch on
  the GPU; a sample of molecules against the oracle (molecules do not interact, so
  each molecule's energy and forces in the batch equal those of the molecule alone),
  and the per-molecule energies against single-molecule GPU evaluations.

Bars: ops within 2e-5 relative (+ magnitude floor); energies 1e-5 relative, forces
1e-4 eV/A absolute.
"""

import math

import numpy as np
import pytest
import torch

from flashcart_amd.data import AtomicGraph, batch_graphs
from flashcart_amd.data.synthetic import model_config, molecules, water_box
from oracle import model as OM
from oracle import ops as O
from tests.helpers import assert_close

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _log(msg):
    print(msg, flush=True)


def _cfg1_inputs(conv: bool):
    rng = np.random.default_rng(0)
    n_recv, deg, E = 512, 8, 4096
    if conv:
        ii = np.repeat(np.arange(n_recv), deg)
        jj = rng.integers(0, n_recv - 1, size=E)
        jj = jj + (jj >= ii)  # uniform over senders != receiver
        n1 = n_recv
    else:
        ii = jj = None
        n1 = E
    in1 = torch.as_tensor(rng.standard_normal((n1, 9 * 32)))
    v = rng.standard_normal((E, 3))
    in2 = O.irreps(torch.as_tensor(v / np.linalg.norm(v, axis=1, keepdims=True)), 2)
    w = torch.as_tensor(rng.standard_normal((E, 11 * 32)))
    go = torch.as_tensor(rng.standard_normal((n1, 35 * 32)))
    ei = None if not conv else torch.as_tensor(np.stack([ii, jj]))
    return in1, in2, w, go, ei


@pytest.mark.parametrize("conv", [True, False], ids=["conv", "dense"])
def test_cfg1_tensor_product(conv):
    from flashcart_amd import o3
    _log(f"cfg1 conv={conv}")
    in1, in2, w, go, ei = _cfg1_inputs(conv)
    tp = o3.TensorProduct(2, 2, 2, 32, 1)
    assert tp.out_paths == [3, 4, 4] and tp.n_total_paths == 11
    leaves = [t.clone().requires_grad_(True) for t in (in1, in2, w)]
    ref = O.tensor_product(*leaves, ei[0] if conv else None, ei[1] if conv else None, 2, 2, 2, 32, 1)
    ref_g = torch.autograd.grad(ref, leaves, go)
    dev = [t.float().to(DEV).requires_grad_(True) for t in (in1, in2, w)]
    out = tp(*dev, ei[0].to(DEV) if conv else None, ei[1].to(DEV) if conv else None)
    got_g = torch.autograd.grad(out, dev, go.float().to(DEV))
    assert out.shape == (in1.shape[0], 35 * 32)
    assert_close(out, ref, 2e-5, 2e-5 * (float(ref.abs().max()) + 1), "cfg1 fwd")
    for k, (a, r) in enumerate(zip(got_g, ref_g)):
        assert_close(a, r, 2e-5, 2e-5 * (float(r.abs().max()) + 1), f"cfg1 grad {k}")


def test_cfg2_expansion_radial_cutoff():
    from flashcart_amd import _lib, o3
    from flashcart_amd.nn import BesselBasis, PolynomialCutoff
    from flashcart_amd.o3 import _ops
    _log("cfg2 200k edges")
    rng = np.random.default_rng(0)
    E = 200_000
    d = rng.uniform(0.8, 5.0, size=E)
    r = rng.standard_normal((E, 3))
    r /= np.linalg.norm(r, axis=1, keepdims=True)
    vec32 = torch.as_tensor(d[:, None] * r, dtype=torch.float32)
    v64 = vec32.double().requires_grad_(True)
    d64 = v64.norm(dim=-1)
    attrs = O.irreps(v64 / d64.unsqueeze(-1), 3)
    feats = O.bessel(d64, 8, 5.0)
    env = O.cutoff(d64, 5.0, 6)
    gen = torch.Generator().manual_seed(1)
    ga, gf, ge = (torch.randn(t.shape, generator=gen, dtype=torch.float64) for t in (attrs, feats, env))
    (ref_gv,) = torch.autograd.grad((attrs * ga).sum() + (feats * gf).sum() + (env * ge).sum(), v64)

    # the three reference modules, one op each
    v = vec32.to(DEV).requires_grad_(True)
    dd = v.norm(dim=-1)
    a = o3.Irreps(3).forward_normalized(v / dd.unsqueeze(-1))
    f = BesselBasis(8, 5.0)(dd)
    e = PolynomialCutoff(5.0, 6)(dd)
    assert_close(a, attrs, 1e-5, 1e-6, "cfg2 attrs")
    assert_close(f, feats, 1e-5, 2e-5, "cfg2 bessel")
    assert_close(e, env, 1e-5, 1e-6, "cfg2 envelope")
    loss = (a * ga.float().to(DEV)).sum() + (f * gf.float().to(DEV)).sum() + (e * ge.float().to(DEV)).sum()
    (gv,) = torch.autograd.grad(loss, v)
    assert_close(gv, ref_gv, 1e-4, 1e-4 * (float(ref_gv.abs().max()) + 1), "cfg2 grad (separate ops)")

    # the fused edge-geometry kernel on the same vectors
    idx = torch.arange(E, dtype=torch.int32, device=DEV)
    rowptr = torch.arange(E + 1, dtype=torch.int32, device=DEV)
    v2 = vec32.to(DEV).requires_grad_(True)
    a2, f2, e2 = _ops.edge_geometry(None, None, idx, idx, v2, rowptr, idx, rowptr, 3, _lib.BASIS_BESSEL, 8, 0.0,
                                    5.0, 6)
    assert_close(a2, attrs, 1e-5, 1e-6, "cfg2 fused attrs")
    assert_close(f2, feats, 1e-5, 2e-5, "cfg2 fused bessel")
    assert_close(e2, env, 1e-5, 1e-6, "cfg2 fused envelope")
    loss2 = (a2 * ga.float().to(DEV)).sum() + (f2 * gf.float().to(DEV)).sum() + (e2 * ge.float().to(DEV)).sum()
    (gv2,) = torch.autograd.grad(loss2, v2)
    assert_close(gv2, ref_gv, 1e-4, 1e-4 * (float(ref_gv.abs().max()) + 1), "cfg2 grad (fused)")


def _model(cfg, seed):
    from flashcart_amd.model import FlashCartPotential
    torch.manual_seed(seed)
    m = FlashCartPotential.from_config(cfg)
    g = torch.Generator().manual_seed(seed + 1)
    with torch.no_grad():
        for name, p in m.named_parameters():
            if "output_linear" in name or "layer_norm.weights" in name:
                p.copy_(torch.randn(p.shape, generator=g) * 0.5 + (1.0 if "layer_norm" in name else 0.0))
    return m


def test_cfg3_water_1536():
    z, p, cell, pbc = water_box(512, seed=0)
    g = AtomicGraph.from_arrays(z, p, ["H", "O"], 5.0, cell=cell, pbc=pbc)
    avg = g.edge_index.shape[1] / g.num_nodes
    _log(f"cfg3 water: {g.num_nodes} atoms, {g.edge_index.shape[1]} edges")
    assert g.num_nodes == 1536 and 45.0 < avg < 60.0
    model = _model(model_config(["H", "O"], 64, 2, avg_neighbors=avg), 31)
    ref = OM.predict(model.state_dict(), model.to_model_config(), g.to_dict(), compute_forces=True)
    out = model.to(DEV).predict(g.to(DEV), compute_forces=True)
    assert_close(out["energy"], ref["energy"], 1e-5, 1e-6, "cfg3 energy")
    assert_close(out["forces"], ref["forces"], 0.0, 1e-4, "cfg3 forces")


def test_cfg5_molecules_512():
    mols = molecules(512, seed=0)
    elements = ["H", "C", "N", "O"]
    graphs = [AtomicGraph.from_arrays(zz, pp, elements, 5.0) for zz, pp in mols]
    batch = batch_graphs(graphs)
    avg = batch.edge_index.shape[1] / batch.num_nodes
    _log(f"cfg5 molecules: {batch.num_nodes} atoms, {batch.edge_index.shape[1]} edges")
    model = _model(model_config(elements, 64, 2, avg_neighbors=avg), 41).to(DEV)
    out = model.predict(batch.to(DEV), compute_forces=True)
    assert out["energy"].shape == (512,) and out["forces"].shape == (batch.num_nodes, 3)
    starts = np.concatenate([[0], np.cumsum([g.num_nodes for g in graphs])])
    sd, mcfg = model.state_dict(), model.to_model_config()
    for k in (0, 1, 100, 257, 511):
        ref = OM.predict(sd, mcfg, graphs[k].to_dict(), compute_forces=True)
        assert_close(out["energy"][k:k + 1], ref["energy"], 1e-5, 1e-6, f"cfg5 energy mol {k}")
        assert_close(out["forces"][starts[k]:starts[k + 1]], ref["forces"], 0.0, 1e-4, f"cfg5 forces mol {k}")
    for k in range(0, 512, 37):
        single = model.predict(graphs[k].to(DEV), compute_forces=True)
        assert_close(out["energy"][k:k + 1], single["energy"], 1e-5, 1e-6, f"cfg5 batched vs single {k}")
        assert_close(out["forces"][starts[k]:starts[k + 1]], single["forces"], 0.0, 1e-4, f"cfg5 forces {k}")


def _frozen_replay(model, gdev, what):
    """``predict(use_compile=True)`` with frozen parameters, as bench.py times cfgs 3 and 5: the
    capture call and one replay, bitwise equal; the fused paths the timed step takes (edge pairs,
    the first layer as a species density, the shared input maps) must have run."""
    from flashcart_amd.nn import fused
    model.requires_grad_(False)
    fused.path_counts.clear()
    _log(f"{what}: frozen parameters, HIP graph capture")
    out = model.predict(gdev, compute_forces=True, use_compile=True)
    _log(f"{what}: replay")
    again = model.predict(gdev, compute_forces=True, use_compile=True)
    for key in ("species", "paired", "entry_maps", "product", "gated"):
        assert fused.path_counts[key] > 0, f"{what}: the timed path did not take the {key} block"
    assert torch.equal(out["energy"], again["energy"]) and torch.equal(out["forces"], again["forces"])
    return again


def test_cfg3_water_1536_timed_path():
    """The whole 1,536-atom water box through the path bench.py times (frozen parameters, edge pairs,
    species density, HIP graph replay) against the float64 oracle at the north-star bars."""
    z, p, cell, pbc = water_box(512, seed=0)
    g = AtomicGraph.from_arrays(z, p, ["H", "O"], 5.0, cell=cell, pbc=pbc)
    avg = g.edge_index.shape[1] / g.num_nodes
    model = _model(model_config(["H", "O"], 64, 2, avg_neighbors=avg), 31)
    ref = OM.predict(model.state_dict(), model.to_model_config(), g.to_dict(), compute_forces=True)
    out = _frozen_replay(model.to(DEV), g.to(DEV), "cfg3 water")
    assert_close(out["energy"], ref["energy"], 1e-5, 1e-6, "cfg3 replay energy")
    assert_close(out["forces"], ref["forces"], 0.0, 1e-4, "cfg3 replay forces")


def test_cfg5_molecules_512_timed_path():
    """The full 512-molecule batch through the timed path (frozen, pairs, species density, replay);
    a sample of molecules against the float64 oracle, and every molecule's energy against the
    eager per-edge evaluation of the same batch."""
    mols = molecules(512, seed=0)
    elements = ["H", "C", "N", "O"]
    graphs = [AtomicGraph.from_arrays(zz, pp, elements, 5.0) for zz, pp in mols]
    batch = batch_graphs(graphs)
    avg = batch.edge_index.shape[1] / batch.num_nodes
    model = _model(model_config(elements, 64, 2, avg_neighbors=avg), 41).to(DEV)
    per_edge = model.predict(batch.to(DEV), compute_forces=True)  # trainable: the per-edge path
    out = _frozen_replay(model, batch.to(DEV), "cfg5 molecules")
    assert out["energy"].shape == (512,)
    assert_close(out["energy"], per_edge["energy"], 1e-5, 1e-6, "cfg5 replay vs per-edge energies")
    assert_close(out["forces"], per_edge["forces"], 0.0, 1e-4, "cfg5 replay vs per-edge forces")
    starts = np.concatenate([[0], np.cumsum([g.num_nodes for g in graphs])])
    sd, mcfg = model.state_dict(), model.to_model_config()
    for k in (0, 3, 128, 300, 511):
        ref = OM.predict(sd, mcfg, graphs[k].to_dict(), compute_forces=True)
        assert_close(out["energy"][k:k + 1], ref["energy"], 1e-5, 1e-6, f"cfg5 replay energy mol {k}")
        assert_close(out["forces"][starts[k]:starts[k + 1]], ref["forces"], 0.0, 1e-4, f"cfg5 replay forces mol {k}")
