"""The oracle against the reference's own outputs (CPU, float64).

Every fixture under tests/golden/ was written by tests/golden/make_fixtures.py from the
reference's modules (flashcart.o3, flashcart.nn, AtomisticModel.predict). Here each oracle
function runs on the fixture's inputs and state dict and must reproduce the outputs and the
vector-Jacobian products (w.r.t. inputs and parameters) to float64 round-off. These pin the
oracle's layouts, path order and layer wiring, which the closed-form checks of test_oracle.py
leave open.
"""

import pytest
import torch

from tests.helpers import assert_close, golden_names, load_golden
from oracle import model as OM
from oracle import ops as O

RTOL = 1e-9


def _close(got, want, what):
    scale = float(want.abs().max()) if want.numel() else 1.0
    assert_close(got, want, rtol=RTOL, atol=1e-11 * max(scale, 1.0), what=what)


def _leaves(d):
    return {k: v.clone().requires_grad_(v.is_floating_point()) for k, v in d.items()}


def _check_vjp(fx, out, ins, sd=None):
    _close(out, fx["out"]["out"], "out")
    names = [k for k in fx.get("grad", {})]
    pnames = [k for k in fx.get("pgrad", {})]
    leaves = [ins[k] for k in names] + [sd[k] for k in pnames]
    grads = torch.autograd.grad(out, leaves, fx["cot"]["out"], allow_unused=True)
    for k, g, leaf in zip(names + pnames, grads, leaves):
        want = fx["grad"][k] if k in fx["grad"] else fx["pgrad"][k]
        _close(torch.zeros_like(leaf) if g is None else g, want, f"d/d{k}")


def _prefixed(sd, prefix="m"):
    return {f"{prefix}.{k}": v for k, v in sd.items()}


@pytest.mark.parametrize("form", ["einsum", "components"])
@pytest.mark.parametrize("name", golden_names("tp"))
def test_tensor_product(name, form):
    """Both evaluation forms of the oracle's tensor product (the dense einsum, and the
    per-component op sequence that the CPU baseline times) against the reference."""
    import contextlib

    with (O.components_form() if form == "components" else contextlib.nullcontext()):
        _tensor_product(name)


def _tensor_product(name):
    fx = load_golden(name)
    m = fx["meta"]
    ins = _leaves(fx["in"])
    ei = fx["in"].get("edge_index")
    in2 = ins["in1"] if m["symmetric_product"] else ins["in2"]
    out = O.tensor_product(ins["in1"], in2, ins["weights"], ei[0] if ei is not None else None,
                           ei[1] if ei is not None else None, m["in1_l_max"], m["in2_l_max"], m["out_l_max"],
                           m["in1_features"], m["in2_features"], m["symmetric_product"], m["shared_weights"],
                           m["reduce_paths"])
    _check_vjp(fx, out, ins)


@pytest.mark.parametrize("name", golden_names("linear"))
def test_linear(name):
    fx = load_golden(name)
    m = fx["meta"]
    ins = _leaves(fx["in"])
    sd = _leaves(fx["sd"])
    n = min(m["in_l_max"], m["out_l_max"]) + 1
    out = O.linear(ins["x"], [sd[f"weight.{l}"] for l in range(n)], m["in_l_max"], m["out_l_max"],
                   m["in_features"], m["out_features"], m["in_paths"])
    _check_vjp(fx, out, ins, sd)


@pytest.mark.parametrize("name", golden_names("interaction"))
def test_interaction(name):
    fx = load_golden(name)
    m = fx["meta"]
    ins = _leaves(fx["in"])
    sd = _leaves(fx["sd"])
    cfg = dict(n_hidden_feats=m["in1_features"], l_max_edge_attrs=m["in2_l_max"], hidden_radial=m["hidden_radial"],
               layer_norm=m["use_layer_norm"])
    out = OM.interaction(_prefixed(sd), "m", cfg, m["in1_l_max"], m["out_l_max"], ins["node_feats"],
                         ins["edge_attrs"], ins["edge_feats"], ins["envelope"], fx["in"]["edge_index"],
                         atom_types=fx["in"]["atom_types"])
    _check_vjp(fx, out, ins, sd)


@pytest.mark.parametrize("name", golden_names("rms_norm"))
def test_rms_norm(name):
    fx = load_golden(name)
    m = fx["meta"]
    ins, sd = _leaves(fx["in"]), _leaves(fx["sd"])
    out = OM.rms_norm(_prefixed(sd), "m", ins["x"], m["l_max"], m["n_features"], m["eps"])
    _check_vjp(fx, out, ins, sd)


@pytest.mark.parametrize("name", golden_names("gated"))
def test_gated(name):
    fx = load_golden(name)
    m = fx["meta"]
    ins, sd = _leaves(fx["in"]), _leaves(fx["sd"])
    cfg = dict(n_hidden_feats=m["in_features"], gate_activation=m["gate_activation"])
    out = OM.gated(_prefixed(sd), "m", cfg, ins["x"], m["l_max"])
    _check_vjp(fx, out, ins, sd)


@pytest.mark.parametrize("name", golden_names("product"))
def test_product(name):
    fx = load_golden(name)
    m = fx["meta"]
    ins, sd = _leaves(fx["in"]), _leaves(fx["sd"])
    cfg = dict(n_hidden_feats=m["in_features"], l_max_edge_attrs=m["in_l_max"], correlation=m["correlation"],
               path_reduced_product=m["path_reduced"], layer_norm=m["use_layer_norm"])
    out = OM.product(_prefixed(sd), "m", cfg, ins["x"], m["out_l_max"], atom_types=fx["in"]["atom_types"])
    _check_vjp(fx, out, ins, sd)


def test_readout():
    fx = load_golden("readout")
    m = fx["meta"]
    ins, sd = _leaves(fx["in"]), _leaves(fx["sd"])
    cfg = dict(n_hidden_feats=m["in_features"], hidden_readout=m["hidden_readout"])
    out = OM.readout(_prefixed(sd), "m", cfg, [ins[f"x{k}"] for k in range(m["n_layers"])])
    _check_vjp(fx, out, ins, sd)


def golden_graph(fx):
    """The fixture's graph as the dict that oracle.model.predict and AtomicGraph take."""
    g = {k: v for k, v in fx["in"].items()}
    g["use_shifts"] = bool(g["pbc"].any())
    return g


@pytest.mark.parametrize("form", ["einsum", "components"])
@pytest.mark.parametrize("name", golden_names("potential"))
def test_potential(name, form):
    """Site energies, energies, forces and stress of the whole potential (FlashCartPotential's
    wiring of the reference's layers, through the reference's AtomisticModel.predict)."""
    fx = load_golden(name)
    cfg = fx["meta"]["config"]
    stress = fx["meta"]["stress"]
    import contextlib

    with (O.components_form() if form == "components" else contextlib.nullcontext()):
        ref = OM.predict(fx["sd"], cfg, golden_graph(fx), compute_forces=True, compute_stress=stress)
    for key in ("node_energies", "energy", "forces") + (("stress",) if stress else ()):
        _close(ref[key], fx["out"][key], key)


@pytest.mark.parametrize("name", golden_names("potential"))
def test_initial_parameters(name):
    """torch.manual_seed(1234) + FlashCartPotential(**config) draws the reference's initial
    parameters under the reference's state-dict keys (construction order of
    src/flashcart/model/flashcart.py:151-221 and of every layer constructor)."""
    from flashcart_amd.model import FlashCartPotential

    fx = load_golden(name)
    torch.manual_seed(1234)
    model = FlashCartPotential(**fx["meta"]["config"])
    sd = model.state_dict()
    assert sorted(sd) == sorted(fx["init"]), set(sd) ^ set(fx["init"])
    for k, want in fx["init"].items():
        got = sd[k].detach().cpu()
        assert got.dtype == want.dtype, k
        assert torch.equal(got, want), k


def test_fullsize_fixture_matches_the_benchmark_workload():
    """tests/golden/fcc25k_step0.npz (the oracle at the benchmark's full size) belongs to the
    workload bench.py times: same first-step graph and same seed-1234 parameters."""
    from tests.golden.make_fullsize import graph_digest, params_digest, workload

    fx = load_golden("fcc25k_step0")
    g, model = workload()
    m = fx["meta"]
    assert (g.num_nodes, int(g.edge_index.shape[1])) == (m["n_atoms"], m["n_edges"])
    assert graph_digest(g) == m["graph_sha256"]
    assert params_digest(model) == m["params_sha256"]
    assert m["f32_vs_f64"]["energy_rel"] < 1e-5
