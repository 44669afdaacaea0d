"""The HIP path against the reference's own outputs (tests/golden/, written by the reference's
modules in float64; see tests/golden/make_fixtures.py).

Each op, layer and potential of flashcart_amd is loaded with the fixture's state dict, run in
float32 on the GPU, and compared with the reference's outputs and vector-Jacobian products.
Bars: ops and layers within 2e-5 of the largest reference magnitude (float32 against float64);
potentials at the north-star bars, energies 1e-5 relative and forces 1e-4 eV/A absolute.
"""

import pytest
import torch

from tests.helpers import assert_close, golden_names, load_golden

pytestmark = pytest.mark.gpu
DEV = "cuda"
REL = 2e-5


def _close(got, want, what, rel=REL):
    scale = max(float(want.abs().max()), 1e-30) if want.numel() else 1.0
    assert_close(got, want, rtol=rel, atol=rel * scale, what=what)


def _dev(d):
    return {k: (v.to(DEV, torch.float32).requires_grad_() if v.is_floating_point() else v.to(DEV))
            for k, v in d.items()}


def _vjp(fx, out, ins, module=None):
    _close(out, fx["out"]["out"], "out")
    names = list(fx.get("grad", {}))
    params = dict(module.named_parameters()) if module is not None else {}
    pnames = [k for k in fx.get("pgrad", {}) if k in params]
    assert len(pnames) == len(fx.get("pgrad", {})), set(fx.get("pgrad", {})) - set(pnames)
    leaves = [ins[k] for k in names] + [params[k] for k in pnames]
    grads = torch.autograd.grad(out, leaves, fx["cot"]["out"].to(DEV, torch.float32), allow_unused=True)
    for k, g, leaf in zip(names + pnames, grads, leaves):
        want = fx["grad"][k] if k in fx["grad"] else fx["pgrad"][k]
        _close(torch.zeros_like(leaf) if g is None else g, want, f"d/d{k}")


def _load(module, fx):
    sd = {k: v.to(torch.float32) if v.is_floating_point() else v for k, v in fx["sd"].items()}
    missing, unexpected = module.load_state_dict(sd, strict=False)
    assert not unexpected, unexpected
    return module.to(DEV)


@pytest.mark.parametrize("name", golden_names("tp"))
def test_tensor_product(name):
    from flashcart_amd import o3

    fx = load_golden(name)
    m = fx["meta"]
    tp = o3.TensorProduct(m["in1_l_max"], m["in2_l_max"], m["out_l_max"], m["in1_features"], m["in2_features"],
                          symmetric_product=m["symmetric_product"], shared_weights=m["shared_weights"],
                          reduce_paths=m["reduce_paths"])
    assert list(tp.out_paths) == m["out_paths"] and tp.n_total_paths == m["n_total_paths"]
    ins = _dev(fx["in"])
    ei = ins.get("edge_index")
    in2 = ins["in1"] if m["symmetric_product"] else ins["in2"]
    out = tp(ins["in1"], in2, ins["weights"], ei[0] if ei is not None else None, ei[1] if ei is not None else None)
    _vjp(fx, out, ins)


@pytest.mark.parametrize("name", golden_names("linear"))
def test_linear(name):
    from flashcart_amd import o3

    fx = load_golden(name)
    m = fx["meta"]
    lay = _load(o3.LinearLayer(m["in_l_max"], m["out_l_max"], m["in_features"], m["out_features"],
                               in_paths=m["in_paths"]), fx)
    ins = _dev(fx["in"])
    _vjp(fx, lay(ins["x"]), ins, lay)


@pytest.mark.parametrize("name", golden_names("interaction"))
def test_interaction(name):
    from flashcart_amd.nn import InteractionLayer

    fx = load_golden(name)
    m = fx["meta"]
    lay = _load(InteractionLayer(m["in1_l_max"], m["in2_l_max"], m["out_l_max"], m["in1_features"],
                                 m["out_features"], m["n_radial"], hidden_radial=m["hidden_radial"],
                                 n_elements=m["n_elements"], element_features=m["element_features"],
                                 avg_neighbors=m["avg_neighbors"], use_sc=m["use_sc"],
                                 use_layer_norm=m["use_layer_norm"]), fx)
    ins = _dev(fx["in"])
    out = lay(ins["node_feats"], ins["edge_attrs"], ins["edge_feats"], ins["edge_index"], ins["envelope"],
              atom_types=ins["atom_types"] if m["n_elements"] else None)
    _vjp(fx, out, ins, lay)


@pytest.mark.parametrize("name", golden_names("rms_norm"))
def test_rms_norm(name):
    from flashcart_amd.nn import RMSLayerNorm

    fx = load_golden(name)
    m = fx["meta"]
    lay = _load(RMSLayerNorm(m["l_max"], m["n_features"], eps=m["eps"]), fx)
    ins = _dev(fx["in"])
    _vjp(fx, lay(ins["x"]), ins, lay)


@pytest.mark.parametrize("name", golden_names("gated"))
def test_gated(name):
    from flashcart_amd.nn import EquivariantGatedLayer

    fx = load_golden(name)
    m = fx["meta"]
    lay = _load(EquivariantGatedLayer(m["l_max"], m["in_features"], m["in_features"],
                                      gate_activation=m["gate_activation"], gate_bias=m["gate_bias"]), fx)
    ins = _dev(fx["in"])
    _vjp(fx, lay(ins["x"]), ins, lay)


@pytest.mark.parametrize("name", golden_names("product"))
def test_product(name):
    from flashcart_amd.nn import ProductLayer

    fx = load_golden(name)
    m = fx["meta"]
    lay = _load(ProductLayer(m["in_l_max"], m["out_l_max"], m["in_features"], n_elements=m["n_elements"],
                             correlation=m["correlation"], path_reduced=m["path_reduced"], use_sc=m["use_sc"],
                             use_layer_norm=m["use_layer_norm"]), fx)
    ins = _dev(fx["in"])
    _vjp(fx, lay(ins["x"], ins["atom_types"] if m["n_elements"] else None), ins, lay)


def test_readout():
    from flashcart_amd.nn import EnergyReadoutLayer

    fx = load_golden("readout")
    m = fx["meta"]
    lay = _load(EnergyReadoutLayer(m["in_features"], m["n_layers"], hidden_readout=m["hidden_readout"]), fx)
    ins = _dev(fx["in"])
    _vjp(fx, lay([ins[f"x{k}"] for k in range(m["n_layers"])]), ins, lay)


def _golden_graph(fx):
    from flashcart_amd.data import AtomicGraph

    g = fx["in"]
    return AtomicGraph(positions=g["positions"].float(), cell=g["cell"].float(), pbc=g["pbc"], shifts=g["shifts"],
                       edge_index=g["edge_index"], atom_types=g["atom_types"], n_atoms=g["n_atoms"],
                       batch=g["batch"], use_shifts=bool(g["pbc"].any()))


@pytest.mark.parametrize("frozen", [False, True])
@pytest.mark.parametrize("name", golden_names("potential"))
def test_potential(name, frozen):
    """Energies, site energies, forces and stress of the whole HIP potential against the
    reference's AtomisticModel.predict (``frozen``: parameters without gradients, the fused
    inference backward)."""
    from flashcart_amd.model import FlashCartPotential

    fx = load_golden(name)
    model = _load(FlashCartPotential(**fx["meta"]["config"]), fx)
    model.requires_grad_(not frozen)
    stress = fx["meta"]["stress"]
    out = model.predict(_golden_graph(fx).to(DEV), compute_forces=True, compute_stress=stress)
    ref = fx["out"]
    assert_close(out["energy"], ref["energy"], 1e-5, 1e-6, "energy")
    _close(out["node_energies"], ref["node_energies"], "node energies", rel=1e-5)
    assert_close(out["forces"], ref["forces"], 0.0, 1e-4, "forces")
    if stress:
        _close(out["stress"], ref["stress"], "stress", rel=1e-5)
