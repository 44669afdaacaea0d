"""End-to-end GPU parity of FlashCartPotential.predict against the CPU oracle.

The oracle evaluates the reference's forward in float64 from the same state dict;
the HIP path runs in float32. Bars (north star): energies within 1e-5 relative,
forces within 1e-4 eV/A absolute.
"""

import numpy as np
import pytest
import torch

from flashcart_amd.data import AtomicGraph, batch_graphs
from flashcart_amd.data.synthetic import fcc_alloy, model_config, molecules, water_box
from oracle import model as OM
from tests.helpers import assert_close

pytestmark = pytest.mark.gpu
DEV = "cuda"
E_REL = 1e-5
F_ABS = 1e-4


def _model(cfg, seed=1234):
    from flashcart_amd.model import FlashCartPotential
    torch.manual_seed(seed)
    m = FlashCartPotential.from_config(cfg)
    # random (non-identity) gate output maps and norm gains so every branch contributes
    g = torch.Generator().manual_seed(seed + 1)
    with torch.no_grad():
        for name, p in m.named_parameters():
            if "output_linear" in name or "layer_norm.weights" in name:
                p.copy_(torch.randn(p.shape, generator=g) * 0.5 + (1.0 if "layer_norm" in name else 0.0))
    return m


def _check(model, graph, cfg, frozen=False):
    """``frozen``: parameters without gradients, which routes the gated and product blocks
    through their fused inference backward (flashcart_amd/nn/fused.py)."""
    sd = model.state_dict()
    ref = OM.predict(sd, model.to_model_config(), graph.to_dict(), compute_forces=True)
    m = model.to(DEV)
    m.requires_grad_(not frozen)
    out = m.predict(graph.to(DEV), compute_forces=True)
    e_ref = ref["energy"]
    assert_close(out["energy"], e_ref, E_REL, 1e-6, "energy")
    assert_close(out["node_energies"], ref["node_energies"], 1e-5, 1e-5 * float(ref["node_energies"].abs().max()),
                 "node energies")
    assert_close(out["forces"], ref["forces"], 0.0, F_ABS, "forces")
    return out, ref


@pytest.mark.parametrize("frozen", [False, True])
def test_fcc_alloy_L3(frozen):
    numbers, pos, cell, pbc = fcc_alloy(2, 2, 2, seed=3)
    cfg = model_config(["Cu", "Ni", "Fe", "Cr"], 16, 3, avg_neighbors=42.0)
    g = AtomicGraph.from_arrays(numbers, pos, cfg["elements"], 5.0, cell=cell, pbc=pbc)
    _check(_model(cfg), g, cfg, frozen)


@pytest.mark.parametrize("frozen", [False, True])
def test_water_L2(frozen):
    numbers, pos, cell, pbc = water_box(16, seed=1)
    cfg = model_config(["H", "O"], 16, 2, avg_neighbors=20.0)
    g = AtomicGraph.from_arrays(numbers, pos, cfg["elements"], 5.0, cell=cell, pbc=pbc)
    _check(_model(cfg, seed=7), g, cfg, frozen)


@pytest.mark.parametrize("frozen", [False, True])
def test_molecule_batch_L2(frozen):
    mols = molecules(4, 5, 12, seed=2)
    cfg = model_config(["H", "C", "N", "O"], 8, 2, avg_neighbors=6.0)
    gs = [AtomicGraph.from_arrays(z, p, cfg["elements"], 5.0) for z, p in mols]
    out, ref = _check(_model(cfg, seed=5), batch_graphs(gs), cfg, frozen)
    assert out["energy"].shape[0] == 4


@pytest.mark.parametrize("frozen", [False, True])
def test_channels_128_L3(frozen):
    numbers, pos, cell, pbc = fcc_alloy(2, 2, 2, seed=4)
    cfg = model_config(["Cu", "Ni", "Fe", "Cr"], 128, 3, avg_neighbors=42.0)
    g = AtomicGraph.from_arrays(numbers, pos, cfg["elements"], 5.0, cell=cell, pbc=pbc)
    _check(_model(cfg, seed=11), g, cfg, frozen)


@pytest.mark.parametrize("frozen", [False, True])
def test_silu_gate_correlation2(frozen, monkeypatch):
    """SiLU gate (activation fused into the gate GEMM) and a two-step product; with frozen
    parameters both blocks must take the fused backward."""
    from flashcart_amd.nn import fused
    calls = {"product": 0, "gated": 0}
    real_p, real_g = fused.product_block, fused.gated_block

    def count(name, fn):
        def wrapped(*a):
            calls[name] += 1
            return fn(*a)
        return wrapped

    monkeypatch.setattr(fused, "product_block", count("product", real_p))
    monkeypatch.setattr(fused, "gated_block", count("gated", real_g))
    numbers, pos, cell, pbc = fcc_alloy(2, 2, 2, seed=6)
    cfg = model_config(["Cu", "Ni", "Fe", "Cr"], 16, 3, avg_neighbors=42.0)
    cfg.update(gate_activation="silu", correlation=2)
    g = AtomicGraph.from_arrays(numbers, pos, cfg["elements"], 5.0, cell=cell, pbc=pbc)
    _check(_model(cfg, seed=13), g, cfg, frozen)
    n_layers = cfg["n_interactions"]
    assert calls == ({"product": n_layers, "gated": n_layers} if frozen else {"product": 0, "gated": 0})


@pytest.mark.parametrize("frozen", [False, True])
def test_predict_replay(frozen):
    """predict(use_compile=True) captures the whole prediction as a HIP graph: replays with
    new positions (and eager work and synchronisations in between) must match the oracle on
    the same inputs (energies, forces and stress at the north-star bars) and the eager
    prediction. avg_neighbors changed between replays (set_avg_neighbors, and an in-place
    copy into the buffer as the reference's broadcast_pre_fit_state does) must reach the replay."""
    numbers, pos, cell, pbc = water_box(12, seed=4)
    cfg = model_config(["H", "O"], 16, 2, avg_neighbors=20.0)
    g = AtomicGraph.from_arrays(numbers, pos, cfg["elements"], 5.0, cell=cell, pbc=pbc).to(DEV)
    m = _model(cfg, seed=17).to(DEV)
    m.requires_grad_(not frozen)
    gen = torch.Generator(device="cpu").manual_seed(0)
    base = g.positions.clone()
    for it in range(6):
        g.positions = base + 0.02 * torch.randn(base.shape, generator=gen).to(DEV)
        if it == 2:  # a new edge-list tensor: the CSR graph replays
            g.edge_index = g.edge_index.clone()
        if it == 3:  # modified in place (same contents): replays as well
            g.edge_index.add_(0)
            m.interactions[0].set_avg_neighbors(12.5)
        if it == 5:
            with torch.no_grad():
                m.interactions[1].sqrt_avg_neighbors.copy_(torch.tensor(31.0 ** 0.5))
        got = m.predict(g, compute_forces=True, compute_stress=True, use_compile=True)
        junk = torch.randn(1000, 1000, device=DEV) @ torch.randn(1000, 1000, device=DEV)  # eager work between
        torch.cuda.synchronize()
        eager = m.predict(g, compute_forces=True, compute_stress=True)
        del junk
        for k in ("energy", "forces", "stress", "node_energies"):
            assert_close(got[k], eager[k].double(), 1e-6, 1e-6 * (float(eager[k].abs().max()) + 1.0),
                         f"replay {it} {k} vs eager")
        ref = OM.predict(m.state_dict(), m.to_model_config(), g.to("cpu").to_dict(), compute_forces=True,
                         compute_stress=True)
        assert_close(got["energy"], ref["energy"], E_REL, 1e-6, f"replay {it} energy vs oracle")
        assert_close(got["forces"], ref["forces"], 0.0, F_ABS, f"replay {it} forces vs oracle")
        assert_close(got["stress"], ref["stress"], 1e-5, 1e-5 * float(ref["stress"].abs().max()),
                     f"replay {it} stress vs oracle")
    # the kernels divide by each interaction's sqrt_avg_neighbors buffer on the device, so the new
    # values reach the captured graph without a re-capture
    assert len(m._replay_cache) == 1
