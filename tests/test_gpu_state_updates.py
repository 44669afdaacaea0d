"""Parameters, buffers and graph inputs changed between calls are seen by the next evaluation,
eager and replayed.

* Weights written through ``param.data.copy_`` (as EMA helpers swap weights), which no version
  counter records, and a new ``sqrt_avg_neighbors`` written the same way: the frozen model (edge
  pairs, species density) and its captured HIP graph must both follow them, compared with the
  float64 oracle of the new state (reference: in-place state writes of
  ``model/flashcart.py:325-340``; layer math ``nn/layers.py:351-369``).
* A replay called with the same edge_index tensor but new periodic shifts must redo the edge
  pairing (which reads the shifts) rather than keep the old pair slots.

Bars: energies 1e-5 relative, forces 1e-4 eV/A absolute.
"""

import pytest
import torch

from flashcart_amd.data import AtomicGraph
from flashcart_amd.data.synthetic import fcc_alloy, model_config
from flashcart_amd.nn import fused
from oracle import model as OM
from tests.helpers import assert_close

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _model(cfg, seed=1234):
    from flashcart_amd.model import FlashCartPotential
    torch.manual_seed(seed)
    m = FlashCartPotential.from_config(cfg)
    g = torch.Generator().manual_seed(seed + 1)
    with torch.no_grad():
        for name, p in m.named_parameters():
            if "output_linear" in name or "layer_norm.weights" in name:
                p.copy_(torch.randn(p.shape, generator=g) * 0.5 + (1.0 if "layer_norm" in name else 0.0))
    return m


def _system():
    numbers, pos, cell, pbc = fcc_alloy(2, 2, 2, seed=3)
    cfg = model_config(["Cu", "Ni", "Fe", "Cr"], 32, 3, avg_neighbors=42.0)
    graph = AtomicGraph.from_arrays(numbers, pos, cfg["elements"], 5.0, cell=cell, pbc=pbc)
    return cfg, graph


def _check(out, sd, mcfg, gdict, what):
    ref = OM.predict(sd, mcfg, gdict, compute_forces=True)
    assert_close(out["energy"], ref["energy"], 1e-5, 1e-6, f"{what} energy")
    assert_close(out["forces"], ref["forces"], 0.0, 1e-4, f"{what} forces")


def test_data_copy_weight_swap_eager_and_replay():
    cfg, graph = _system()
    model = _model(cfg)
    mcfg = model.to_model_config()
    m = model.to(DEV)
    m.requires_grad_(False)
    gd = graph.to(DEV)
    sd0 = {k: v.detach().cpu().clone() for k, v in m.state_dict().items()}
    print("state updates: first state, eager and replay", flush=True)
    fused.path_counts.clear()
    e0 = m.predict(gd, compute_forces=True)
    r0 = m.predict(gd, compute_forces=True, use_compile=True)
    assert fused.path_counts["species"] > 0 and fused.path_counts["paired"] > 0
    _check(e0, sd0, mcfg, graph.to_dict(), "state 0 eager")
    _check(r0, sd0, mcfg, graph.to_dict(), "state 0 replay")
    # a second state written through .data (no version counter records it)
    gen = torch.Generator().manual_seed(77)
    with torch.no_grad():
        for name, p in m.named_parameters():
            new = p.detach().cpu() * 1.1 + 0.05 * torch.randn(p.shape, generator=gen)
            p.data.copy_(new.to(DEV))
        for layer in m.interactions:
            layer.sqrt_avg_neighbors.data.copy_(layer.sqrt_avg_neighbors.data * 1.37)
    sd1 = {k: v.detach().cpu().clone() for k, v in m.state_dict().items()}
    print("state updates: second state, eager and replay", flush=True)
    e1 = m.predict(gd, compute_forces=True)
    r1 = m.predict(gd, compute_forces=True, use_compile=True)
    assert float((e1["energy"] - e0["energy"]).abs().max()) > 1e-3, "the new weights had no effect"
    _check(e1, sd1, mcfg, graph.to_dict(), "state 1 eager")
    _check(r1, sd1, mcfg, graph.to_dict(), "state 1 replay")


def test_replay_redoes_pairing_for_new_shifts():
    cfg, graph = _system()
    model = _model(cfg)
    sd, mcfg = model.state_dict(), model.to_model_config()
    m = model.to(DEV)
    m.requires_grad_(False)
    gd = graph.to(DEV).to_dict()
    print("state updates: replay with the original shifts", flush=True)
    r0 = m.predict(gd, compute_forces=True, use_compile=True)
    r0 = m.predict(gd, compute_forces=True, use_compile=True)
    _check(r0, sd, mcfg, graph.to_dict(), "original shifts")
    # the same edge_index tensor with new shifts: edge 5 moved by one cell (its reverse no longer
    # carries the negated shift, so the pairing breaks)
    new_shifts = gd["shifts"].clone()
    new_shifts[5, 0] += 1
    gd2 = dict(gd)
    gd2["shifts"] = new_shifts
    cpu2 = dict(graph.to_dict())
    cpu2["shifts"] = new_shifts.cpu()
    print("state updates: replay with new shifts, same edge_index tensor", flush=True)
    r1 = m.predict(gd2, compute_forces=True, use_compile=True)
    _check(r1, sd, mcfg, cpu2, "new shifts")
    assert float((r1["energy"] - r0["energy"]).abs().max()) > 0.0
    # back to the original shifts (a third tensor): the pairing holds again
    gd3 = dict(gd)
    gd3["shifts"] = gd["shifts"].clone()
    r2 = m.predict(gd3, compute_forces=True, use_compile=True)
    _check(r2, sd, mcfg, graph.to_dict(), "original shifts again")
