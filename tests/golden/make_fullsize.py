"""Writes tests/golden/fcc25k_step0.npz: the oracle's energies and forces for the benchmark's
first step at full size.

Workload (flashcart_amd.data.synthetic, the definition bench.py times): 25x25x10 fcc cells =
25,000 atoms, a = 3.6 A, jitter 0.05 A, first MD-style step (N(0, 0.01^2) A, rng seed 1), the
host neighbour list within r_max = 5 A; the default architecture at C = 128, L_max = 3 from
torch.manual_seed(1234), avg_neighbors = E / N of this graph.

The oracle runs on CPU with the radial MLP and convolution evaluated per range of 1,024 receivers
(oracle.model.interaction(chunk=...)), once in float32 (the reference's working precision, and
the same float32 positions and edge-vector arithmetic as the GPU path) and once in float64. The
fixture holds both, plus hashes of the graph and the parameters so that the GPU test can check
that it evaluates the same inputs. Usage: python tests/golden/make_fullsize.py (a few minutes).
"""

from __future__ import annotations

import hashlib
import json
import os
import sys
import time

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)

from flashcart_amd.data.synthetic import FCC25K_ELEMENTS, StepGraphs, fcc25k_model, fcc25k_system  # noqa: E402
from oracle import model as OM  # noqa: E402

CHUNK = 1024


def digest(*arrays) -> str:
    h = hashlib.sha256()
    for a in arrays:
        a = a.detach().cpu().contiguous() if torch.is_tensor(a) else torch.as_tensor(np.ascontiguousarray(a))
        h.update(str(a.dtype).encode() + str(tuple(a.shape)).encode())
        h.update(a.numpy().tobytes())
    return h.hexdigest()


def workload():
    """The first benchmark step graph (CPU) and its model (float32, frozen parameters)."""
    numbers, pos, cell, pbc = fcc25k_system()
    g = StepGraphs(numbers, pos, cell, pbc, list(FCC25K_ELEMENTS), 1).graph(0)
    model, cfg = fcc25k_model(g.edge_index.shape[1] / len(numbers))
    return g, model


def graph_digest(g) -> str:
    return digest(g.positions, g.cell, g.shifts, g.edge_index, g.atom_types)


def params_digest(model) -> str:
    sd = model.state_dict()
    return digest(*[sd[k] for k in sorted(sd)])


def main():
    torch.set_num_threads(min(8, os.cpu_count() or 1))
    g, model = workload()
    sd = {k: v.detach().cpu() for k, v in model.state_dict().items()}
    mcfg = model.to_model_config()
    gd = g.to_dict()
    n, E = g.num_nodes, int(g.edge_index.shape[1])
    print(f"N={n} E={E} avg={E / n:.4f}", flush=True)
    res = {}
    for dtype in (torch.float32, torch.float64):
        t0 = time.time()
        out = OM.predict(sd, mcfg, gd, compute_forces=True, dtype=dtype, chunk=CHUNK)
        res[dtype] = out
        print(f"{dtype}: E={float(out['energy'][0]):.10f} |F|max={float(out['forces'].abs().max()):.6f} "
              f"({time.time() - t0:.0f} s)", flush=True)
    f32, f64 = res[torch.float32], res[torch.float64]
    meta = dict(kind="fullsize", n_atoms=n, n_edges=E, avg_neighbors=E / n, chunk=CHUNK,
                graph_sha256=graph_digest(g), params_sha256=params_digest(model),
                f32_vs_f64=dict(energy_rel=float(abs(f32["energy"].double() - f64["energy"]).max() / abs(f64["energy"]).max()),
                                forces_abs=float((f32["forces"].double() - f64["forces"]).abs().max()),
                                node_energies_abs=float((f32["node_energies"].double() - f64["node_energies"]).abs().max())))
    print(json.dumps(meta["f32_vs_f64"]), flush=True)
    arrays = {"meta": np.array(json.dumps(meta, sort_keys=True)),
              "out/energy_f32": f32["energy"].double().numpy(), "out/energy_f64": f64["energy"].numpy(),
              "out/node_energies_f32": f32["node_energies"].float().numpy(),
              "out/node_energies_f64": f64["node_energies"].numpy(),
              "out/forces_f32": f32["forces"].float().numpy(), "out/forces_f64": f64["forces"].numpy()}
    path = os.path.join(HERE, "fcc25k_step0.npz")
    np.savez_compressed(path, **arrays)
    print(f"wrote {path} ({os.path.getsize(path) / 1024:.0f} KiB)")


if __name__ == "__main__":
    main()
