"""Shared test helpers: seeded synthetic graphs, comparison utilities, golden fixtures."""

import json
import os

import numpy as np
import torch


def random_csr_graph(n_nodes, degrees, seed=0, allow_self=False):
    """Receiver-sorted random edges: node i receives degrees[i % len(degrees)] edges."""
    rng = np.random.default_rng(seed)
    ii, jj = [], []
    for i in range(n_nodes):
        d = degrees[i % len(degrees)]
        for _ in range(d):
            j = int(rng.integers(0, n_nodes))
            if not allow_self and n_nodes > 1:
                while j == i:
                    j = int(rng.integers(0, n_nodes))
            ii.append(i)
            jj.append(j)
    return torch.tensor([ii, jj], dtype=torch.long)


def unit_vectors(n, seed=0, dtype=torch.float64):
    g = torch.Generator().manual_seed(seed)
    v = torch.randn(n, 3, generator=g, dtype=dtype)
    return v / v.norm(dim=-1, keepdim=True)


def assert_close(got, want, rtol, atol, what=""):
    got = got.detach().to("cpu", torch.float64)
    want = want.detach().to("cpu", torch.float64)
    assert got.shape == want.shape, f"{what}: shape {tuple(got.shape)} != {tuple(want.shape)}"
    err = (got - want).abs()
    tol = atol + rtol * want.abs()
    bad = err > tol
    if bad.any():
        k = int(torch.argmax((err - tol).reshape(-1)))
        raise AssertionError(f"{what}: {int(bad.sum())} / {err.numel()} elements off; worst at flat {k}: "
                             f"got {got.reshape(-1)[k]:.8g} want {want.reshape(-1)[k]:.8g} "
                             f"(max abs err {float(err.max()):.3e})")


GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def load_golden(name):
    """One fixture of tests/golden/ (written by tests/golden/make_fixtures.py from the reference's
    own modules): {"meta": dict, "sd": {...}, "in": {...}, "out": {...}, ...} of CPU tensors."""
    z = np.load(os.path.join(GOLDEN, f"{name}.npz"))
    out = {"meta": json.loads(str(z["meta"]))}
    for key in z.files:
        if key == "meta":
            continue
        group, sub = key.split("/", 1)
        out.setdefault(group, {})[sub] = torch.from_numpy(z[key].copy())
    return out


def golden_names(kind=None):
    names = sorted(f[:-4] for f in os.listdir(GOLDEN) if f.endswith(".npz"))
    if kind is None:
        return names
    return [n for n in names if json.loads(str(np.load(os.path.join(GOLDEN, n + ".npz"))["meta"]))["kind"] == kind]
