"""Oracle: functional CPU restatement of the FlashCart potential (energies and forces).

TEST INFRASTRUCTURE ONLY (checker and CPU baseline); never imported by flashcart_amd.

Evaluates the potential from a state dict (the parameter names of the reference's
module tree) and the model config, following the reference forward:
  FlashCartPotential.forward      src/flashcart/model/flashcart.py:223-317 (wiring :151-221)
  InteractionLayer.forward        src/flashcart/nn/layers.py:310-379
  RMSLayerNorm.forward            src/flashcart/nn/layers.py:494-528
  EquivariantGatedLayer.forward   src/flashcart/nn/layers.py:609-635
  ProductLayer.forward            src/flashcart/nn/layers.py:949-995
  EnergyReadoutLayer / ScaleShift src/flashcart/nn/layers.py:1045-1063, :1097-1108
  AtomisticModel._predict_impl    src/flashcart/model/atomistic.py:276-340
Forces are -dE/dpositions through torch autograd on CPU, as the reference's CPU path.
"""

from __future__ import annotations

from typing import Any, Dict, List, Optional

import torch

from oracle import ops as O
from oracle.cartesian import enumerate_paths


def _paths(l1, l2, lo, sym=False):
    ps = enumerate_paths(l1, l2, lo, sym)
    counts = [0] * (lo + 1)
    for p in ps:
        counts[p[2]] += 1
    return counts, len(ps)


def _o3_linear(sd, prefix, x, in_l_max, out_l_max, fin, fout, in_paths=None):
    n = min(in_l_max, out_l_max) + 1
    ws = [sd[f"{prefix}.weight.{l}"] for l in range(n)]
    return O.linear(x, ws, in_l_max, out_l_max, fin, fout, in_paths)


def _mlp(sd, prefix, x, n_layers):
    for k in range(n_layers):
        w = sd[f"{prefix}.{2 * k}.weight"]
        b = sd.get(f"{prefix}.{2 * k}.bias")
        x = O.dense(x, w, b)
        if k < n_layers - 1:
            x = O.silu(x)
    return x


def rms_norm(sd, prefix, x, l_max, C, eps=1e-6):
    n = x.shape[0]
    _, P = _paths(l_max, l_max, 0, True)
    inv = O.tensor_product(x, x, torch.ones(P * C, dtype=x.dtype), None, None, l_max, l_max, 0, C, C,
                           symmetric_product=True, shared_weights=True).view(n, l_max + 1, C)
    lw = torch.tensor([1.0 / ((2 * l + 1) * (l_max + 1)) for l in range(l_max + 1)], dtype=torch.float64)
    mean_sq = (inv * lw.to(inv.dtype).view(1, -1, 1)).sum(dim=1).mean(dim=-1, keepdim=True)
    scaled = x * torch.pow(mean_sq + eps, -0.5)
    g = torch.cat([sd[f"{prefix}.weights.{l}"].repeat(2 * l + 1) for l in range(l_max + 1)]).view(1, -1)
    return scaled * g


def _conv_chunked(sd, prefix, cfg, h, edge_attrs, mlp_in, idx_i, idx_j, lin, L, lout, C, chunk):
    """Radial MLP + convolution TP over ranges of ``chunk`` receivers (edges sorted by receiver),
    each under torch.utils.checkpoint: same sums as the one-shot form, but the per-edge weights
    and path outputs of one range at a time (recomputed for the backward)."""
    from torch.utils.checkpoint import checkpoint

    rows = h.shape[0]
    n_mlp = len(cfg.get("hidden_radial", [64, 64])) + 1
    bounds = torch.searchsorted(idx_i, torch.arange(0, rows + chunk, chunk).clamp_max(rows)).tolist()

    def part(h_, attrs_c, mlp_c, ii, jj, n_out):
        w = _mlp(sd, f"{prefix}.radial_mlp", mlp_c, n_mlp)
        return O.tensor_product(h_, attrs_c, w, ii, jj, lin, L, lout, C, 1, out_rows=n_out)

    outs = []
    for k, a in enumerate(range(0, rows, chunk)):
        e0, e1 = bounds[k], bounds[k + 1]
        n_out = min(rows, a + chunk) - a
        outs.append(checkpoint(part, h, edge_attrs[e0:e1], mlp_in[e0:e1], idx_i[e0:e1] - a, idx_j[e0:e1], n_out,
                               use_reentrant=False))
    return torch.cat(outs, dim=0)


def interaction(sd, prefix, cfg, lin, lout, node_feats, edge_attrs, edge_feats, envelope, edge_index,
                atom_types=None, chunk=None):
    """InteractionLayer.forward (src/flashcart/nn/layers.py:310-379): linear_first, radial MLP on the
    envelope-scaled radial features (with the sender/receiver element embeddings appended when the
    layer is element-conditioned, :346-350), conv TP, / sqrt(avg_neighbors), linear_second, skip
    projection (rank-0 slice add when lin == 0, :370-375), RMS norm. ``chunk``: evaluate the radial
    MLP and the convolution per range of that many receivers (large graphs)."""
    C = cfg["n_hidden_feats"]
    L = cfg["l_max_edge_attrs"]
    out_paths, P = _paths(lin, L, lout)
    residual = node_feats
    idx_i, idx_j = edge_index[0], edge_index[1]
    if f"{prefix}.emb_i.weight" in sd:
        if atom_types is None:
            raise ValueError("atom_types required for an element-conditioned interaction")
        emb_i = sd[f"{prefix}.emb_i.weight"][atom_types][idx_i]
        emb_j = sd[f"{prefix}.emb_j.weight"][atom_types][idx_j]
        mlp_in = torch.cat([edge_feats, emb_i, emb_j], dim=-1) * envelope.unsqueeze(-1)
    else:
        mlp_in = edge_feats * envelope.unsqueeze(-1)
    h = _o3_linear(sd, f"{prefix}.linear_first", node_feats, lin, lin, C, C)
    if chunk:
        agg = _conv_chunked(sd, prefix, cfg, h, edge_attrs, mlp_in, idx_i, idx_j, lin, L, lout, C, chunk)
    else:
        w = _mlp(sd, f"{prefix}.radial_mlp", mlp_in, len(cfg.get("hidden_radial", [64, 64])) + 1)
        agg = O.tensor_product(h, edge_attrs, w, idx_i, idx_j, lin, L, lout, C, 1)
    agg = agg / sd[f"{prefix}.sqrt_avg_neighbors"].to(agg.dtype)
    out = _o3_linear(sd, f"{prefix}.linear_second", agg, lout, lout, C, C, out_paths)
    if lin == 0:
        skip = O.dense(residual, sd[f"{prefix}.skip_projection.weight"])
        out = torch.cat([out[:, :C] + skip, out[:, C:]], dim=-1)
    else:
        out = out + _o3_linear(sd, f"{prefix}.skip_projection", residual, lin, lout, C, C)
    if cfg.get("layer_norm", False):
        out = rms_norm(sd, f"{prefix}.layer_norm", out, lout, C)
    return out


def gated(sd, prefix, cfg, x, l_max):
    C = cfg["n_hidden_feats"]
    n = x.shape[0]
    values = _o3_linear(sd, f"{prefix}.value_linear", x, l_max, l_max, C, C)
    pre = O.dense(x[:, :C], sd[f"{prefix}.gate_linear.weight"], sd.get(f"{prefix}.gate_linear.bias"))
    if cfg.get("gate_activation", "silu") == "silu":
        gates = O.silu(pre)
    else:
        gates = O.stored(O.SIGMOID_SCALE) * torch.sigmoid(pre)
    gates = gates.view(n, l_max + 1, C)
    blocks, off = [], 0
    for l in range(l_max + 1):
        b = values[:, off:off + (2 * l + 1) * C].view(n, 2 * l + 1, C)
        blocks.append((b * gates[:, l].unsqueeze(1)).flatten(1))
        off += (2 * l + 1) * C
    return x + _o3_linear(sd, f"{prefix}.output_linear", torch.cat(blocks, dim=-1), l_max, l_max, C, C)


def product(sd, prefix, cfg, x, out_l_max, atom_types=None):
    """ProductLayer.forward (src/flashcart/nn/layers.py:949-995): B_0 = x (times the rank-expanded
    step-0 path weights when those are learnable, :960-963), B_k = TP(B_{k-1}, x, 1 + delta_k),
    per-step product linear (or path norm), sum of the selected ranks, final linear (reduced),
    skip projection, RMS norm. Element-dependent deltas (ProductPathWeights, :703-766) are rows of
    an embedding indexed by the atom type, so the products then take per-row weights."""
    C = cfg["n_hidden_feats"]
    L = cfg["l_max_edge_attrs"]
    corr = cfg.get("correlation", 3)
    reduced = cfg.get("path_reduced_product", True)
    out_dim = (out_l_max + 1) ** 2 * C
    output = x.new_zeros(x.shape[0], out_dim)
    feats = x
    for k in range(corr):
        p_out = out_l_max if k == corr - 1 else L
        l2, f2 = (0, 1) if k == 0 else (L, C)
        out_paths, P = _paths(L, l2, p_out)
        table = sd.get(f"{prefix}.path_weights.{k}.delta.weight")
        per_row = table is not None
        if per_row:
            if atom_types is None:
                raise ValueError("atom_types required for element-dependent product weights")
            w = 1.0 + table[atom_types]
        else:
            delta = sd.get(f"{prefix}.path_weights.{k}.delta")
            w = 1.0 + (delta if delta is not None else torch.zeros(P * C, dtype=x.dtype))
        if k == 0:
            if reduced or per_row:
                idx = torch.cat([torch.arange(l * C, (l + 1) * C).repeat(2 * l + 1) for l in range(L + 1)])
                feats = x * w[..., idx]
            else:
                feats = x
        else:
            feats = O.tensor_product(feats, x, w, None, None, L, L, p_out, C, C, shared_weights=not per_row,
                                     reduce_paths=reduced)
        if reduced:
            norm = torch.cat([torch.full(((2 * l + 1) * C,), out_paths[l] ** -0.5) for l in range(p_out + 1)])
            if not torch.all(norm == 1.0):
                feats = feats * norm.to(feats.dtype)
        else:
            feats = _o3_linear(sd, f"{prefix}.product_linears.{k}", feats, p_out,
                               p_out if k < corr - 1 else out_l_max, C, C, out_paths)
        output = output + feats[:, :out_dim]
    if reduced:
        output = _o3_linear(sd, f"{prefix}.final_linear", output, out_l_max, out_l_max, C, C)
    output = output + _o3_linear(sd, f"{prefix}.skip_projection", x, L, out_l_max, C, C)
    if cfg.get("layer_norm", False):
        output = rms_norm(sd, f"{prefix}.layer_norm", output, out_l_max, C)
    return output


def readout(sd, prefix, cfg, outs):
    """EnergyReadoutLayer.forward (src/flashcart/nn/layers.py:1045-1063): MLP on the concatenated
    first C columns of every layer's output."""
    C = cfg["n_hidden_feats"]
    x = torch.cat([o[:, :C] for o in outs], dim=1)
    return _mlp(sd, f"{prefix}.readout_mlp", x, len(cfg.get("hidden_readout", [64, 64])) + 1).squeeze(-1)


def node_energies(sd: Dict[str, torch.Tensor], cfg: Dict[str, Any], graph: Dict[str, Any],
                  chunk: Optional[int] = None) -> torch.Tensor:
    """FlashCartPotential.forward (src/flashcart/model/flashcart.py:249-317; ranks of each layer
    from :155-162): interaction in ranks [0, Lh, ...], interaction out L (or the product out ranks
    when correlation is 1), gate at the interaction's out rank, product out [Lh, ..., 0], readout on
    the first C columns of every layer, per-element scale."""
    C = cfg["n_hidden_feats"]
    L = cfg["l_max_edge_attrs"]
    Lh = cfg["l_max_hidden_feats"]
    n_int = cfg["n_interactions"]
    ei = graph["edge_index"]
    types = graph["atom_types"]
    vec = graph.get("vectors")
    if vec is None:
        vec = O.edge_vectors(graph["positions"], graph["cell"], graph["shifts"], ei, graph["batch"],
                             graph.get("use_shifts", True))
    d = vec.norm(dim=-1)
    r = vec / d.clamp_min(O.MIN_EDGE_LENGTH).unsqueeze(-1)
    attrs = O.irreps(r, L)
    feats = O.chebyshev(d, cfg.get("n_radial", 8), cfg["r_max"], cfg.get("r_min", 0.0),
                        cfg.get("radial_mapping", "affine"))
    env = O.cutoff(d, cfg["r_max"], cfg.get("cutoff_poly_order", 6))
    x = sd["embedding.weight"][types]
    use_products = cfg.get("correlation", 3) > 1
    prod_out = [Lh if k < n_int - 1 else 0 for k in range(n_int)]
    int_out = [L] * n_int if use_products else prod_out
    outs = []
    for k in range(n_int):
        y = interaction(sd, f"interactions.{k}", cfg, 0 if k == 0 else Lh, int_out[k], x, attrs, feats, env, ei,
                        atom_types=types, chunk=chunk)
        if cfg.get("nonlinearity", False):
            y = gated(sd, f"nonlinearities.{k}", cfg, y, int_out[k])
        if use_products:
            x = product(sd, f"products.{k}", cfg, y, prod_out[k], atom_types=types)
        else:
            x = y
        outs.append(x[:, :C])
    e = readout(sd, "readout", cfg, outs)
    return sd["scale_shift.scales"][types] * e


def predict(sd: Dict[str, torch.Tensor], cfg: Dict[str, Any], graph: Dict[str, Any], compute_forces: bool = True,
            dtype: torch.dtype = torch.float64, compute_stress: bool = False,
            chunk: Optional[int] = None) -> Dict[str, torch.Tensor]:
    """Energies (per structure and per atom), forces and optionally stress, on CPU in ``dtype``.

    Stress follows src/flashcart/model/atomistic.py:200-210,290-302: positions and cell
    are multiplied by (I + sym(D)) for a zero displacement D, and
    stress = dE/dD / det(cell) in Voigt order xx, yy, zz, yz, xz, xy.
    """
    sd = {k: v.detach().to("cpu", dtype) if v.is_floating_point() else v.detach().cpu() for k, v in sd.items()}
    g = {k: (v.detach().cpu() if torch.is_tensor(v) else v) for k, v in graph.items()}
    pos = g["positions"].to(dtype).requires_grad_(compute_forces)
    cell = g["cell"].to(dtype)
    inputs = [pos] if compute_forces else []
    if compute_stress:
        disp = torch.zeros_like(cell).requires_grad_(True)
        scaling = torch.eye(3, dtype=dtype) + 0.5 * (disp + disp.transpose(-1, -2))
        g["positions"] = (pos.unsqueeze(-2) @ scaling[g["batch"]]).squeeze(-2)
        g["cell"] = cell @ scaling
        inputs.append(disp)
    else:
        g["positions"] = pos
        g["cell"] = cell
    e_node = node_energies(sd, cfg, g, chunk=chunk)
    n_graphs = int(g["n_atoms"].shape[0])
    energy = O.scatter_sum(e_node, g["batch"], n_graphs)
    out = {"node_energies": e_node.detach(), "energy": energy.detach()}
    if inputs:
        grads = torch.autograd.grad(energy.sum(), inputs)
        if compute_forces:
            out["forces"] = -grads[0]
        if compute_stress:
            s = grads[-1] / torch.det(cell).view(-1, 1, 1)
            out["stress"] = torch.stack([s[:, 0, 0], s[:, 1, 1], s[:, 2, 2], (s[:, 1, 2] + s[:, 2, 1]) / 2,
                                         (s[:, 0, 2] + s[:, 2, 0]) / 2, (s[:, 0, 1] + s[:, 1, 0]) / 2], dim=-1)
    return out


def force_loss_grads(sd: Dict[str, torch.Tensor], cfg: Dict[str, Any], graph: Dict[str, Any],
                     energy_ref: torch.Tensor, forces_ref: torch.Tensor, names: List[str],
                     w_energy: float = 1.0, w_forces: float = 1.0,
                     dtype: torch.dtype = torch.float64) -> Dict[str, torch.Tensor]:
    """Gradients of the force-matching loss
        w_e * mean((E - E_ref)^2) + w_f * mean((F - F_ref)^2),  F = -dE/dR (create_graph=True)
    with respect to the parameters ``names`` of the state dict, in ``dtype`` on CPU.

    The second derivatives come from torch autograd over the oracle's forward, as in the
    reference's training step (src/flashcart/model/atomistic.py:276-340 with
    create_graph=True; src/flashcart/training/loss.py:127-305). Returns the loss under
    "loss" and one gradient per name.
    """
    params = {k: v.detach().to("cpu", dtype) if v.is_floating_point() else v.detach().cpu() for k, v in sd.items()}
    for k in names:
        params[k].requires_grad_(True)
    g = {k: (v.detach().cpu() if torch.is_tensor(v) else v) for k, v in graph.items()}
    pos = g["positions"].to(dtype).requires_grad_(True)
    g["positions"] = pos
    g["cell"] = g["cell"].to(dtype)
    e_node = node_energies(params, cfg, g)
    energy = O.scatter_sum(e_node, g["batch"], int(g["n_atoms"].shape[0]))
    (de,) = torch.autograd.grad(energy.sum(), pos, create_graph=True)
    forces = -de
    loss = w_energy * ((energy - energy_ref.to(dtype)) ** 2).mean() + \
        w_forces * ((forces - forces_ref.to(dtype)) ** 2).mean()
    grads = torch.autograd.grad(loss, [params[k] for k in names], allow_unused=True)
    out = {k: (gr if gr is not None else torch.zeros_like(params[k])) for k, gr in zip(names, grads)}
    out["loss"] = loss.detach()
    return out
