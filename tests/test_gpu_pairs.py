"""Edge pairs (i <- j, S) / (j <- i, -S) and the radial weights shared within a pair.

``fc_edge_pairs`` is index work, checked bit for bit against a plain restatement here. The
premise of sharing (both edges of a pair have bitwise the same radial-MLP input) is checked on
the device geometry itself; the tensor product with ``pair_slot`` is checked bit for bit
against the same product with the weights expanded per edge; the potential with pairs against
the float64 oracle at the north-star bars, and against its own unpaired evaluation.
"""

import numpy as np
import pytest
import torch

from flashcart_amd.data import AtomicGraph, batch_graphs
from flashcart_amd.data.synthetic import fcc_alloy, model_config, molecules, water_box
from oracle import model as OM
from tests.helpers import assert_close, random_csr_graph
from flashcart_amd.nn import fused

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _np_pairs(ii, jj, shifts):
    """Restatement of fc_edge_pairs on receiver rows sorted by strictly increasing (sender, shift):
    the reverse of edge e is the edge of receiver jj[e] with sender ii[e] and shift -S; pairs are
    mutual reverses, numbered by their lower edge. An edge whose (sender, shift) does not exceed
    its predecessor's in the row has no reverse."""
    ii, jj = np.asarray(ii), np.asarray(jj)
    n_edges = ii.shape[0]
    s = np.zeros((n_edges, 3), np.int64) if shifts is None else np.asarray(shifts, np.int64)
    starts = {}
    for e in range(n_edges):
        starts.setdefault(int(ii[e]), []).append(e)
    rev = np.full(n_edges, -1, np.int64)
    for e in range(n_edges):
        if e > 0 and ii[e - 1] == ii[e] and (int(jj[e - 1]), *s[e - 1]) >= (int(jj[e]), *s[e]):
            rev[e] = -2
            continue
        for k in starts.get(int(jj[e]), []):
            if k != e and jj[k] == ii[e] and (s[k] == -s[e]).all():
                rev[e] = k
                break
    slot = np.full(n_edges, -1, np.int64)
    edge = []
    bad = 0
    for e in range(n_edges):
        r = rev[e]
        if r < 0 or rev[r] != e:
            bad += 1
            continue
        if r > e:
            p = len(edge)
            edge.append(e)
            slot[e], slot[r] = 2 * p, 2 * p + 1
    return slot, np.asarray(edge, np.int64), bad


def _graphs():
    numbers, pos, cell, pbc = fcc_alloy(2, 2, 2, seed=3)  # 7.2 A box, r_max 5: several images per pair
    yield "fcc_small_cell", AtomicGraph.from_arrays(numbers, pos, ["Cu", "Ni", "Fe", "Cr"], 5.0, cell=cell, pbc=pbc)
    numbers, pos, cell, pbc = water_box(64, seed=1)
    yield "water", AtomicGraph.from_arrays(numbers, pos, ["H", "O"], 5.0, cell=cell, pbc=pbc)
    mols = molecules(6, seed=2)
    yield "molecules", batch_graphs([AtomicGraph.from_arrays(z, p, ["H", "C", "N", "O"], 5.0) for z, p in mols])


def _csr(g):
    from flashcart_amd.o3._graph import build_graph
    return build_graph(g.edge_index.to(DEV), int(g.atom_types.shape[0]))


@pytest.mark.parametrize("name,graph", list(_graphs()), ids=lambda v: v if isinstance(v, str) else "")
def test_pairs_match_restatement(name, graph):
    from flashcart_amd.o3._graph import launch_edge_pairs
    csr = _csr(graph)
    use_shifts = bool(graph.to_dict().get("use_shifts", True))
    shifts = graph.shifts.to(DEV) if use_shifts else None
    print(f"pairs: {name}, {csr.n_edges} edges", flush=True)
    pairs, counts = launch_edge_pairs(csr, shifts)
    slot, edge, bad = _np_pairs(graph.edge_index[0].numpy(), graph.edge_index[1].numpy(),
                                graph.shifts.numpy() if use_shifts else None)
    assert bad == 0 and 2 * len(edge) == csr.n_edges
    assert counts.tolist() == [0, len(edge)]
    assert np.array_equal(pairs.slot.cpu().numpy(), slot)
    assert np.array_equal(pairs.edge.cpu().numpy(), edge)
    assert csr.edge_pairs(shifts) is not None


def test_incomplete_pairings_are_refused():
    from flashcart_amd.o3._graph import build_graph, find_edge_pairs, launch_edge_pairs
    # random directed edges in unsorted rows: refused
    ei = random_csr_graph(40, [3, 5, 0, 8], seed=4)
    csr = build_graph(ei.to(DEV), 40)
    pairs, counts = launch_edge_pairs(csr, None)
    assert counts.tolist()[0] > 0
    assert find_edge_pairs(csr, None) is None
    # the same edges with every row sorted: most still have no reverse
    order = torch.argsort(ei[0] * 1000 + ei[1], stable=True)
    ei = ei[:, order]
    keep = torch.ones(ei.shape[1], dtype=torch.bool)
    keep[1:] = (ei[:, 1:] != ei[:, :-1]).any(0)  # drop duplicate edges
    ei = ei[:, keep]
    csr = build_graph(ei.to(DEV), 40)
    pairs, counts = launch_edge_pairs(csr, None)
    slot, edge, bad = _np_pairs(ei[0].numpy(), ei[1].numpy(), None)
    assert counts.tolist() == [bad, len(edge)] and bad > 0
    assert np.array_equal(pairs.slot.cpu().numpy(), slot)
    assert find_edge_pairs(csr, None) is None
    # a symmetric list with one row out of order: refused
    numbers, pos, cell, pbc = fcc_alloy(2, 2, 2, seed=3)
    g = AtomicGraph.from_arrays(numbers, pos, ["Cu", "Ni", "Fe", "Cr"], 5.0, cell=cell, pbc=pbc)
    ei, sh = g.edge_index.clone(), g.shifts.clone()
    ei[:, [3, 4]] = ei[:, [4, 3]]
    sh[[3, 4]] = sh[[4, 3]]
    assert int(ei[0, 3]) == int(ei[0, 4])
    assert find_edge_pairs(build_graph(ei.to(DEV), int(g.atom_types.shape[0])), sh.to(DEV)) is None
    # a symmetric list with one pair's shift broken
    numbers, pos, cell, pbc = fcc_alloy(2, 2, 2, seed=3)
    g = AtomicGraph.from_arrays(numbers, pos, ["Cu", "Ni", "Fe", "Cr"], 5.0, cell=cell, pbc=pbc)
    csr = _csr(g)
    shifts = g.shifts.clone()
    shifts[7, 0] += 5
    assert find_edge_pairs(csr, shifts.to(DEV)) is None
    assert find_edge_pairs(csr, g.shifts.to(DEV)) is not None
    # ghost senders (rows beyond the receivers) have no reverse
    ei = torch.tensor([[0, 0, 1, 1], [1, 2, 0, 3]])
    csr = build_graph(ei.to(DEV), 2, n_sender_rows=4)
    assert find_edge_pairs(csr, None) is None
    # empty and odd edge lists
    csr = build_graph(torch.zeros(2, 0, dtype=torch.long, device=DEV), 3)
    assert find_edge_pairs(csr, None) is None
    assert launch_edge_pairs(csr, None)[1].tolist() == [0, 0]


def test_pair_edges_have_identical_radial_inputs():
    """The premise: with antisymmetric shift vectors both edges of a pair get bitwise the same
    edge length, radial features and envelope from the device edge geometry."""
    from flashcart_amd.o3 import _ops
    from flashcart_amd.utils.geometry import shift_vectors
    numbers, pos, cell, pbc = fcc_alloy(3, 3, 3, seed=5, jitter=0.3)
    g = AtomicGraph.from_arrays(numbers, pos, ["Cu", "Ni", "Fe", "Cr"], 5.0, cell=cell, pbc=pbc).to(DEV)
    csr = _csr(g)
    pairs = csr.edge_pairs(g.shifts)
    assert pairs is not None
    sv = shift_vectors(g.cell, g.shifts, csr.idx_i, g.batch, antisymmetric=True)
    posd = g.positions.to(torch.float32) + 1e-3 * torch.randn_like(g.positions.to(torch.float32))
    attrs, feats, env = _ops.edge_geometry(posd, sv, csr.idx_i, csr.idx_j, None, csr.rowptr, csr.sender_perm,
                                           csr.sender_ptr, 3, 1, 8, 0.0, 5.0, 6)
    order = torch.empty_like(pairs.slot, dtype=torch.long)
    order[pairs.slot.long()] = torch.arange(csr.n_edges, device=DEV)  # order[2p], order[2p + 1]: pair p
    lo, hi = order[0::2], order[1::2]
    assert torch.equal(lo, pairs.edge.long())
    assert torch.equal(feats[lo], feats[hi]) and torch.equal(env[lo], env[hi])
    # edge attributes of the reverse edge: (-1)^l times the forward ones, l of each component
    sign = torch.tensor([1.0] + [-1.0] * 3 + [1.0] * 5 + [-1.0] * 7, device=DEV)
    assert torch.equal(attrs[hi], attrs[lo] * sign)


def _tp(l1, l2, lo, c):
    from flashcart_amd.o3 import TensorProduct
    return TensorProduct(l1, l2, lo, c, 1, shared_weights=False, reduce_paths=False)


@pytest.mark.parametrize("l1,c", [(2, 128), (0, 64), (1, 32)])
def test_tp_with_pair_slot_equals_expanded_weights(l1, c):
    """Forward and backward with pair_slot are the per-edge computation with the pair's weight row,
    bit for bit (the weight gradient per edge, in edge order)."""
    from flashcart_amd.o3 import _ops
    numbers, pos, cell, pbc = fcc_alloy(2, 2, 2, seed=3)
    g = AtomicGraph.from_arrays(numbers, pos, ["Cu", "Ni", "Fe", "Cr"], 5.0, cell=cell, pbc=pbc).to(DEV)
    csr = _csr(g)
    pairs = csr.edge_pairs(g.shifts)
    tp = _tp(l1, 3, 3, c)
    n, e = csr.n_nodes, csr.n_edges
    gen = torch.Generator(device=DEV).manual_seed(11)
    x = torch.randn(n, tp.in1_dim, device=DEV, generator=gen)
    y = torch.randn(e, 16, device=DEV, generator=gen)
    wp = torch.randn(pairs.n_pairs, tp.n_total_paths * c, device=DEV, generator=gen)
    w_edge = wp[(pairs.slot // 2).long()]
    args = (tp.in1_l_max, tp.in2_l_max, tp.out_l_max, tp.in1_features, tp.in2_features, False, False,
            *tp.op_meta, False)
    csr_args = (csr.rowptr, csr.sender_perm, csr.sender_ptr)
    out_p = _ops.tp_fwd(x, y, wp, csr.idx_i, csr.idx_j, *args, *csr_args, 0.3, pairs.slot)
    out_e = _ops.tp_fwd(x, y, w_edge, csr.idx_i, csr.idx_j, *args, *csr_args, 0.3)
    assert torch.equal(out_p, out_e)
    go = torch.randn_like(out_e)
    g1p, g2p, gwp = _ops.tp_bwd(go, x, y, wp, csr.idx_i, csr.idx_j, *args, True, True, True, *csr_args, 0.3,
                                pairs.slot)
    g1e, g2e, gwe = _ops.tp_bwd(go, x, y, w_edge, csr.idx_i, csr.idx_j, *args, True, True, True, *csr_args, 0.3)
    assert torch.equal(g1p, g1e) and torch.equal(g2p, g2e)
    assert gwp.shape == gwe.shape and torch.equal(gwp, gwe)
    # through autograd the pair-shared weights get the sum of both edges' gradients
    wq = wp.clone().requires_grad_(True)
    _ops.tp_fwd(x, y, wq, csr.idx_i, csr.idx_j, *args, *csr_args, 0.3, pairs.slot).backward(go)
    want = gwe.new_zeros(wp.shape).index_add_(0, (pairs.slot // 2).long(), gwe)
    assert_close(wq.grad, want, 1e-6, 1e-6, "pair weight gradient")


def test_unpaired_slot_contributes_nothing():
    """An edge whose pair slot is -1 (a pairing left it without a partner) has no weight row and no
    h row: the kernels' guards read its weights and h as zero and skip its h-gradient row, so the
    products equal the per-edge computation with that edge's weights (or h) zeroed, bit for bit for
    the tensor product, and the species density matches its float64 definition."""
    from flashcart_amd import _lib
    from flashcart_amd.o3 import _ops
    numbers, pos, cell, pbc = fcc_alloy(2, 2, 2, seed=3)
    g = AtomicGraph.from_arrays(numbers, pos, ["Cu", "Ni", "Fe", "Cr"], 5.0, cell=cell, pbc=pbc).to(DEV)
    csr = _csr(g)
    pairs = csr.edge_pairs(g.shifts)
    k = 7
    slot = pairs.slot.clone()
    slot[k] = -1
    tp = _tp(2, 3, 3, 128)
    n, e = csr.n_nodes, csr.n_edges
    gen = torch.Generator(device=DEV).manual_seed(13)
    x = torch.randn(n, tp.in1_dim, device=DEV, generator=gen)
    y = torch.randn(e, 16, device=DEV, generator=gen)
    wp = torch.randn(pairs.n_pairs, tp.n_total_paths * 128, device=DEV, generator=gen)
    w_edge = wp[(pairs.slot // 2).long()].clone()
    w_edge[k] = 0.0
    args = (tp.in1_l_max, tp.in2_l_max, tp.out_l_max, tp.in1_features, tp.in2_features, False, False,
            *tp.op_meta, False)
    csr_args = (csr.rowptr, csr.sender_perm, csr.sender_ptr)
    print("unpaired slot: tensor product", flush=True)
    out_p = _ops.tp_fwd(x, y, wp, csr.idx_i, csr.idx_j, *args, *csr_args, 1.0, slot)
    out_e = _ops.tp_fwd(x, y, w_edge, csr.idx_i, csr.idx_j, *args, *csr_args, 1.0)
    assert torch.equal(out_p, out_e)
    go = torch.randn_like(out_e)
    gp = _ops.tp_bwd(go, x, y, wp, csr.idx_i, csr.idx_j, *args, True, True, True, *csr_args, 1.0, slot)
    ge = _ops.tp_bwd(go, x, y, w_edge, csr.idx_i, csr.idx_j, *args, True, True, True, *csr_args, 1.0)
    for a, b in zip(gp, ge):
        assert torch.equal(a, b)
    print("unpaired slot: species density", flush=True)
    n_sp, d = 4, 16
    zj = torch.randint(0, n_sp, (e,), device=DEV, generator=gen, dtype=torch.int32)
    h = torch.randn(pairs.n_pairs, 64, device=DEV, generator=gen)
    st = _lib.csr_struct(n, e, csr.idx_j, csr.rowptr, pair_slot=slot)
    dens = _ops.species_density_fwd(st, 3, 3, n_sp, zj, h, y, n)
    he = h.double()[(pairs.slot // 2).long()].clone()
    he[k] = 0.0
    onehot = torch.nn.functional.one_hot(zj.long(), n_sp).double()
    per_edge = (he[:, None, :] * y.double()[:, :, None])[:, :, None, :] * onehot[:, None, :, None]
    want = torch.zeros(n, d, n_sp, 64, dtype=torch.float64, device=DEV).index_add_(0, csr.idx_i.long(), per_edge)
    assert_close(dens.view(n, d, n_sp, 64), want, 1e-5, 1e-5, "density with an unpaired edge")
    gd = torch.randn(n, d * n_sp * 64, device=DEV, generator=gen)
    g_h, g_y = _ops.species_density_bwd(st, 3, 3, n_sp, zj, h, y, gd)
    gsel = (gd.double().view(n, d, n_sp, 64)[csr.idx_i.long()] * onehot[:, None, :, None]).sum(2)
    want_h = (gsel * y.double()[:, :, None]).sum(1)
    want_y = (gsel * he[:, None, :]).sum(2)
    keep = torch.arange(e, device=DEV) != k
    assert_close(g_h[pairs.slot.long()][keep], want_h[keep], 1e-5, 1e-5, "dL/dh of the paired edges")
    assert_close(g_y, want_y, 1e-5, 1e-5, "dL/dy with an unpaired edge")


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


@pytest.mark.parametrize("case", ["fcc_L3_C128", "water_L2_C64", "molecules_L2_C32"])
def test_paired_potential_matches_oracle_and_unpaired(case):
    if case == "fcc_L3_C128":
        numbers, pos, cell, pbc = fcc_alloy(2, 2, 2, seed=3)
        cfg = model_config(["Cu", "Ni", "Fe", "Cr"], 128, 3, avg_neighbors=42.0)
        graph = AtomicGraph.from_arrays(numbers, pos, cfg["elements"], 5.0, cell=cell, pbc=pbc)
    elif case == "water_L2_C64":
        numbers, pos, cell, pbc = water_box(64, seed=1)
        cfg = model_config(["H", "O"], 64, 2, avg_neighbors=50.0)
        graph = AtomicGraph.from_arrays(numbers, pos, cfg["elements"], 5.0, cell=cell, pbc=pbc)
    else:
        cfg = model_config(["H", "C", "N", "O"], 32, 2, avg_neighbors=12.0)
        graph = batch_graphs([AtomicGraph.from_arrays(z, p, cfg["elements"], 5.0) for z, p in molecules(5, seed=7)])
    model = _model(cfg)
    ref = OM.predict(model.state_dict(), model.to_model_config(), graph.to_dict(), compute_forces=True)
    m = model.to(DEV)
    m.requires_grad_(False)
    gd = graph.to(DEV)
    print(f"paired potential: {case}", flush=True)
    out = m.predict(gd, compute_forces=True)
    csr = gd.csr
    assert any(v is not None for v in csr.__dict__.get("_pairs", {}).values()), "the paired path was not taken"
    # the second layer's input maps and the first readout's columns ran as one Function
    nxt = m.interactions[1]
    assert fused.entry_maps_apply(nxt, torch.empty(1, nxt.linear_first.in_dim, device=DEV), m.n_hidden_feats)
    assert_close(out["energy"], ref["energy"], 1e-5, 1e-6, "energy")
    assert_close(out["forces"], ref["forces"], 0.0, 1e-4, "forces")
    # the same potential with the radial MLP parameters trainable takes the per-edge path
    for layer in m.interactions:
        layer.radial_mlp.requires_grad_(True)
    assert not m.wants_edge_pairs(gd.positions)
    un = m.predict(graph.to(DEV), compute_forces=True)
    assert_close(out["energy"], un["energy"], 5e-6, 1e-6, "paired vs per-edge energy")
    # float32 round-off of force sums whose terms reach the largest force
    assert_close(out["forces"], un["forces"], 0.0, 5e-6 * float(un["forces"].abs().max()) + 1e-6,
                 "paired vs per-edge forces")


def test_replay_falls_back_when_pairing_breaks():
    """A captured prediction takes the pairing of its first edge list; an edge list of the same
    size that does not pair up is evaluated eagerly (and correctly)."""
    numbers, pos, cell, pbc = fcc_alloy(2, 2, 2, seed=3)
    cfg = model_config(["Cu", "Ni", "Fe", "Cr"], 16, 3, avg_neighbors=42.0)
    graph = AtomicGraph.from_arrays(numbers, pos, cfg["elements"], 5.0, cell=cell, pbc=pbc)
    model = _model(cfg)
    sd, mc = model.state_dict(), model.to_model_config()
    m = model.to(DEV)
    m.requires_grad_(False)
    gd = graph.to(DEV)
    out0 = m.predict(gd, compute_forces=True, use_compile=True)
    entry = next(iter(m._replay_cache.values()))
    assert entry.paired
    ref0 = OM.predict(sd, mc, graph.to_dict(), compute_forces=True)
    assert_close(out0["forces"], ref0["forces"], 0.0, 1e-4, "replayed forces")
    # break one pair: redirect an edge to a different sender (same edge count, receivers sorted)
    broken = graph.to_dict()
    ei = broken["edge_index"].clone()
    e = 5
    ei[1, e] = (ei[1, e] + 1) % int(broken["atom_types"].shape[0])
    if ei[1, e] == ei[0, e]:
        ei[1, e] = (ei[1, e] + 1) % int(broken["atom_types"].shape[0])
    broken["edge_index"] = ei
    ref1 = OM.predict(sd, mc, broken, compute_forces=True)
    bd = {k: (v.to(DEV) if torch.is_tensor(v) else v) for k, v in broken.items()}
    out1 = m.predict(bd, compute_forces=True, use_compile=True)
    assert_close(out1["energy"], ref1["energy"], 1e-5, 1e-6, "fallback energy")
    assert_close(out1["forces"], ref1["forces"], 0.0, 1e-4, "fallback forces")
    # and back to a pairable list: replayed again
    out2 = m.predict(gd, compute_forces=True, use_compile=True)
    assert_close(out2["forces"], ref0["forces"], 0.0, 1e-4, "replayed forces after fallback")


def test_pair_inputs_op():
    """fc_pair_inputs_fwd/bwd against the same gather written with torch indexing."""
    from flashcart_amd.o3 import _ops
    numbers, pos, cell, pbc = fcc_alloy(2, 2, 2, seed=3)
    g = AtomicGraph.from_arrays(numbers, pos, ["Cu", "Ni", "Fe", "Cr"], 5.0, cell=cell, pbc=pbc).to(DEV)
    csr = _csr(g)
    pairs = csr.edge_pairs(g.shifts)
    gen = torch.Generator(device=DEV).manual_seed(2)
    feats = torch.randn(csr.n_edges, 8, device=DEV, generator=gen, requires_grad=True)
    env = torch.rand(csr.n_edges, device=DEV, generator=gen, requires_grad=True)
    x = _ops.pair_inputs(feats, env, pairs.edge, pairs.slot)
    pe = pairs.edge.long()
    ref = feats[pe] * env[pe].unsqueeze(-1)
    assert torch.equal(x, ref)
    gx = torch.randn_like(x)
    gf, ge = torch.autograd.grad(x, (feats, env), gx)
    rf, re = torch.autograd.grad(ref, (feats, env), gx)
    assert torch.equal(gf, rf)
    assert_close(ge, re, 1e-6, 1e-6, "envelope gradient")


@pytest.mark.parametrize("l_max,y_l_max", [(3, 3), (2, 3), (1, 1)])
def test_species_density_op(l_max, y_l_max):
    """fc_species_density_fwd/bwd against their definitions evaluated in float64 with torch."""
    from flashcart_amd import _lib
    from flashcart_amd.o3 import _ops
    numbers, pos, cell, pbc = fcc_alloy(2, 2, 2, seed=3)
    g = AtomicGraph.from_arrays(numbers, pos, ["Cu", "Ni", "Fe", "Cr"], 5.0, cell=cell, pbc=pbc).to(DEV)
    csr = _csr(g)
    pairs = csr.edge_pairs(g.shifts)
    n, e, n_sp = csr.n_nodes, csr.n_edges, 3
    gen = torch.Generator(device=DEV).manual_seed(5)
    zj = torch.randint(0, n_sp, (e,), device=DEV, generator=gen, dtype=torch.int32)
    h = torch.randn(pairs.n_pairs, 64, device=DEV, generator=gen)
    dy = (y_l_max + 1) ** 2
    y = torch.randn(e, dy, device=DEV, generator=gen)
    d = (l_max + 1) ** 2
    st = _lib.csr_struct(n, e, csr.idx_j, csr.rowptr, pair_slot=pairs.slot)
    dens = _ops.species_density_fwd(st, l_max, y_l_max, n_sp, zj, h, y, n)
    he = h.double()[(pairs.slot // 2).long()]                       # (E, 64)
    contrib = he[:, None, :] * y.double()[:, :d, None]              # (E, d, 64)
    onehot = torch.nn.functional.one_hot(zj.long(), n_sp).double()  # (E, Z)
    per_edge = contrib[:, :, None, :] * onehot[:, None, :, None]    # (E, d, Z, 64)
    want = torch.zeros(n, d, n_sp, 64, dtype=torch.float64, device=DEV).index_add_(0, csr.idx_i.long(), per_edge)
    assert_close(dens.view(n, d, n_sp, 64), want, 1e-5, 1e-5, "density")
    gd = torch.randn(n, d * n_sp * 64, device=DEV, generator=gen)
    g_h, g_y = _ops.species_density_bwd(st, l_max, y_l_max, n_sp, zj, h, y, gd)
    gde = gd.double().view(n, d, n_sp, 64)[csr.idx_i.long()]        # (E, d, Z, 64)
    gsel = (gde * onehot[:, None, :, None]).sum(2)                  # (E, d, 64)
    want_h = (gsel * y.double()[:, :d, None]).sum(1)                # (E, 64) per edge
    want_y = torch.zeros(e, dy, dtype=torch.float64, device=DEV)
    want_y[:, :d] = (gsel * he[:, None, :]).sum(2)
    assert_close(g_h[pairs.slot.long()], want_h, 1e-5, 1e-5, "dL/dh per edge")
    assert_close(g_y, want_y, 1e-5, 1e-5, "dL/dy")


@pytest.mark.parametrize("n_sp,c_in,c_mid,c_out,nh,n_ranks", [(4, 128, 128, 128, 64, 4), (2, 64, 64, 64, 64, 3),
                                                              (3, 20, 40, 24, 48, 1), (8, 16, 100, 17, 64, 2)])
def test_species_maps_op(n_sp, c_in, c_mid, c_out, nh, n_ranks):
    """fc_species_maps (every rank in one launch) against its definition in float64: the species'
    sender features s table W_first^T / alpha_div, then per rank sum_c W_second[o, c] x[Z, c] W2[l c_mid + c, k];
    partial o blocks and hidden widths below 64 included."""
    from flashcart_amd.o3 import _ops
    gen = torch.Generator(device=DEV).manual_seed(n_sp + c_mid)
    table = torch.randn(n_sp, c_in, device=DEV, generator=gen)
    wf = torch.randn(c_mid, c_in, device=DEV, generator=gen)
    ws = [torch.randn(c_out, c_mid, device=DEV, generator=gen) for _ in range(n_ranks)]
    w2 = torch.randn(n_ranks * c_mid + 5, nh, device=DEV, generator=gen)
    div = torch.tensor([6.5], device=DEV)
    mats = _ops.species_maps(table, wf, 0.125, div, ws, w2)
    x = 0.125 * table.double() @ wf.double().t() / 6.5                       # (Z, c)
    for l in range(n_ranks):
        blk = w2.double()[l * c_mid:(l + 1) * c_mid]                          # (c, k)
        want = torch.einsum("oc,zc,ck->ozk", ws[l].double(), x, blk).reshape(c_out, n_sp * nh)
        assert mats[l].shape == (c_out, n_sp * nh)
        assert_close(mats[l], want, 1e-5, 1e-5 * float(want.abs().max()), f"species map rank {l}")


def test_species_conv_matches_paired_conv():
    """The first interaction layer as a species density (linear_second folded in) against the same
    layer over edge pairs followed by linear_second: outputs and input gradients (edge attributes,
    radial inputs) at float32 round-off; a second call forms the same maps again."""
    from flashcart_amd.o3 import _ops
    numbers, pos, cell, pbc = fcc_alloy(3, 3, 3, seed=4)
    cfg = model_config(["Cu", "Ni", "Fe", "Cr"], 128, 3, avg_neighbors=42.0)
    g = AtomicGraph.from_arrays(numbers, pos, cfg["elements"], 5.0, cell=cell, pbc=pbc).to(DEV)
    model = _model(cfg).to(DEV)
    model.requires_grad_(False)
    layer = model.interactions[0]
    csr = _csr(g)
    pairs = csr.edge_pairs(g.shifts)
    gen = torch.Generator(device=DEV).manual_seed(8)
    y = torch.randn(csr.n_edges, 16, device=DEV, generator=gen, requires_grad=True)
    xp = torch.rand(pairs.n_pairs, 8, device=DEV, generator=gen, requires_grad=True)
    table = model.embedding.weight
    zj = torch.index_select(g.atom_types.to(torch.int32), 0, csr.idx_j)
    alpha = layer.sqrt_avg_neighbors
    node = model.embedding(g.atom_types)
    assert fused.species_conv_applies(layer, node, table.shape[0])
    out_s = fused.species_conv(layer, y, xp, csr, pairs, zj, table, alpha)
    out_p = layer.linear_second(fused.paired_conv(layer, layer.linear_first(node), y, xp, csr, pairs, alpha))
    again = fused.species_conv(layer, y, xp, csr, pairs, zj, table, alpha)
    assert torch.equal(out_s, again)
    assert_close(out_s, out_p, 1e-5, 1e-5 * float(out_p.abs().max()), "species vs paired output")
    go = torch.randn_like(out_p)
    gs = torch.autograd.grad(out_s, (y, xp), go)
    gp = torch.autograd.grad(out_p, (y, xp), go)
    for a, b, what in zip(gs, gp, ("edge attributes", "radial inputs")):
        assert_close(a, b, 1e-5, 1e-5 * float(b.abs().max()), f"species vs paired gradient of {what}")
    # the maps follow in-place changes of the table and of linear_first's weights
    with torch.no_grad():
        table.mul_(1.5)
        layer.linear_first.weight[0].add_(0.25)
    node = model.embedding(g.atom_types)
    out_s = fused.species_conv(layer, y, xp, csr, pairs, zj, table, alpha)
    out_p = layer.linear_second(fused.paired_conv(layer, layer.linear_first(node), y, xp, csr, pairs, alpha))
    assert not torch.equal(out_s, again)
    assert_close(out_s, out_p, 1e-5, 1e-5 * float(out_p.abs().max()), "species vs paired output after an update")


@pytest.mark.parametrize("m", [2176, 272])
@pytest.mark.parametrize("gathered", [False, True])
def test_dense_bwd_pairs(m, gathered):
    """The pair-summed input gradient (fc_dense_fwd_pairsum with adjacent or gathered rows, and the
    summed-then-multiplied form for widths that are not multiples of 32) against torch float64."""
    from flashcart_amd.o3 import _ops
    gen = torch.Generator(device=DEV).manual_seed(9)
    g = torch.randn(2 * 1001, m, device=DEV, generator=gen)
    w = torch.randn(m, 64, device=DEV, generator=gen)
    if gathered:
        perm = torch.randperm(2 * 1001, device=DEV, generator=gen).to(torch.int32)
        lo, hi = perm[:1001], perm[1001:]
        got = _ops.dense_bwd_pairs(g, w, 0.37, lo, hi)
        want = 0.37 * (g.double()[lo.long()] + g.double()[hi.long()]) @ w.double()
    else:
        got = _ops.dense_bwd_pairs(g, w, 0.37)
        want = 0.37 * (g.double()[0::2] + g.double()[1::2]) @ w.double()
    assert_close(got, want, 1e-5, 1e-5 * float(want.abs().max()), "pair-summed input gradient")
