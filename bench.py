"""Benchmark: FlashCart energy+forces inference on one MI355X.

Workload (the metric's config): periodic fcc random alloy,
25x25x10 conventional cells (25,000 atoms, a = 3.6 A, 4 species, jitter 0.05 A),
FlashCartPotential with the packaged default architecture at 128 channels, L_max = 3,
2 interactions, r_max = 5 A, random-init weights (seed 1234), float32. Each step is one
MD-style evaluation (energy + forces via autograd) after a fresh N(0, 0.01^2) A
perturbation of the positions. Neighbour lists for every step are built before the
timed region (host cell list at r_max + skin, filtered to r_max per step, rebuilt when an
atom moved more than skin / 2), as in the reference's timing protocol; the receiver
CSR of each step's graph is built on the GPU inside the timed region.

Prints one JSON line: atom-steps/s, the roofline of the dominant kernel (measured
live with HIP events on the stream it is launched on), and the CPU baseline (the
oracle restatement of the reference PyTorch path on a bounded 256-atom sample).
"""

from __future__ import annotations

import argparse
import json
import os
import sys
import time

import numpy as np

# Edge counts change from step to step, so the multi-GB per-edge tensors change size every
# step; rounding allocations to 1/8 power-of-two steps lets the caching allocator reuse its
# blocks instead of reserving new ones until it has to flush (set before torch allocates).
os.environ.setdefault("PYTORCH_HIP_ALLOC_CONF", "roundup_power2_divisions:8")

import torch  # noqa: E402

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0
# HBM bytes per launch of the dominant kernel from rocprofv3 memory-request counters of
# `bench.py --kernel-only` (first step graph, E = 1,080,166, weight rows shared by edge pairs as the
# step runs them): read bytes by request size (TCC_EA0_RDREQ_32B/64B/128B), written bytes from
# TCC_EA0_WRREQ / WRREQ_64B; a 2 GiB copy reads back 2.148 / 2.147 GB. See
# profiles/hbm_counter_method.md and profiles/tp_conv_l1_fcc25k_kernel_only.md.
MEASURED_TRAFFIC_BYTES = 11.33e9
# The same for the layer-1 backward op (tp_bwd_conv_kernel + segment_rows_kernel).
MEASURED_TRAFFIC_BWD_BYTES = 32.14e9
from flashcart_amd.data.synthetic import FCC25K_R_MAX as R_MAX  # noqa: E402
from flashcart_amd.data.synthetic import FCC25K_SIGMA_STEP as SIGMA_STEP  # noqa: E402
from flashcart_amd.data.synthetic import FCC25K_SKIN as SKIN  # noqa: E402
from flashcart_amd.data.synthetic import StepGraphs  # noqa: E402
from flashcart_amd.data.synthetic import fcc25k_model as build_model  # noqa: E402
from flashcart_amd.data.synthetic import fcc25k_system as make_system  # noqa: E402

# The counter runs' graph (the first step graph: N = 25,000, E = 1,080,166) and the compulsory
# bytes of the layer-1 convolution on it (d1 = 9, d2 = 16, P = 17, C = 128, 71 output rows).
TRAFFIC_E = 1080166


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def tp_conv_bytes(n_nodes, n_send, E, d1, d2, P, C, nout):
    """Compulsory HBM bytes of one convolution TP forward (fp32, int32 indices): in1 rows, edge
    attributes, per-edge weights and the receiver outputs once each, the sender index and rowptr."""
    return 4 * (n_send * d1 * C + E * d2 + E * P * C + n_nodes * nout * C) + 4 * E + 4 * (n_nodes + 1)


def tp_conv_bwd_bytes(n_nodes, E, d1, d2, P, C, nout):
    """Compulsory HBM bytes of one convolution TP backward with all three gradients (the
    per-edge formula of the hot-path survey's measurement table,
    4 (N o C + 2 N d1 C + 2 E d2 + 2 E P C) + 8 E + 4 (N + 1)): the output gradient read once,
    in1 read and its gradient written, edge attributes read and their gradient written, weights
    read and their gradient written, two index arrays and rowptr. Per-edge sender messages or any
    other intermediate of an implementation are not counted."""
    return 4 * (n_nodes * nout * C + 2 * n_nodes * d1 * C + 2 * E * d2 + 2 * E * P * C) + 8 * E + 4 * (n_nodes + 1)




def device_time_ms(fn, reps, dev, warmup=3):
    """Average device time of ``fn`` replayed from a captured HIP graph: HIP events on the
    stream the replays run on bracket ``reps`` replays (no host launch overhead inside)."""
    side = torch.cuda.Stream(dev)
    side.wait_stream(torch.cuda.current_stream(dev))
    with torch.cuda.stream(side):
        for _ in range(warmup):
            fn()
    torch.cuda.current_stream(dev).wait_stream(side)
    torch.cuda.synchronize(dev)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        fn()
    graph.replay()
    torch.cuda.synchronize(dev)
    stream = torch.cuda.current_stream(dev)
    ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    ev0.record(stream)
    for _ in range(reps):
        graph.replay()
    ev1.record(stream)
    torch.cuda.synchronize(dev)
    return ev0.elapsed_time(ev1) / reps


def calibration_kernels(dev, reps):
    """Two kernels of known HBM bytes that check the memory-request counters: a streaming copy
    (2 GiB read, 2 GiB written) and a row gather by a random permutation (index_select of 2^22
    rows of 512 B: 2 GiB of rows + 32 MiB of int64 indices read, 2 GiB written), the access
    pattern of the convolution's in1 rows."""
    src = torch.ones(2 ** 29, device=dev)  # 2 GiB
    dst = torch.empty_like(src)
    rows = src.view(2 ** 22, 128)
    perm = torch.randperm(2 ** 22, device=dev)
    out = torch.empty_like(rows)
    for _ in range(reps):
        torch.mul(src, 1.0, out=dst)
    for _ in range(reps):
        torch.index_select(rows, 0, perm, out=out)
    torch.cuda.synchronize(dev)
    return {"copy_bytes_each_way": src.numel() * 4, "gather_bytes_read": src.numel() * 4 + perm.numel() * 8,
            "gather_bytes_written": src.numel() * 4}


def measure_dominant(model, graph, dev, reps=10, with_backward=False):
    """Average duration of the layer-1 TP convolution forward (the north star's TP kernel),
    timed with HIP events on the stream the op launches on (torch's current stream), and
    with ``with_backward`` also of its backward op (the largest kernel of the step by time).
    As the step runs them: when the edge list pairs up, one weight row per edge pair read by
    both edges (pair_slot)."""
    from flashcart_amd.o3 import _ops
    from flashcart_amd.o3._graph import build_graph
    inter = model.interactions[1]
    tp = inter.tp
    n = graph.num_nodes
    csr = build_graph(graph.edge_index, n)
    E = csr.n_edges
    pairs = csr.edge_pairs(graph.shifts if bool(getattr(graph, "use_shifts", True)) else None)
    g = torch.Generator(device=dev).manual_seed(0)
    in1 = torch.randn(n, tp.in1_dim, device=dev, generator=g)
    in2 = torch.randn(E, tp.in2_dim, device=dev, generator=g)
    w_rows = pairs.n_pairs if pairs is not None else E
    w = torch.randn(w_rows, tp.n_total_paths * tp.in1_features, device=dev, generator=g)
    args = (in1, in2, w, csr.idx_i, csr.idx_j, tp.in1_l_max, tp.in2_l_max, tp.out_l_max, tp.in1_features,
            tp.in2_features, False, False, *tp.op_meta, False, csr.rowptr, csr.sender_perm, csr.sender_ptr, 1.0,
            pairs.slot if pairs is not None else None)
    for _ in range(2):
        _ops.tp_fwd(*args)
    stream = torch.cuda.current_stream(dev)
    ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize(dev)
    ev0.record(stream)
    for _ in range(reps):
        _ops.tp_fwd(*args)
    ev1.record(stream)
    torch.cuda.synchronize(dev)
    ms = ev0.elapsed_time(ev1) / reps
    nout = tp.out_dim // tp.in1_features
    d1, d2, P, C = (tp.in1_l_max + 1) ** 2, (tp.in2_l_max + 1) ** 2, tp.n_total_paths, tp.in1_features
    byts = tp_conv_bytes(n, n, E, d1, d2, P, C, nout)
    # bytes of distinct data: with pairs each weight row is read by two edges (the formula counts E)
    uniq = byts - 4 * (E - w_rows) * P * C
    info = {"weight_rows": w_rows, "edges": E, "distinct_bytes_fwd": uniq}
    if not with_backward:
        return ms, byts, info
    # The backward op as the energy+forces step runs it (gradients for in1, in2 and the
    # weights): the backward kernel, then the sender-ordered segmented sum of the per-edge
    # messages; achieved bandwidth on the compulsory bytes of the three gradients.
    go = torch.randn(n, tp.out_dim, device=dev, generator=g)
    bargs = (go,) + args[:17] + (False, True, True, True) + args[18:]
    for _ in range(2):
        _ops.tp_bwd(*bargs)
    torch.cuda.synchronize(dev)
    ev0.record(stream)
    for _ in range(reps):
        _ops.tp_bwd(*bargs)
    ev1.record(stream)
    torch.cuda.synchronize(dev)
    ms_b = ev0.elapsed_time(ev1) / reps
    byts_b = tp_conv_bwd_bytes(n, E, d1, d2, P, C, nout)
    info["distinct_bytes_bwd"] = byts_b - 4 * (E - w_rows) * P * C
    return ms, byts, ms_b, byts_b, info


def _socket_power_sampler(samples, stop):
    """Append (socket W, mean GFX clock MHz) read by ``amd-smi metric -p -c`` until ``stop``."""
    import re
    import subprocess
    while not stop.is_set():
        try:
            txt = subprocess.run(["amd-smi", "metric", "-p", "-c"], capture_output=True, text=True,
                                 timeout=10).stdout
        except (OSError, subprocess.TimeoutExpired):
            return
        p = re.search(r"SOCKET_POWER: (\d+)", txt)
        c = [int(v) for v in re.findall(r"GFX_\d+:\s*CLK: (\d+) MHz", txt)]
        if p and c:
            samples.append((int(p.group(1)), sum(c) / len(c)))


def power_per_kernel(model, graphs, dev, seconds=4.0):
    """Socket power while each of the step's heavy ops runs alone in a loop (and the whole
    energy+forces step, cycling over ``graphs``), sampled by amd-smi over the last 3 s of each
    loop. Returns {op: {"ms_per_call", "watts", "clock_mhz", "samples"}}."""
    import ctypes
    import threading
    from flashcart_amd import _lib
    from flashcart_amd.o3 import _ops
    from flashcart_amd.o3._graph import build_graph
    graph = graphs[0]
    inter = model.interactions[1]
    tp = inter.tp
    n = graph.num_nodes
    csr = build_graph(graph.edge_index, n)
    pairs = csr.edge_pairs(graph.shifts)
    g = torch.Generator(device=dev).manual_seed(0)
    in1 = torch.randn(n, tp.in1_dim, device=dev, generator=g)
    in2 = torch.randn(csr.n_edges, tp.in2_dim, device=dev, generator=g)
    rows = pairs.n_pairs if pairs is not None else csr.n_edges
    w = torch.randn(rows, tp.n_total_paths * tp.in1_features, device=dev, generator=g)
    args = (in1, in2, w, csr.idx_i, csr.idx_j, tp.in1_l_max, tp.in2_l_max, tp.out_l_max, tp.in1_features,
            tp.in2_features, False, False, *tp.op_meta, False, csr.rowptr, csr.sender_perm, csr.sender_ptr, 1.0,
            pairs.slot if pairs is not None else None)
    go = torch.randn(n, tp.out_dim, device=dev, generator=g)
    bargs = (go,) + args[:17] + (False, True, True, True) + args[18:]
    lin = model.products[0].product_linears[1]
    x_lin = torch.randn(n, lin.in_dim, device=dev, generator=g)
    mlp = inter.radial_mlp
    x_mlp = torch.randn(rows, mlp[0].weight.shape[1], device=dev, generator=g)
    src = torch.ones(2 ** 29, device=dev)
    dst = torch.empty_like(src)
    step_k = [0]

    def step():
        model.predict(graphs[step_k[0] % len(graphs)], compute_forces=True)
        step_k[0] += 1

    ops = {
        "idle": None,
        "copy_2GiB": lambda: torch.mul(src, 1.0, out=dst),
        "gemm_product_linear_fwd": lambda: lin(x_lin),
        "tp_conv_fwd_layer1": lambda: _ops.tp_fwd(*args),
        "tp_conv_bwd_layer1": lambda: _ops.tp_bwd(*bargs),
        "radial_mlp_fwd_layer1": lambda: _ops.radial_mlp_fwd(x_mlp, mlp[0].weight, mlp[0]._scale, mlp[2].weight,
                                                             mlp[2]._scale, mlp[4].weight, mlp[4]._scale),
        "energy_forces_step": step,
    }
    out = {}
    for name, fn in ops.items():
        if fn is not None and name != "energy_forces_step":
            fn = torch.no_grad()(fn)
        if fn is not None:
            for _ in range(3):
                fn()
        torch.cuda.synchronize(dev)
        samples, stop = [], threading.Event()
        sampler = threading.Thread(target=_socket_power_sampler, args=(samples, stop), daemon=True)
        calls, t0 = 0, time.perf_counter()
        while time.perf_counter() - t0 < seconds:
            if fn is None:
                time.sleep(0.05)
            else:
                for _ in range(5):
                    fn()
                calls += 5
                torch.cuda.synchronize(dev)
            if not sampler.is_alive() and not stop.is_set() and time.perf_counter() - t0 > seconds - 3.0:
                sampler.start()
        dt = time.perf_counter() - t0
        stop.set()
        sampler.join(timeout=15)
        out[name] = {"ms_per_call": round(1e3 * dt / calls, 4) if calls else None,
                     "watts": round(sum(p for p, _ in samples) / len(samples), 1) if samples else None,
                     "clock_mhz": round(sum(c for _, c in samples) / len(samples)) if samples else None,
                     "samples": len(samples)}
        log(f"power {name}: {out[name]}")
    return out


def cpu_baseline(model, cfg, avg_neighbors, budget_s=20.0, cells=(8, 8, 8)):
    """Oracle (CPU PyTorch restatement of the reference path), float32, on a bounded sample of the
    same system: fcc 8x8x8 cells = 2,048 atoms of the same model, at least 3 calls after 1 warmup."""
    from flashcart_amd.data.graph import AtomicGraph
    from oracle import model as OM
    cores = len(os.sched_getaffinity(0))
    torch.set_num_threads(cores)
    numbers, pos, cell, pbc = make_system(*cells, seed=5)
    g = AtomicGraph.from_arrays(numbers, pos, cfg["elements"], R_MAX, cell=cell, pbc=pbc)
    sd = {k: v.detach().cpu() for k, v in model.state_dict().items()}
    mcfg = model.to_model_config()
    gd = g.to_dict()
    from oracle import ops as O
    with O.components_form():  # the reference's per-component CPU op sequence
        OM.predict(sd, mcfg, gd, dtype=torch.float32, chunk=512)  # warmup
        t0 = time.perf_counter()
        calls = 0
        while calls < 3 or (time.perf_counter() - t0 < budget_s and calls < 50):
            OM.predict(sd, mcfg, gd, dtype=torch.float32, chunk=512)
            calls += 1
    dt = time.perf_counter() - t0
    n = len(numbers)
    return {"value": n * calls / dt, "unit": "atom-steps/s", "cores": cores, "kind": "port",
            "sample": f"oracle (CPU PyTorch restatement of the reference path; tensor products as per-component "
                      f"polynomials, the reference's generated CPU op sequence), float32, fcc {cells[0]}x{cells[1]}x"
                      f"{cells[2]} = {n} atoms, "
                      f"{int(g.edge_index.shape[1])} edges, same model config and weights, {calls} calls after "
                      f"1 warmup, {dt:.1f} s, torch threads = {cores}"}


def _timed(fn, steps, warmup, dev):
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize(dev)
    t0 = time.perf_counter()
    for _ in range(steps):
        out = fn()
    torch.cuda.synchronize(dev)
    return time.perf_counter() - t0, out


def _oracle_rate(sd, mcfg, gd, n_atoms, budget_s=20.0):
    """Oracle energy+forces on the host cores, float32, tensor products in the reference's
    per-component CPU op sequence."""
    from oracle import model as OM
    from oracle import ops as O
    cores = len(os.sched_getaffinity(0))
    torch.set_num_threads(cores)
    with O.components_form():
        t0 = time.perf_counter()
        OM.predict(sd, mcfg, gd, dtype=torch.float32)  # warmup
        warm = time.perf_counter() - t0
        calls, t0 = 0, time.perf_counter()
        while calls < 1 or (calls < 3 and time.perf_counter() - t0 + warm < budget_s):
            OM.predict(sd, mcfg, gd, dtype=torch.float32)
            calls += 1
        dt = time.perf_counter() - t0
    return n_atoms * calls / dt, cores, calls, dt


CONFIG_LINES = ("cfg1_tp_standalone", "cfg2_expansion_radial", "cfg3_water_1536", "cfg5_molecules_512")


def _cpu_rate(fn, units, budget_s=8.0):
    """Units per second of ``fn`` on the host cores (1 warmup, then calls within ``budget_s``)."""
    cores = len(os.sched_getaffinity(0))
    torch.set_num_threads(cores)
    fn()
    calls, t0 = 0, time.perf_counter()
    while calls < 3 or (time.perf_counter() - t0 < budget_s and calls < 200):
        fn()
        calls += 1
    dt = time.perf_counter() - t0
    return units * calls / dt, cores, calls, dt


MFMA_PEAK_TFLOPS = 157.3  # MI355X dense fp32 MFMA


def mfma_in_step(step, dev, launches=None):
    """In-step MFMA utilisation of the linear maps: ``step()`` (one energy+forces evaluation, run
    eagerly) under ``_ops.mfma_timer``, which brackets every MFMA kernel launch of the step with HIP
    events on its stream; achieved = the launches' algorithmic FLOPs (by formula from each call's
    shapes) / the sum of their event durations, per family and overall, against the fp32 MFMA peak."""
    from flashcart_amd.o3 import _ops
    with _ops.mfma_timer() as rec:
        step()
    torch.cuda.synchronize(dev)
    groups = {}
    for name, group, flops, e0, e1, shape in rec:
        ms = e0.elapsed_time(e1)
        if launches is not None:
            launches.append({"entry_point": name, "family": group, "shape": shape, "gflop": flops / 1e9,
                             "us": ms * 1e3, "tflops": flops / (ms * 1e-3) / 1e12})
        g = groups.setdefault(group, {"launches": 0, "flops": 0.0, "ms": 0.0})
        g["launches"] += 1
        g["flops"] += flops
        g["ms"] += ms
    tot_f = sum(g["flops"] for g in groups.values())
    tot_ms = sum(g["ms"] for g in groups.values())
    for g in groups.values():
        g["tflops"] = g["flops"] / (g["ms"] * 1e-3) / 1e12
        g["frac"] = g["tflops"] / MFMA_PEAK_TFLOPS
    achieved = tot_f / (tot_ms * 1e-3) / 1e12 if tot_ms > 0 else 0.0
    return {"bound": "mfma", "kernel": "every MFMA launch of one step (equivariant linear maps, dense layers, "
                                       "radial MLP)",
            "achieved": achieved, "peak": MFMA_PEAK_TFLOPS, "unit": "TFLOP/s", "frac": achieved / MFMA_PEAK_TFLOPS,
            "flops_per_step": tot_f, "ms_per_step": tot_ms, "launches": sum(g["launches"] for g in groups.values()),
            "groups": groups,
            "method": "HIP events around each MFMA launch inside one eager energy+forces step (the stream the "
                      "kernels run on); FLOPs from each call's shapes: 2 n (2l+1) C_in paths_l C_out per rank for "
                      "the equivariant maps, 2 n k m for dense layers, each layer for the radial MLP kernels"}


def config_line(name, dev, steps, warmup, cpu, extras=True):
    """One BASELINE configuration other than the metric's: throughput from device time (HIP
    events around HIP-graph replays, so that host launch work is not counted), the roofline
    fraction of its tensor-product work on the compulsory bytes, and (``cpu``) the oracle on
    the host cores on the same inputs or a stated sample. ``extras=False`` (the kernel-trace
    runs of the model configurations) times the replays only: no eager timing, no separate
    launches of the dominant kernels, no MFMA event run, so that the trace holds exactly the
    kernels of the timed path."""
    from flashcart_amd import o3
    from flashcart_amd.data import AtomicGraph, batch_graphs
    from flashcart_amd.data.synthetic import model_config, molecules, water_box
    from flashcart_amd.o3 import _ops
    from flashcart_amd.o3._graph import build_graph
    from oracle import ops as O
    res = {"workload": name}
    if name == "cfg1_tp_standalone":
        # TensorProduct(2, 2, 2, 32, 1), conv mode: 512 receivers x 8 sorted in-edges, E = 4096;
        # forward and the gradients of both inputs (the weight gradient is formed as well, so the
        # compulsory-byte formula of the forward + full backward applies unchanged)
        rng = np.random.default_rng(0)
        n_recv, E, C = 512, 4096, 32
        ii = np.repeat(np.arange(n_recv), 8)
        jj = rng.integers(0, n_recv - 1, size=E)
        jj = jj + (jj >= ii)
        tp = o3.TensorProduct(2, 2, 2, C, 1)
        v = rng.standard_normal((E, 3))
        v = torch.as_tensor(v / np.linalg.norm(v, axis=1, keepdims=True), dtype=torch.float32, device=dev)
        in2 = o3.Irreps(2).forward_normalized(v)
        gen = torch.Generator(device=dev).manual_seed(0)
        in1 = torch.randn(n_recv, 9 * C, device=dev, generator=gen)
        w = torch.randn(E, tp.n_total_paths * C, device=dev, generator=gen)
        go = torch.randn(n_recv, tp.out_dim, device=dev, generator=gen)
        ei = torch.stack([torch.as_tensor(ii, device=dev), torch.as_tensor(jj, device=dev)])
        csr = build_graph(ei, n_recv)
        args = (in1, in2, w, csr.idx_i, csr.idx_j, 2, 2, 2, C, 1, False, False, *tp.op_meta, False, csr.rowptr,
                csr.sender_perm, csr.sender_ptr, 1.0)

        def step():
            _ops.tp_fwd(*args)
            return _ops.tp_bwd(go, *args[:17], False, True, True, True, *args[18:])
        ms = device_time_ms(step, steps, dev)
        fwd = tp_conv_bytes(n_recv, n_recv, E, 9, 9, tp.n_total_paths, C, tp.out_dim // C)
        bwd = tp_conv_bwd_bytes(n_recv, E, 9, 9, tp.n_total_paths, C, tp.out_dim // C)
        res.update({"metric": "TP forward + gradients per second (E=4096, 2x2->2, C=32, conv)", "value": 1e3 / ms,
                    "unit": "calls/s", "ms_per_step": ms,
                    "roofline": {"bound": "hbm", "kernel": "tp_fwd + tp_bwd (conv, one call each)",
                                 "algorithmic_bytes": fwd + bwd, "achieved": (fwd + bwd) / (ms * 1e-3) / 1e9,
                                 "peak": HBM_PEAK_GBS, "unit": "GB/s",
                                 "frac": (fwd + bwd) / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS,
                                 "note": "24 MB per call: bound by launch and tail latency, not bandwidth"}})
        if cpu:
            c1, c2, cw = in1.cpu().requires_grad_(), in2.cpu().requires_grad_(), w.cpu().requires_grad_()
            cgo, ci, cj = go.cpu(), ei[0].cpu(), ei[1].cpu()

            def cstep():
                with O.components_form():
                    out = O.tensor_product(c1, c2, cw, ci, cj, 2, 2, 2, C, 1)
                return torch.autograd.grad(out, [c1, c2, cw], cgo)
            rate, cores, calls, cdt = _cpu_rate(cstep, 1)
            res["cpu_baseline"] = {"value": rate, "unit": "calls/s", "cores": cores, "kind": "port",
                                   "sample": f"oracle float32 (per-component op sequence), same inputs, {calls} calls "
                                             f"in {cdt:.1f} s"}
    elif name == "cfg2_expansion_radial":
        # E = 200,000 edge vectors (|v| ~ U[0.8, 5.0] A, direction uniform): Eq. (1) l <= 3, 8 Bessel
        # functions, polynomial cutoff p = 6 at 5 A, one fused kernel
        from flashcart_amd import _lib as L
        rng = np.random.default_rng(0)
        E = 200_000
        d = rng.uniform(0.8, 5.0, size=E)
        r = rng.standard_normal((E, 3))
        r /= np.linalg.norm(r, axis=1, keepdims=True)
        vec = torch.as_tensor(d[:, None] * r, dtype=torch.float32, device=dev)
        idx = torch.arange(E, dtype=torch.int32, device=dev)
        rowptr = torch.arange(E + 1, dtype=torch.int32, device=dev)
        ms = device_time_ms(lambda: _ops.edge_geometry(None, None, idx, idx, vec, rowptr, idx, rowptr, 3,
                                                        L.BASIS_BESSEL, 8, 0.0, 5.0, 6), steps, dev)
        byts = 112 * E
        res.update({"metric": "edges/s (expansion l<=3 + 8 Bessel + cutoff p=6, fused, E=200k)",
                    "value": E / (ms * 1e-3), "unit": "edges/s", "ms_per_step": ms,
                    "roofline": {"bound": "hbm", "kernel": "edge_fwd_kernel (vector given)", "algorithmic_bytes": byts,
                                 "achieved": byts / (ms * 1e-3) / 1e9, "peak": HBM_PEAK_GBS, "unit": "GB/s",
                                 "frac": byts / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS,
                                 "note": "22.4 MB per launch: a few microseconds, bound by launch latency"}})
        if cpu:
            cv = vec.cpu()

            def cstep():
                dd = cv.norm(dim=-1)
                u = cv / dd.unsqueeze(-1)
                return O.irreps(u, 3), O.bessel(dd, 8, 5.0), O.cutoff(dd, 5.0, 6)
            rate, cores, calls, cdt = _cpu_rate(cstep, E)
            res["cpu_baseline"] = {"value": rate, "unit": "edges/s", "cores": cores, "kind": "port",
                                   "sample": f"oracle float32, same 200k edges, {calls} calls in {cdt:.1f} s"}
    else:
        if name == "cfg3_water_1536":
            z, p, cell, pbc = water_box(512, seed=0)
            elements, C, L = ["H", "O"], 64, 2
            graph = AtomicGraph.from_arrays(z, p, elements, R_MAX, cell=cell, pbc=pbc)
            oracle_graph = graph
        else:
            mols = molecules(512, seed=0)
            elements, C, L = ["H", "C", "N", "O"], 64, 2
            gs = [AtomicGraph.from_arrays(zz, pp, elements, R_MAX) for zz, pp in mols]
            graph = batch_graphs(gs)
            oracle_graph = batch_graphs(gs[:16])
        n_atoms = graph.num_nodes
        avg = graph.edge_index.shape[1] / n_atoms
        from flashcart_amd.model import FlashCartPotential
        torch.manual_seed(1234)
        model = FlashCartPotential.from_config(model_config(elements, C, L, r_max=R_MAX, avg_neighbors=avg))
        for q in model.parameters():
            q.requires_grad_(False)
        model = model.to(dev)
        gdev = graph.to(dev)
        dt_eager = _timed(lambda: model.predict(gdev, compute_forces=True), steps, warmup, dev)[0] if extras else None
        # fixed topology: the whole prediction replayed as one HIP graph (predict(use_compile=True))
        for _ in range(warmup):
            model.predict(gdev, compute_forces=True, use_compile=True)
        stream = torch.cuda.current_stream(dev)
        ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize(dev)
        ev0.record(stream)
        for _ in range(steps):
            out = model.predict(gdev, compute_forces=True, use_compile=True)
        ev1.record(stream)
        torch.cuda.synchronize(dev)
        ms = ev0.elapsed_time(ev1) / steps
        if not bool(torch.isfinite(out["energy"]).all()):
            raise RuntimeError(f"{name}: non-finite energy")
        res.update({"metric": "atom-steps/s (energy+forces)", "value": n_atoms / (ms * 1e-3), "unit": "atom-steps/s",
                    "ms_per_step": ms, "mode": "HIP graph replay of predict (use_compile=True), frozen parameters",
                    "config": {"n_atoms": n_atoms, "n_graphs": graph.num_graphs,
                               "n_edges": int(graph.edge_index.shape[1]), "channels": C, "l_max_edge_attrs": L}})
        if extras:
            f_ms, f_b, b_ms, b_b, _ = measure_dominant(model, gdev, dev, with_backward=True)
            res.update({
                "eager": {"value": n_atoms * steps / dt_eager, "ms_per_step": 1e3 * dt_eager / steps},
                "roofline": {"bound": "hbm", "kernel": "layer-1 TP convolution backward op (64 channels: "
                                                       "tp_bwd_send_kernel, in sender order)",
                             "algorithmic_bytes": b_b, "avg_launch_ms": b_ms,
                             "achieved": b_b / (b_ms * 1e-3) / 1e9, "peak": HBM_PEAK_GBS, "unit": "GB/s",
                             "frac": b_b / (b_ms * 1e-3) / 1e9 / HBM_PEAK_GBS},
                "roofline_tp_fwd": {"bound": "hbm", "kernel": "layer-1 TP convolution forward", "algorithmic_bytes": f_b,
                                    "avg_launch_ms": f_ms, "achieved": f_b / (f_ms * 1e-3) / 1e9,
                                    "peak": HBM_PEAK_GBS, "unit": "GB/s",
                                    "frac": f_b / (f_ms * 1e-3) / 1e9 / HBM_PEAK_GBS},
                "roofline_linear": mfma_in_step(lambda: model.predict(gdev, compute_forces=True), dev)})
        if cpu:
            sd = {k: v.detach().cpu() for k, v in model.state_dict().items()}
            rate, cores, calls, cdt = _oracle_rate(sd, model.to_model_config(), oracle_graph.to_dict(),
                                                   oracle_graph.num_nodes)
            res["cpu_baseline"] = {"value": rate, "unit": "atom-steps/s", "cores": cores, "kind": "port",
                                   "sample": f"oracle float32 (per-component op sequence) on {oracle_graph.num_nodes} atoms "
                                             f"({oracle_graph.num_graphs} graphs), {calls} calls, {cdt:.1f} s"}
    if cpu:
        res["speedup_vs_cpu"] = res["value"] / res["cpu_baseline"]["value"]
    return res


def run_other_workload(name, args, dev):
    """Throughput of the other BASELINE configurations (parity-tested in tests/test_gpu_configs.py).
    Prints one JSON line per call; the default invocation measures the 25k-atom configuration."""
    from flashcart_amd import o3
    from flashcart_amd.data import AtomicGraph, batch_graphs
    from flashcart_amd.data.synthetic import model_config, molecules, water_box
    res = {"workload": name, "n_gpus": 1, "steps": args.steps, "warmup": args.warmup, "dtype": "f32",
           "data": "synthetic (seeded)"}
    if name in CONFIG_LINES:
        res.update(config_line(name, dev, args.steps, args.warmup, not args.no_cpu_baseline,
                               extras=not args.trace_timed))
    elif name.startswith("train_"):
        run_training(name, args, dev, res)
    elif name == "lammps_fcc25k":
        # The LAMMPS ML-IAP path on the cfg 4 system as a single rank hands it over: owned atoms,
        # ghost images, pair indices and device pair vectors (SingleRankMLIAPData); one step =
        # FlashCartLAMMPSUnified.compute_forces (site energies + pair forces, ghost exchange hooks).
        from flashcart_amd.calculators import FlashCartLAMMPSUnified, SingleRankMLIAPData
        numbers, pos, cell, pbc = make_system()
        graph = AtomicGraph.from_arrays(numbers, pos, ["Cu", "Ni", "Fe", "Cr"], R_MAX, cell=cell, pbc=pbc)
        avg = graph.edge_index.shape[1] / graph.num_nodes
        model, cfg = build_model(avg)
        unified = FlashCartLAMMPSUnified(model.to(dev))
        data = SingleRankMLIAPData(graph, device=dev)
        dt, _ = _timed(lambda: unified.compute_forces(data), args.steps, args.warmup, dev)
        if not np.isfinite(data.energy):
            raise RuntimeError("non-finite energy")
        res.update({"metric": "atom-steps/s (LAMMPS ML-IAP compute_forces, 25k-atom fcc, L_max=3)",
                    "value": data.nlocal * args.steps / dt, "unit": "atom-steps/s",
                    "ms_per_step": 1e3 * dt / args.steps,
                    "config": {"n_local": data.nlocal, "n_ghost": data.ntotal - data.nlocal, "n_pairs": data.npairs,
                               "channels": 128, "l_max_edge_attrs": 3}})
        if not args.no_cpu_baseline:
            res["cpu_baseline"] = cpu_baseline(model.cpu(), cfg, avg)
            res["speedup_vs_cpu"] = res["value"] / res["cpu_baseline"]["value"]
    elif name == "nl_fcc25k":
        # Neighbour list of the cfg 4 system at r_max + skin, built on the GPU from positions in
        # HBM (fc_neighbor_list_device), a fresh N(0, 0.01^2) perturbation per build; the CPU
        # baseline is the host cell list of this library (identical pairs) on the same system.
        from flashcart_amd.data.neighbors import neighbor_pairs, neighbor_pairs_device
        numbers, pos, cell, pbc = make_system()
        rng = np.random.default_rng(1)
        steps = [torch.as_tensor(pos + rng.normal(scale=SIGMA_STEP, size=pos.shape), device=dev)
                 for _ in range(args.warmup + args.steps)]
        for k in range(args.warmup):
            neighbor_pairs_device(steps[k], cell, pbc, R_MAX + SKIN)
        torch.cuda.synchronize(dev)
        t0 = time.perf_counter()
        for k in range(args.warmup, args.warmup + args.steps):
            ei, _ = neighbor_pairs_device(steps[k], cell, pbc, R_MAX + SKIN)
        torch.cuda.synchronize(dev)
        dt = time.perf_counter() - t0
        ms = 1e3 * dt / args.steps
        res.update({"metric": "neighbour-list builds per second (25,000-atom fcc, cutoff 6 A, on the GPU)",
                    "value": args.steps / dt, "unit": "builds/s", "ms_per_step": ms,
                    "pairs": int(ei.shape[1]), "dtype": "f64",
                    "config": {"n_atoms": len(numbers), "cutoff": R_MAX + SKIN, "pbc": [True, True, True]}})
        if not args.no_cpu_baseline:
            t0 = time.perf_counter()
            calls = 0
            while calls < 3 or time.perf_counter() - t0 < 2.0:
                neighbor_pairs(pos, cell, pbc, R_MAX + SKIN)
                calls += 1
            rate = calls / (time.perf_counter() - t0)
            res["cpu_baseline"] = {"value": rate, "unit": "builds/s", "cores": 1, "kind": "port",
                                   "sample": f"host cell list (fc_neighbor_list), same system, {calls} builds"}
            res["speedup_vs_cpu"] = res["value"] / rate
    else:
        raise SystemExit(f"unknown workload {name}")
    print(json.dumps(res), flush=True)


def run_training(name, args, dev, res):
    """Force-loss training step: energies and forces with create_graph=True, the reference's
    default loss (Huber on per-atom energies, delta 0.005, weight 1; Huber on force components,
    delta 0.05, weight 0.01; src/flashcart/configs/default.yaml:95-106), its backward through
    the second derivatives, and an AdamW update of every parameter."""
    from flashcart_amd.data import AtomicGraph, batch_graphs
    from flashcart_amd.data.synthetic import fcc_alloy, model_config, molecules
    from flashcart_amd.model import FlashCartPotential
    if name == "train_molecules_192":
        mols = molecules(192, seed=0)
        elements = ["H", "C", "N", "O"]
        gs = [AtomicGraph.from_arrays(zz, pp, elements, R_MAX) for zz, pp in mols]
        graph, oracle_graph = batch_graphs(gs), batch_graphs(gs[:4])
    elif name == "train_fcc_2048":
        z, p, cell, pbc = fcc_alloy(8, 8, 8, a=3.6, jitter=0.05, seed=0)
        elements = ["Cu", "Ni", "Fe", "Cr"]
        graph = AtomicGraph.from_arrays(z, p, elements, R_MAX, cell=cell, pbc=pbc)
        zo, po, co, pbo = fcc_alloy(2, 2, 2, a=3.6, jitter=0.05, seed=0)
        oracle_graph = AtomicGraph.from_arrays(zo, po, elements, R_MAX, cell=co, pbc=pbo)
    else:
        raise SystemExit(f"unknown workload {name}")
    n_atoms, n_graphs = graph.num_nodes, graph.num_graphs
    avg = graph.edge_index.shape[1] / n_atoms
    torch.manual_seed(1234)
    model = FlashCartPotential.from_config(model_config(elements, 128, 3, r_max=R_MAX, avg_neighbors=avg)).to(dev)
    opt = torch.optim.AdamW(model.parameters(), lr=1e-4)
    gdev = graph.to(dev)
    gen = torch.Generator().manual_seed(0)
    e_ref = torch.randn(n_graphs, generator=gen).to(dev)
    f_ref = (0.1 * torch.randn(gdev.positions.shape, generator=gen)).to(dev)
    per_atom = gdev.n_atoms.to(torch.float32)

    def step():
        opt.zero_grad(set_to_none=True)
        out = model.predict(gdev, compute_forces=True, create_graph=True)
        loss = torch.nn.functional.huber_loss(out["energy"] / per_atom, e_ref, reduction="sum", delta=0.005) + \
            0.01 * torch.nn.functional.huber_loss(out["forces"], f_ref, reduction="sum", delta=0.05)
        loss.backward()
        opt.step()
        return loss

    torch.cuda.reset_peak_memory_stats(dev)
    dt, loss = _timed(step, args.steps, args.warmup, dev)
    if not torch.isfinite(loss):
        raise RuntimeError("non-finite training loss")
    ms = 1e3 * dt / args.steps
    res.update({"metric": "training atom-steps/s (energy+force loss, create_graph, AdamW)",
                "value": n_atoms * args.steps / dt, "unit": "atom-steps/s", "ms_per_step": ms,
                "structures_per_s": n_graphs * args.steps / dt,
                "peak_memory_gb": torch.cuda.max_memory_allocated(dev) / 1e9,
                "config": {"n_atoms": n_atoms, "n_graphs": n_graphs, "n_edges": int(graph.edge_index.shape[1]),
                           "channels": 128, "l_max_edge_attrs": 3, "l_max_hidden_feats": 2}})
    if not args.no_cpu_baseline:
        from oracle import model as OM
        cores = len(os.sched_getaffinity(0))
        torch.set_num_threads(cores)
        sd = {k: v.detach().cpu() for k, v in model.state_dict().items()}
        names = [k for k, _ in model.named_parameters()]
        gd = oracle_graph.to_dict()
        eo = torch.zeros(oracle_graph.num_graphs)
        fo = torch.zeros(oracle_graph.num_nodes, 3)
        OM.force_loss_grads(sd, model.to_model_config(), gd, eo, fo, names, dtype=torch.float32)  # warmup
        calls, t0 = 0, time.perf_counter()
        while calls < 1 or (calls < 3 and time.perf_counter() - t0 < 20.0):
            OM.force_loss_grads(sd, model.to_model_config(), gd, eo, fo, names, dtype=torch.float32)
            calls += 1
        cdt = time.perf_counter() - t0
        rate = oracle_graph.num_nodes * calls / cdt
        res["cpu_baseline"] = {"value": rate, "unit": "atom-steps/s", "cores": cores, "kind": "port",
                               "sample": f"oracle float32 force-loss gradients on {oracle_graph.num_nodes} atoms "
                                         f"({oracle_graph.num_graphs} graphs), {calls} calls, {cdt:.1f} s"}
        res["speedup_vs_cpu"] = res["value"] / rate


WORKLOADS = ("cfg4_fcc25k", "cfg1_tp_standalone", "cfg2_expansion_radial", "cfg3_water_1536", "cfg5_molecules_512",
             "train_molecules_192", "train_fcc_2048", "nl_fcc25k", "lammps_fcc25k")


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=100)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--cells", type=int, nargs=3, default=[25, 25, 10])
    ap.add_argument("--workload", choices=WORKLOADS, default="cfg4_fcc25k",
                    help="cfg4_fcc25k (the metric's configuration) or one of the other BASELINE configurations")
    ap.add_argument("--kernel-only", action="store_true",
                    help="only launch the layer-1 convolution forward and backward ops (7x each) and the two "
                         "calibration kernels (5x each), for counter runs")
    ap.add_argument("--profile-step", action="store_true",
                    help="two energy+forces steps on the first step graph, then the calibration kernels (2x), "
                         "for per-kernel counter runs")
    ap.add_argument("--power", action="store_true",
                    help="socket power (amd-smi) of the step's heavy ops, each looping alone for 4 s, and of "
                         "the energy+forces step")
    ap.add_argument("--trace-timed", action="store_true",
                    help="with --workload cfg3_water_1536 / cfg5_molecules_512: time the graph replays only (no "
                         "eager timing, no separate dominant-kernel launches, no MFMA event step), for kernel traces "
                         "that hold exactly the timed path")
    ap.add_argument("--mfma-launches", action="store_true",
                    help="one energy+forces step on the first step graph with HIP events around every MFMA launch: "
                         "prints each launch (entry point, shape, GFLOP, microseconds, TFLOP/s) as JSON lines")
    ap.add_argument("--no-configs", action="store_true",
                    help="measure only the metric's configuration (no lines for the other BASELINE configurations)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(json.dumps({"error": "this build runs on one GPU; multi-GPU runs are not part of it "
                                   "(periodic systems would shard by spatial domain with a one-layer halo "
                                   "exchange, molecule batches by molecule)", "n_gpus": args.gpus}))
        sys.exit(2)
    from flashcart_amd import _lib
    _lib.load()
    dev = torch.device("cuda", 0)
    if args.workload != "cfg4_fcc25k":
        run_other_workload(args.workload, args, dev)
        return
    numbers, pos, cell, pbc = make_system(*args.cells)
    if args.profile_step:
        sg = StepGraphs(numbers, pos, cell, pbc, ["Cu", "Ni", "Fe", "Cr"], 1)
        g = sg.graph(0, dev)
        model, _ = build_model(g.edge_index.shape[1] / len(numbers))
        model = model.to(dev)
        for _ in range(2):
            model.predict(g, compute_forces=True)
        cal = calibration_kernels(dev, 2)
        print(json.dumps({"profile_step": True, "n_atoms": len(numbers), "n_edges": int(g.edge_index.shape[1]),
                          **cal}), flush=True)
        return
    if args.power:
        sg = StepGraphs(numbers, pos, cell, pbc, ["Cu", "Ni", "Fe", "Cr"], 8)
        graphs = [sg.graph(k, dev) for k in range(8)]
        model, _ = build_model(graphs[0].edge_index.shape[1] / len(numbers))
        print(json.dumps({"power": power_per_kernel(model.to(dev), graphs, dev)}), flush=True)
        return
    if args.mfma_launches:
        sg = StepGraphs(numbers, pos, cell, pbc, ["Cu", "Ni", "Fe", "Cr"], 1)
        g = sg.graph(0, dev)
        model, _ = build_model(g.edge_index.shape[1] / len(numbers))
        model = model.to(dev)
        for _ in range(3):
            model.predict(g, compute_forces=True)
        rows = []
        summary = mfma_in_step(lambda: model.predict(g, compute_forces=True), dev, rows)
        for r in rows:
            print(json.dumps(r), flush=True)
        print(json.dumps({"summary": {k: v for k, v in summary.items() if k != "method"}}), flush=True)
        return
    if args.kernel_only:
        sg = StepGraphs(numbers, pos, cell, pbc, ["Cu", "Ni", "Fe", "Cr"], 1)
        model, _ = build_model(43.0)
        g = sg.graph(0, dev)
        ms, byts, ms_b, byts_b, _ = measure_dominant(model.to(dev), g, dev, reps=5, with_backward=True)
        cal = calibration_kernels(dev, 5)
        print(json.dumps({"kernel_only": True, "avg_launch_ms": ms, "algorithmic_bytes": byts,
                          "avg_bwd_op_ms": ms_b, "algorithmic_bytes_bwd": byts_b, **cal}), flush=True)
        return
    n_steps = args.warmup + args.steps
    log(f"building {n_steps} step graphs for {len(numbers)} atoms")
    t0 = time.time()
    sg = StepGraphs(numbers, pos, cell, pbc, ["Cu", "Ni", "Fe", "Cr"], n_steps)
    n_edges = [g[1].shape[1] for g in sg.graphs]
    avg_nbr = float(np.mean(n_edges)) / len(numbers)
    log(f"graphs ready in {time.time() - t0:.1f}s: mean E = {np.mean(n_edges):.0f} ({avg_nbr:.2f}/atom), "
        f"{sg.n_rebuild} skin-list builds")
    model, cfg = build_model(avg_nbr)
    model = model.to(dev)
    graphs = [sg.graph(k, dev) for k in range(n_steps)]
    torch.cuda.synchronize(dev)
    log("warmup")
    for k in range(args.warmup):
        out = model.predict(graphs[k], compute_forces=True)
    torch.cuda.synchronize(dev)
    log("timed steps")
    t0 = time.perf_counter()
    for k in range(args.warmup, n_steps):
        out = model.predict(graphs[k], compute_forces=True)
    torch.cuda.synchronize(dev)
    dt = time.perf_counter() - t0
    n_atoms = len(numbers)
    e = float(out["energy"][0])
    fmax = float(out["forces"].abs().max())
    if not (np.isfinite(e) and np.isfinite(fmax)):
        raise RuntimeError("non-finite energy or forces")
    log(f"{args.steps} steps in {dt:.3f}s ({1e3 * dt / args.steps:.3f} ms/step); E={e:.6f} |F|max={fmax:.4f}")
    # the TP ops on the first step graph: the graph `bench.py --kernel-only` builds for the counter
    # runs whose HBM bytes are the lines' `traffic` (same positions, same edge list)
    ms, byts, ms_b, byts_b, dom = measure_dominant(model, graphs[0], dev, with_backward=True)
    gbs = byts / (ms * 1e-3) / 1e9
    gbs_b = byts_b / (ms_b * 1e-3) / 1e9
    log(f"tp_fwd conv (layer 1): {ms:.3f} ms/launch, {byts / 1e9:.3f} GB algorithmic, {gbs:.1f} GB/s; "
        f"backward op: {ms_b:.3f} ms, {byts_b / 1e9:.3f} GB, {gbs_b:.1f} GB/s")
    mfma = mfma_in_step(lambda: model.predict(graphs[0], compute_forces=True), dev)
    log(f"MFMA launches in one step: {mfma['launches']}, {mfma['flops_per_step'] / 1e9:.1f} GFLOP in "
        f"{mfma['ms_per_step']:.3f} ms = {mfma['achieved']:.1f} TFLOP/s ({mfma['frac']:.3f} of peak)")
    result = {
        "metric": "atom-steps/s (energy+forces) at 25k atoms L_max=3",
        "value": n_atoms * args.steps / dt,
        "unit": "atom-steps/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": 1e3 * dt / args.steps,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic (seeded fcc random alloy, random-init weights)",
        "config": {"workload": "fcc_alloy_25k_L3_C128_energy_forces", "n_atoms": n_atoms,
                   "mean_edges": float(np.mean(n_edges)), "channels": 128, "l_max_edge_attrs": 3,
                   "l_max_hidden_feats": 2, "n_interactions": 2, "r_max": R_MAX, "parallelism": "single GPU"},
        # the step's largest kernel by time: the layer-1 TP backward op (the backward kernel + the
        # sender-ordered sum of its per-edge messages), on the compulsory bytes of its three gradients
        "roofline": {"bound": "hbm", "kernel": "tp_bwd_conv_kernel<2,3,3> + segment_rows_kernel (layer-1 TP "
                                                "convolution backward op)",
                     "achieved": gbs_b, "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": gbs_b / HBM_PEAK_GBS,
                     "traffic": MEASURED_TRAFFIC_BWD_BYTES,
                     "traffic_graph": f"first step graph, E={dom['edges']} (measured on E={TRAFFIC_E} by "
                                      "bench.py --kernel-only, which builds the same graph)",
                     "traffic_over_algorithmic": MEASURED_TRAFFIC_BWD_BYTES / byts_b,
                     "algorithmic_bytes": byts_b, "avg_launch_ms": ms_b, "edges": dom["edges"],
                     "weight_rows": dom["weight_rows"],
                     "distinct_bytes": dom["distinct_bytes_bwd"],
                     "distinct_frac": dom["distinct_bytes_bwd"] / (ms_b * 1e-3) / 1e9 / HBM_PEAK_GBS,
                     "note": "the step's largest TP kernel by time; algorithmic_bytes = the survey's compulsory "
                             "per-edge formula (weights read and their gradient written per edge); distinct_bytes "
                             "count each pair's shared weight row once"},
        # the north star's TP forward kernel as the step runs it (the two edges of a pair read one
        # weight row)
        "roofline_tp_fwd": {"bound": "hbm", "kernel": "tp_fwd_kernel<2,3,3> (conv, layer 1)", "achieved": gbs,
                            "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": gbs / HBM_PEAK_GBS,
                            "traffic": MEASURED_TRAFFIC_BYTES,
                            "traffic_graph": f"first step graph, E={dom['edges']} (measured on E={TRAFFIC_E})",
                            "traffic_over_algorithmic": MEASURED_TRAFFIC_BYTES / byts,
                            "algorithmic_bytes": byts, "avg_launch_ms": ms,
                            "distinct_bytes": dom["distinct_bytes_fwd"],
                            "distinct_frac": dom["distinct_bytes_fwd"] / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS},
        # in-step MFMA utilisation of the equivariant linear maps, dense layers and radial MLP
        "roofline_linear": mfma,
        "energy": e,
    }
    if not args.no_configs:
        result["configs"] = {}
        for name in CONFIG_LINES:
            log(f"configuration {name}")
            result["configs"][name] = config_line(name, dev, 30, 5, not args.no_cpu_baseline)
    if not args.no_cpu_baseline:
        log("cpu baseline")
        result["cpu_baseline"] = cpu_baseline(model.cpu(), cfg, avg_nbr)
        result["speedup_vs_cpu"] = result["value"] / result["cpu_baseline"]["value"]
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
