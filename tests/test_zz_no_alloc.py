"""The allocation-free neighbour list (fc_neighbor_list_device_noalloc) against the entry point
with a caller workspace (fc_neighbor_list_device), both called through the C ABI.

Two calls in a row, the second with a smaller system, so that the second call runs on the
scratch array that still holds the first call's contents; pairs and shifts must be identical
(index work, bit-exact), a system above the scratch limit must be refused with
FC_ERR_SCRATCH_LIMIT before anything is launched, and a call must leave the device's free
memory unchanged (it allocates nothing).
"""

import numpy as np
import pytest
import torch

from flashcart_amd import _lib
from flashcart_amd.data.synthetic import fcc_alloy, water_box

pytestmark = pytest.mark.gpu
DEV = "cuda"
FC_ERR_SCRATCH_LIMIT = 7


def _call(lib, fn, pos, cell, pbc, cutoff, with_workspace):
    n = pos.shape[0]
    cell_np = np.ascontiguousarray(cell, dtype=np.float64).reshape(3, 3)
    flags = np.ascontiguousarray(np.broadcast_to(np.asarray(pbc, dtype=np.int32), (3,)))
    cap = n * 128
    ei = torch.full((2, cap), -1, dtype=torch.int64, device=DEV)
    sh = torch.full((cap, 3), -1, dtype=torch.int32, device=DEV)
    stream = torch.cuda.current_stream().cuda_stream
    if with_workspace:
        ws_bytes = int(lib.fc_neighbor_list_device_workspace(n))
        ws = torch.empty(ws_bytes, dtype=torch.uint8, device=DEV)
        cnt = fn(n, pos.data_ptr(), cell_np.ctypes.data, flags.ctypes.data, float(cutoff), cap, ei[0].data_ptr(),
                 ei[1].data_ptr(), sh.data_ptr(), ws.data_ptr(), ws_bytes, stream)
    else:
        cnt = fn(n, pos.data_ptr(), cell_np.ctypes.data, flags.ctypes.data, float(cutoff), cap, ei[0].data_ptr(),
                 ei[1].data_ptr(), sh.data_ptr(), stream)
    assert 0 < cnt <= cap, cnt
    torch.cuda.synchronize()
    return ei[:, :cnt].cpu(), sh[:cnt].cpu()


def test_noalloc_matches_workspace_entry_point():
    lib = _lib.load()
    systems = []
    numbers, pos, cell, pbc = fcc_alloy(8, 8, 8, seed=3)          # 2,048 atoms, periodic
    systems.append((pos, cell, pbc, 5.0))
    numbers, pos, cell, pbc = water_box(64, seed=2)                # 192 atoms (smaller second call)
    systems.append((pos, cell, pbc, 4.0))
    for k, (p, cell, pbc, cutoff) in enumerate(systems):
        print(f"noalloc neighbour list: call {k}, {p.shape[0]} atoms, cutoff {cutoff}", flush=True)
        pos = torch.as_tensor(p, dtype=torch.float64, device=DEV).contiguous()
        want_ei, want_sh = _call(lib, lib.fc_neighbor_list_device, pos, cell, pbc, cutoff, True)
        got_ei, got_sh = _call(lib, lib.fc_neighbor_list_device_noalloc, pos, cell, pbc, cutoff, False)
        assert torch.equal(got_ei, want_ei) and torch.equal(got_sh, want_sh)


def test_noalloc_call_allocates_no_device_memory():
    """hipMemGetInfo's free bytes around a call (outputs allocated beforehand, one warm-up call):
    equal, so the entry point took no device memory of its own."""
    lib = _lib.load()
    numbers, p, cell, pbc = fcc_alloy(6, 6, 6, seed=5)  # 864 atoms, periodic
    pos = torch.as_tensor(p, dtype=torch.float64, device=DEV).contiguous()
    n = pos.shape[0]
    cell_np = np.ascontiguousarray(cell, dtype=np.float64).reshape(3, 3)
    flags = np.ascontiguousarray(np.broadcast_to(np.asarray(pbc, dtype=np.int32), (3,)))
    cap = n * 128
    ei = torch.full((2, cap), -1, dtype=torch.int64, device=DEV)
    sh = torch.full((cap, 3), -1, dtype=torch.int32, device=DEV)
    stream = torch.cuda.current_stream().cuda_stream

    def call():
        return lib.fc_neighbor_list_device_noalloc(n, pos.data_ptr(), cell_np.ctypes.data, flags.ctypes.data, 5.0,
                                                   cap, ei[0].data_ptr(), ei[1].data_ptr(), sh.data_ptr(), stream)
    print(f"noalloc neighbour list: free-memory check, {n} atoms", flush=True)
    first = call()
    torch.cuda.synchronize()
    free0 = torch.cuda.mem_get_info()[0]
    second = call()
    torch.cuda.synchronize()
    free1 = torch.cuda.mem_get_info()[0]
    assert 0 < first <= cap and second == first
    assert free1 == free0, f"free device memory changed by {free0 - free1} bytes during the call"


def test_noalloc_refuses_systems_above_the_scratch_limit():
    lib = _lib.load()
    n_max = int(lib.fc_neighbor_list_device_noalloc_max_atoms())
    assert n_max > 100_000
    n = n_max + 1
    cell = np.ascontiguousarray(np.eye(3) * 100.0)
    flags = np.ones(3, dtype=np.int32)
    pos = torch.zeros(4, 3, dtype=torch.float64, device=DEV)  # never read: refused on the sizes alone
    cnt = lib.fc_neighbor_list_device_noalloc(n, pos.data_ptr(), cell.ctypes.data, flags.ctypes.data, 5.0, 0,
                                              None, None, None, torch.cuda.current_stream().cuda_stream)
    assert cnt == -FC_ERR_SCRATCH_LIMIT
    assert "allocation-free" in lib.fc_status_string(FC_ERR_SCRATCH_LIMIT).decode()
