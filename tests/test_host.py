"""Host-side logic, the C ABI surface and the code generator (no GPU needed)."""

import ctypes
import itertools
import re
from fractions import Fraction
from pathlib import Path

import numpy as np
import pytest
import sympy as sp
import torch

ROOT = Path(__file__).resolve().parents[1]


def _declared_symbols():
    text = (ROOT / "include" / "flashcart_hip.h").read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(fc_[a-z0-9_]+)\s*\(", text)))


def test_library_exports_every_declared_symbol():
    from flashcart_amd import _lib
    lib = _lib.load()
    declared = _declared_symbols()
    assert len(declared) >= 20
    for name in declared:
        assert hasattr(lib, name), f"{name} declared in include/flashcart_hip.h but not exported"
    assert set(declared) == set(_lib.EXPORTED_SYMBOLS)
    assert lib.fc_kernel_l_max() == 3 and lib.fc_version() >= 100


def test_rank_limit_selects_the_library(monkeypatch):
    """FLASHCART_KERNEL_L_MAX (read at import, as by the reference) picks the rank-3 or the rank-4
    library and the limit the modules enforce; above 4 is refused."""
    import importlib

    from flashcart_amd import _lib
    from flashcart_amd.o3 import kernel_config
    assert _lib.library_path(3).endswith("libflashcart_hip.so")
    assert _lib.library_path(2).endswith("libflashcart_hip.so")
    assert _lib.library_path(4).endswith("libflashcart_hip_l4.so")
    try:
        monkeypatch.setenv("FLASHCART_KERNEL_L_MAX", "4")
        assert importlib.reload(kernel_config).KERNEL_L_MAX == 4
        monkeypatch.setenv("FLASHCART_KERNEL_L_MAX", "5")
        with pytest.raises(RuntimeError):
            importlib.reload(kernel_config)
        monkeypatch.delenv("FLASHCART_KERNEL_L_MAX")
        assert importlib.reload(kernel_config).KERNEL_L_MAX == 3
    finally:
        monkeypatch.delenv("FLASHCART_KERNEL_L_MAX", raising=False)
        importlib.reload(kernel_config)


@pytest.mark.skipif(not (ROOT / "flashcart_amd" / "libflashcart_hip_l4.so").exists(),
                    reason="libflashcart_hip_l4.so not built (FLASHCART_KERNEL_L_MAX=4 python -m flashcart_amd.build)")
def test_rank4_library_exports_and_metadata():
    """The rank-4 build exports the same symbols with the same descriptor layout and accepts rank 4
    (42 paths of 4 x 4 -> 4, the reference's count)."""
    from flashcart_amd import _lib
    lib = ctypes.CDLL(str(ROOT / "flashcart_amd" / "libflashcart_hip_l4.so"))
    for name in _declared_symbols():
        assert hasattr(lib, name), name
    lib.fc_kernel_l_max.restype = ctypes.c_int
    assert lib.fc_kernel_l_max() == 4
    lib.fc_tp_num_paths.argtypes = [ctypes.POINTER(_lib.TPDesc)]
    lib.fc_tp_out_dim.argtypes = [ctypes.POINTER(_lib.TPDesc)]
    lib.fc_tp_out_dim.restype = ctypes.c_int64
    d = _lib.tp_desc(4, 4, 4, 8, 1, False, False, False)
    assert lib.fc_tp_num_paths(ctypes.byref(d)) == 42
    assert lib.fc_tp_num_paths(ctypes.byref(_lib.tp_desc(5, 4, 4, 8, 1, False, False, False))) == -2


def test_abi_metadata_calls_without_gpu():
    from flashcart_amd import _lib
    lib = _lib.load()
    d = _lib.tp_desc(2, 3, 3, 128, 1, False, False, False)
    assert lib.fc_tp_num_paths(d) == 17
    assert lib.fc_tp_out_dim(d) == 71 * 128
    bad = _lib.tp_desc(4, 3, 3, 128, 1, False, False, False)
    assert lib.fc_tp_num_paths(bad) == -2  # FC_ERR_UNSUPPORTED_L
    assert lib.fc_status_string(6) == b"workspace missing or too small"


def test_path_order_matches_layout_contract():
    from flashcart_amd.codegen.cartesian import enumerate_paths
    got = [f"{a}{b}{c}{'s' if s else 'f'}" for a, b, c, s in enumerate_paths(2, 3, 3, False)]
    want = ["000f", "110f", "220f", "101f", "211f", "101s", "211s", "321s", "112f", "202f", "222f", "202s",
            "312s", "213f", "213s", "303s", "323s"]
    assert got == want


def test_path_counts():
    from flashcart_amd.o3.utils import count_output_paths
    assert count_output_paths(0, 3, 3) == ([1, 1, 1, 1], 4)
    assert count_output_paths(3, 3, 3)[1] == 23
    assert count_output_paths(3, 3, 0, symmetric_product=True) == ([4], 4)
    assert count_output_paths(2, 2, 2) == ([3, 4, 4], 11)


def test_codegen_coefficients_match_oracle():
    from flashcart_amd.codegen.emit_hip import ordered_triples, triple_coefficients
    from oracle.cartesian import path_tensor
    for r1, r2, lo in ordered_triples(3):
        B = np.zeros((2 * lo + 1, 2 * r1 + 1, 2 * r2 + 1))
        for (a, b, c), v in triple_coefficients(r1, r2, lo).items():
            B[a, b, c] = float(v)
        ref = path_tensor(r1, r2, lo) if r1 >= r2 else np.transpose(path_tensor(r2, r1, lo), (0, 2, 1))
        assert np.abs(B - ref).max() < 1e-13, (r1, r2, lo)


def test_codegen_expansion_matches_oracle():
    from flashcart_amd.codegen.cartesian import X, Y, Z, expansion_polynomials
    from oracle.ops import irreps
    r = torch.randn(7, 3, dtype=torch.float64)
    o = irreps(r, 3)
    col = 0
    for l in range(4):
        for p in expansion_polynomials(l):
            f = sp.lambdify((X, Y, Z), p, "numpy")
            v = np.broadcast_to(f(*[r[:, k].numpy() for k in range(3)]), (7,))
            assert np.allclose(v, o[:, col].numpy(), atol=1e-13)
            col += 1


def test_generated_header_is_current_and_literals_round_once():
    from flashcart_amd.codegen.emit_hip import emit_tp_header, flit
    hdr = (ROOT / "flashcart_amd" / "csrc" / "generated" / "fc_tp_paths.h").read_text()
    assert hdr == emit_tp_header()
    for frac in [Fraction(2, 3), Fraction(5, 9), Fraction(-3, 7), Fraction(1, 1)]:
        lit = flit(frac)
        assert np.float32(float(lit[:-1])) == np.float32(float(frac))


def test_neighbor_list_matches_brute_force():
    from flashcart_amd.data.neighbors import neighbor_pairs
    from flashcart_amd.data.synthetic import fcc_alloy
    from oracle.neighbors import brute_force_pairs
    rng = np.random.default_rng(0)
    z, p, cell, pbc = fcc_alloy(2, 2, 2, seed=1)
    tri = np.array([[7.0, 0.0, 0.0], [2.1, 6.5, 0.0], [-1.3, 0.7, 7.4]])
    cases = [(p, cell, pbc, 5.0), (rng.uniform(0, 6, (20, 3)) @ np.linalg.inv(np.eye(3) * 6) @ tri, tri,
                                   np.array([True, True, True]), 4.0),
             (rng.uniform(0, 5, (15, 3)), np.zeros((3, 3)), np.array([False] * 3), 3.0),
             (rng.uniform(0, 5, (15, 3)), np.eye(3) * 5.0, np.array([True, False, True]), 3.5)]
    for pos, c, pb, rc in cases:
        ei, sh = neighbor_pairs(pos, c, pb, rc)
        got = [(int(a), int(b)) + tuple(int(s) for s in S) for a, b, S in zip(ei[0], ei[1], sh)]
        want = brute_force_pairs(pos, c if abs(np.linalg.det(c)) > 1e-7 else np.eye(3), pb, rc)
        assert got == want
        assert np.all(np.diff(ei[0]) >= 0)


def test_neighbor_count_known_answers():
    """Average neighbour counts 1, 2 and 2/3 (reference tests/data/test_data.py:96-108)."""
    from flashcart_amd.data.neighbors import neighbor_pairs
    h = 1.5 * np.sqrt(3) / 2
    for pos, want in [([[0, 0, 0], [1.4, 0, 0]], 1.0), ([[0, 0, 0], [1.5, 0, 0], [0.75, h, 0]], 2.0),
                      ([[0, 0, 0], [1.0, 0, 0], [50.0, 0, 0]], 2.0 / 3.0)]:
        ei, _ = neighbor_pairs(np.array(pos, float), np.zeros((3, 3)), False, 5.0)
        assert abs(ei.shape[1] / len(pos) - want) < 1e-12


def test_periodic_self_images_exist():
    from flashcart_amd.data.neighbors import neighbor_pairs
    ei, sh = neighbor_pairs(np.zeros((1, 3)), np.eye(3) * 3.0, True, 3.5)
    assert ei.shape[1] == 6 and np.all(ei == 0)  # six face images of a single atom


REFERENCE_KEYS = [
    "embedding.weight", "radial_basis.r_min", "radial_basis.r_max", "cutoff_fn.poly_order", "cutoff_fn.r_max",
    "cutoff_fn.coeff1", "interactions.0.sqrt_avg_neighbors", "interactions.0.radial_mlp.0.weight",
    "interactions.0.radial_mlp.2.weight", "interactions.0.radial_mlp.4.weight", "interactions.0.linear_first.weight.0",
    "interactions.0.linear_second.weight.3", "interactions.0.skip_projection.weight",
    "interactions.0.layer_norm.weights.3", "interactions.1.skip_projection.weight.2",
    "products.0.skip_projection.weight.2", "products.0.layer_norm.weights.2", "products.0.product_linears.0.weight.3",
    "products.0.product_linears.2.weight.2", "products.1.product_linears.2.weight.0",
    "nonlinearities.0.value_linear.weight.3", "nonlinearities.0.gate_linear.weight",
    "nonlinearities.0.gate_linear.bias", "nonlinearities.1.output_linear.weight.0", "readout.readout_mlp.0.weight",
    "readout.readout_mlp.4.weight", "scale_shift.shifts", "scale_shift.scales",
]


def test_state_dict_names_and_shapes():
    from flashcart_amd.data.synthetic import model_config
    from flashcart_amd.model import FlashCartPotential
    m = FlashCartPotential.from_config(model_config(["Cu", "Ni", "Fe", "Cr"], 16, 3, avg_neighbors=40.0))
    sd = m.state_dict()
    for k in REFERENCE_KEYS:
        assert k in sd, k
    assert tuple(sd["interactions.1.radial_mlp.4.weight"].shape) == (17 * 16, 64)
    assert tuple(sd["interactions.1.linear_second.weight.3"].shape) == (16, 16 * 4)
    assert tuple(sd["products.0.product_linears.1.weight.3"].shape) == (16, 16 * 6)
    assert tuple(sd["readout.readout_mlp.0.weight"].shape) == (64, 32)
    assert not any("dummy_tp_weights" in k or "l_weights" in k for k in sd)
    assert abs(float(sd["interactions.0.sqrt_avg_neighbors"]) - 40.0 ** 0.5) < 1e-6


def test_ops_reject_cpu_tensors():
    from flashcart_amd import o3
    tp = o3.TensorProduct(1, 1, 1, 4, 4)
    x = torch.randn(3, 16)
    with pytest.raises(RuntimeError, match="ROCm"):
        tp(x, x, torch.randn(3, tp.n_total_paths * 4))
    with pytest.raises(RuntimeError, match="ROCm"):
        o3.Irreps(2).forward_normalized(torch.tensor([[1.0, 0.0, 0.0]]))


def test_tp_op_schema_follows_reference():
    """Positional schema of torch.ops.flashcart.tp_fwd/tp_bwd as registered by the reference
    (src/flashcart/o3/_tensor_product.py:332-352,588-611), extra arguments only at the end."""
    from flashcart_amd.o3 import _ops
    ref_fwd = ["in1", "in2", "weights", "idx_i", "idx_j", "in1_l_max", "in2_l_max", "out_l_max", "in1_features",
               "in2_features", "symmetric_product", "shared_weights", "in1_offs", "in2_offs", "out_sizes",
               "n_paths_per_l", "n_total_paths", "reduce_paths"]
    ref_bwd = ["grad_out"] + ref_fwd[:17] + ["reduce_paths", "need_grad_in1", "need_grad_in2", "need_grad_weights"]
    for op, ref in ((torch.ops.flashcart.tp_fwd.default, ref_fwd), (torch.ops.flashcart.tp_bwd.default, ref_bwd)):
        names = [a.name for a in op._schema.arguments]
        assert names[:len(ref)] == ref
        assert all(a.has_default_value() for a in op._schema.arguments[len(ref):])
    # Layout lists, as the reference builds them for (2 x 3 -> 3, C=128, in2 single channel):
    # _slice_offsets pads rank-block starts, _out_block_sizes = paths * (2l+1) * C.
    in1_offs, in2_offs, sizes, n_paths, total = _ops.tp_meta(2, 3, 3, 128, 1, False, False)
    assert in1_offs == [0, 128, 512, 0] and in2_offs == [0, 1, 4, 9]
    assert n_paths == [3, 5, 5, 4] and total == 17
    assert sizes == [3 * 128, 5 * 3 * 128, 5 * 5 * 128, 4 * 7 * 128]
    assert _ops.tp_meta(2, 2, 2, 8, 8, True, True)[2] == [8, 24, 40, 0]
    tp = __import__("flashcart_amd").o3.TensorProduct(1, 1, 1, 4, 4)
    x = torch.randn(3, 16)
    bad = list(tp.op_meta)
    bad[0] = [0, 8, 0, 0]
    with pytest.raises(ValueError, match="in1_offs"):
        torch.ops.flashcart.tp_fwd(x, x, torch.randn(3, tp.n_total_paths * 4), None, None, 1, 1, 1, 4, 4, False,
                                   False, *bad, False)


def test_checkpoint_round_trip(tmp_path):
    from flashcart_amd.data.synthetic import model_config
    from flashcart_amd.model import FlashCartPotential
    m = FlashCartPotential.from_config(model_config(["H", "O"], 8, 2, avg_neighbors=12.0))
    m.save_inference_checkpoint(tmp_path)
    m2 = FlashCartPotential.from_checkpoint(tmp_path)
    for (k, a), (k2, b) in zip(m.state_dict().items(), m2.state_dict().items()):
        assert k == k2 and torch.equal(a, b)
    assert torch.equal(m2.interactions[0].sqrt_avg_neighbors, m.interactions[0].sqrt_avg_neighbors)


def test_device_neighbor_list_host_fallback_decision():
    """Only the device list's size limit (-FC_ERR_SHAPE: > 1024 pairs for one atom or a shift
    component >= 512) sends the build to the host list; other failures stay errors."""
    from flashcart_amd.data.neighbors import host_fallback_needed

    assert host_fallback_needed(-4)
    assert not any(host_fallback_needed(s) for s in (0, 17, -1, -3, -5, -6, -7))


def test_linear_and_irreps_op_schemas_follow_reference():
    """torch.ops.flashcart.linear_fwd / linear_bwd / linear_dbwd / irreps_dbwd take the
    reference's positional arguments (src/flashcart/o3/_linear.py:328-343, :457-472, :571-591;
    src/flashcart/o3/_irreps.py:153-159) and return its outputs."""
    import flashcart_amd.o3._second_order  # noqa: F401  (registers the double backward)

    lists = ["in_offsets", "out_offsets", "weight_offsets", "m_values", "f_in_values", "f_out_values"]
    want = {
        "linear_fwd": ["x", "weights", "meta", "out_size", "use_fp64", "dot_input_precision"] + lists + ["scale"],
        "linear_bwd": ["grad_out", "x", "weights", "need_x", "need_weight", "use_fp64",
                       "dot_input_precision"] + lists + ["scale"],
        "linear_dbwd": ["grad_out", "x", "weights", "v_grad_x", "v_grad_weight", "use_fp64", "dot_input_precision",
                        "need_d_grad_out", "need_d_x", "need_d_weight", "has_v_grad_x",
                        "has_v_grad_weight"] + lists + ["scale"],
        "irreps_dbwd": ["grad_output", "x", "v", "l_max"],
    }
    n_out = {"linear_fwd": 1, "linear_bwd": 2, "linear_dbwd": 3, "irreps_dbwd": 2}
    for name, ref in want.items():
        schema = getattr(torch.ops.flashcart, name).default._schema
        assert [a.name for a in schema.arguments] == ref, name
        assert len(schema.returns) == n_out[name], name
    # the build's own residual / alpha variants live under names of their own
    assert [a.name for a in torch.ops.flashcart.equiv_linear_fwd.default._schema.arguments][-2:] == ["alpha",
                                                                                                      "residual"]


def test_rounded_row_allocations():
    from flashcart_amd import _lib
    assert [_lib.rounded_rows(n) for n in (0, 1, 15, 16, 17, 31, 32, 33)] == [0, 1, 15, 16, 18, 32, 32, 36]
    for n in [1080166, 1081496, 1100110, 1179648, 1179649, 7, 4096, 123457]:
        r = _lib.rounded_rows(n)
        q = 1 << max(n.bit_length() - 4, 0)
        assert n <= r < n + q and r % q == 0 and (r - n) <= n / 8
    # edge counts of an MD run drifting by ~0.1% per step share one rounded size
    assert len({_lib.rounded_rows(n) for n in range(1080166, 1179648, 997)}) == 1
    like = torch.empty(0)
    small = _lib.rows_empty(like, 1000, 16)
    assert small.shape == (1000, 16) and small.untyped_storage().nbytes() == 1000 * 16 * 4
    big = _lib.rows_empty(like, 1080166, 16)
    assert big.shape == (1080166, 16) and big.is_contiguous() and big.storage_offset() == 0
    assert big.untyped_storage().nbytes() == _lib.rounded_rows(1080166) * 16 * 4
    flat = _lib.rows_empty(like, 20_000_000, dtype=torch.int32)
    assert flat.shape == (20_000_000,) and flat.dtype == torch.int32


def test_alias_as_flashcart():
    """The reference's module names resolve to this package after alias_as_flashcart()."""
    import sys

    import flashcart_amd

    saved = {k: v for k, v in sys.modules.items() if k == "flashcart" or k.startswith("flashcart.")}
    try:
        for k in saved:
            del sys.modules[k]
        flashcart_amd.alias_as_flashcart()
        import flashcart
        import flashcart.data
        import flashcart.o3
        from flashcart.model import FlashCartPotential
        from flashcart.nn import InteractionLayer
        from flashcart.utils.lammps import lammps_data_slot

        assert flashcart is flashcart_amd and flashcart.o3.TensorProduct is flashcart_amd.o3.TensorProduct
        assert FlashCartPotential.__module__.startswith("flashcart_amd.model")
        assert InteractionLayer is flashcart_amd.nn.InteractionLayer
        assert flashcart.data.NeighborList is flashcart_amd.data.NeighborList and callable(lammps_data_slot)
    finally:
        for k in [k for k in sys.modules if k == "flashcart" or k.startswith("flashcart.")]:
            del sys.modules[k]
        sys.modules.update(saved)
