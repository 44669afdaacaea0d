"""ctypes binding of ``libflashcart_hip.so`` (the C ABI declared in include/flashcart_hip.h).

The library is loaded lazily on first use and must exist: there is no fallback
implementation. ``require_device`` rejects tensors that are not float32 on a ROCm
device before any pointer crosses the ABI.
"""

from __future__ import annotations

import ctypes
import os
from typing import Optional, Sequence

import torch

_HERE = os.path.dirname(os.path.abspath(__file__))
# Rank slots of the descriptors (FC_MAX_RANKS of include/flashcart_hip.h).
MAX_RANKS = 5
_ENV_L_MAX = "FLASHCART_KERNEL_L_MAX"


def library_path(l_max: Optional[int] = None) -> str:
    """The library for the requested rank limit (default: ``FLASHCART_KERNEL_L_MAX``, else 3):
    ``libflashcart_hip.so`` holds the kernels of ranks 0..3, ``libflashcart_hip_l4.so`` (built with
    ``FLASHCART_KERNEL_L_MAX=4 python -m flashcart_amd.build``) those of ranks 0..4, as the
    reference generates its kernels for the limit that variable sets."""
    if l_max is None:
        l_max = int(os.environ.get(_ENV_L_MAX, "3"))
    return os.path.join(_HERE, "libflashcart_hip_l4.so" if l_max >= 4 else "libflashcart_hip.so")


LIB_PATH = library_path()

c_int = ctypes.c_int
c_i32 = ctypes.c_int32
c_i64 = ctypes.c_int64
c_f32 = ctypes.c_float
c_f64 = ctypes.c_double
c_vp = ctypes.c_void_p
c_cp = ctypes.c_char_p


class RadialDesc(ctypes.Structure):
    _fields_ = [("basis", c_i32), ("n_radial", c_i32), ("r_min", c_f32), ("r_max", c_f32), ("poly_order", c_i32)]


class EdgeDesc(ctypes.Structure):
    _fields_ = [("l_max", c_i32), ("radial", RadialDesc)]


class CSR(ctypes.Structure):
    _fields_ = [
        ("n_nodes", c_i64), ("n_edges", c_i64), ("idx_j", c_vp), ("rowptr", c_vp),
        ("sender_perm", c_vp), ("sender_ptr", c_vp), ("n_sender_rows", c_i64), ("pair_slot", c_vp),
        ("idx_i", c_vp),
    ]


class TPDesc(ctypes.Structure):
    _fields_ = [
        ("in1_l_max", c_i32), ("in2_l_max", c_i32), ("out_l_max", c_i32),
        ("in1_features", c_i32), ("in2_features", c_i32),
        ("symmetric_product", c_i32), ("shared_weights", c_i32), ("reduce_paths", c_i32),
        ("alpha_div", c_vp),
    ]


class LinearDesc(ctypes.Structure):
    _fields_ = [
        ("in_l_max", c_i32), ("out_l_max", c_i32), ("in_features", c_i32), ("out_features", c_i32),
        ("in_paths", c_i32 * MAX_RANKS), ("weight", c_vp * MAX_RANKS), ("scale", c_f32 * MAX_RANKS),
    ]


class LinearDescF64(ctypes.Structure):
    _fields_ = [
        ("in_l_max", c_i32), ("out_l_max", c_i32), ("in_features", c_i32), ("out_features", c_i32),
        ("in_paths", c_i32 * MAX_RANKS), ("weight", c_vp * MAX_RANKS), ("scale", c_f64 * MAX_RANKS),
    ]


BASIS_CHEBYSHEV_AFFINE = 0
BASIS_CHEBYSHEV_COSINE = 1
BASIS_BESSEL = 2
BASIS_NONE = 3

# name -> (restype, argtypes)
_SIGNATURES = {
    "fc_version": (c_int, []),
    "fc_kernel_l_max": (c_int, []),
    "fc_status_string": (c_cp, [c_int]),
    "fc_irreps_fwd": (c_int, [c_i64, c_i32, c_vp, c_vp, c_vp]),
    "fc_irreps_bwd": (c_int, [c_i64, c_i32, c_vp, c_vp, c_vp, c_vp]),
    "fc_irreps_dbwd": (c_int, [c_i64, c_i32, c_vp, c_vp, c_vp, c_vp, c_vp, c_vp]),
    "fc_radial_fwd": (c_int, [ctypes.POINTER(RadialDesc), c_i64, c_vp, c_vp, c_vp, c_vp]),
    "fc_radial_bwd": (c_int, [ctypes.POINTER(RadialDesc), c_i64, c_vp, c_vp, c_vp, c_vp, c_vp]),
    "fc_shift_vectors": (c_int, [c_i64, c_i32, c_vp, c_vp, c_vp, c_vp, c_i64, c_vp, c_vp]),
    "fc_edge_geometry_fwd": (c_int, [ctypes.POINTER(EdgeDesc), c_i64, c_vp, c_vp, c_vp, c_vp, c_vp, c_vp, c_vp, c_vp, c_vp]),
    "fc_edge_geometry_bwd": (c_int, [ctypes.POINTER(EdgeDesc), c_i64, c_vp, c_vp, c_vp, c_vp, c_vp, c_vp, c_vp, c_vp, c_vp, c_vp]),
    "fc_edge_geometry_dbwd": (c_int, [ctypes.POINTER(EdgeDesc), c_i64] + [c_vp] * 14),
    "fc_csr_from_sorted": (c_int, [c_i64, c_vp, c_i64, c_vp, c_vp]),
    "fc_edge_grad_to_nodes": (c_int, [ctypes.POINTER(CSR), c_vp, c_vp, c_vp]),
    "fc_edge_pairs_workspace": (c_i64, [c_i64]),
    "fc_edge_pairs": (c_int, [ctypes.POINTER(CSR), c_vp, c_vp, c_vp, c_vp, c_vp, c_vp, c_i64, c_vp, c_vp, c_i64,
                              c_vp]),
    "fc_pair_inputs_fwd": (c_int, [c_i64, c_i32, c_vp, c_vp, c_vp, c_vp, c_vp]),
    "fc_pair_inputs_bwd": (c_int, [c_i64, c_i32, c_vp, c_vp, c_vp, c_vp, c_vp, c_vp, c_vp]),
    "fc_tp_num_paths": (c_int, [ctypes.POINTER(TPDesc)]),
    "fc_tp_out_dim": (c_i64, [ctypes.POINTER(TPDesc)]),
    "fc_tp_fwd": (c_int, [ctypes.POINTER(TPDesc), ctypes.POINTER(CSR), c_i64, c_vp, c_vp, c_vp, c_f32, c_vp, c_vp]),
    "fc_tp_bwd_workspace": (c_i64, [ctypes.POINTER(TPDesc), ctypes.POINTER(CSR), c_i64, c_int, c_int]),
    "fc_tp_bwd": (c_int, [ctypes.POINTER(TPDesc), ctypes.POINTER(CSR), c_i64, c_vp, c_vp, c_vp, c_vp, c_f32,
                          c_vp, c_vp, c_vp, c_vp, c_i64, c_vp]),
    "fc_tp_bwd_rows_acc": (c_int, [ctypes.POINTER(TPDesc), c_i64, c_vp, c_vp, c_vp, c_vp, c_f32, c_vp, c_i32,
                                   c_vp, c_i32, c_vp, c_vp, c_vp]),
    "fc_linear_fwd": (c_int, [ctypes.POINTER(LinearDesc), c_i64, c_vp, c_f32, c_vp, c_vp, c_vp]),
    "fc_linear_dgrad": (c_int, [ctypes.POINTER(LinearDesc), c_i64, c_vp, c_f32, c_vp, c_vp, c_vp]),
    "fc_dense_fwd": (c_int, [c_i64, c_i32, c_i32, c_vp, c_vp, c_f32, c_vp, c_i32, c_vp, c_vp, c_vp]),
    "fc_dense_fwd_pairsum": (c_int, [c_i64, c_i32, c_i32, c_vp, c_vp, c_vp, c_vp, c_f32, c_vp, c_vp]),
    "fc_dense_dgrad": (c_int, [c_i64, c_i32, c_i32, c_vp, c_vp, c_vp, c_f32, c_i32, c_vp, c_vp]),
    "fc_radial_mlp_fwd": (c_int, [c_i64, c_i32, c_vp, c_vp, c_f32, c_vp, c_f32, c_i32, c_vp, c_f32, c_vp, c_vp]),
    "fc_radial_mlp_hidden_fwd": (c_int, [c_i64, c_i32, c_vp, c_vp, c_f32, c_vp, c_f32, c_vp, c_vp]),
    "fc_species_density_fwd": (c_int, [ctypes.POINTER(CSR), c_i32, c_i32, c_i32, c_vp, c_vp, c_vp, c_vp, c_vp]),
    "fc_species_density_bwd": (c_int, [ctypes.POINTER(CSR), c_i32, c_i32, c_i32, c_vp, c_vp, c_vp, c_vp, c_vp, c_vp,
                                       c_vp]),
    "fc_species_maps": (c_int, [c_i32, c_i32, c_i32, c_i32, c_i32, c_i32, c_vp, c_vp, c_f32, c_vp, ctypes.POINTER(c_vp),
                                c_vp, ctypes.POINTER(c_vp), c_vp]),
    "fc_radial_mlp_bwd_pairsum": (c_int, [c_i64, c_i32, c_vp, c_vp, c_f32, c_vp, c_f32, c_vp, c_vp, c_vp]),
    "fc_radial_mlp_bwd": (c_int, [c_i64, c_i32, c_vp, c_vp, c_f32, c_vp, c_f32, c_vp, c_vp, c_vp]),
    "fc_linear_wgrad_workspace": (c_i64, [ctypes.POINTER(LinearDesc), c_i64, ctypes.POINTER(c_vp)]),
    "fc_linear_wgrad": (c_int, [ctypes.POINTER(LinearDesc), c_i64, c_vp, c_vp, c_f32, ctypes.POINTER(c_vp), c_vp,
                                c_i64, c_vp]),
    "fc_linear_fwd_f64": (c_int, [ctypes.POINTER(LinearDescF64), c_i64, c_vp, c_f64, c_vp, c_vp, c_vp]),
    "fc_linear_dgrad_f64": (c_int, [ctypes.POINTER(LinearDescF64), c_i64, c_vp, c_f64, c_vp, c_vp, c_vp]),
    "fc_linear_wgrad_f64_workspace": (c_i64, [ctypes.POINTER(LinearDescF64), c_i64, ctypes.POINTER(c_vp)]),
    "fc_linear_wgrad_f64": (c_int, [ctypes.POINTER(LinearDescF64), c_i64, c_vp, c_vp, c_f64, ctypes.POINTER(c_vp),
                                    c_vp, c_i64, c_vp]),
    "fc_dense_wgrad_workspace": (c_i64, [c_i64, c_i32, c_i32, c_i32]),
    "fc_dense_wgrad": (c_int, [c_i64, c_i32, c_i32, c_vp, c_vp, c_i32, c_vp, c_f32, c_vp, c_vp, c_vp, c_i64, c_vp]),
    "fc_silu_grad_mix": (c_int, [c_i64, c_vp, c_vp, c_vp, c_vp, c_vp, c_vp, c_vp]),
    "fc_segment_sum": (c_int, [c_i64, c_i64, c_vp, c_vp, c_vp, c_vp, c_vp]),
    "fc_gate_fwd": (c_int, [c_i64, c_int, c_int, c_vp, c_vp, c_int, c_vp, c_vp]),
    "fc_gate_bwd": (c_int, [c_i64, c_int, c_int, c_vp, c_vp, c_vp, c_int, c_vp, c_vp, c_vp]),
    "fc_rms_norm_fwd": (c_int, [c_i64, c_int, c_int, c_vp, c_vp, c_f32, c_vp, c_vp, c_vp]),
    "fc_rms_norm_bwd": (c_int, [c_i64, c_int, c_int, c_vp, c_vp, c_vp, c_vp, c_vp, c_vp]),
    "fc_rms_norm_dbwd": (c_int, [c_i64, c_int, c_int, c_vp, c_vp, c_vp, c_vp, c_vp, c_vp, c_vp, c_vp, c_vp]),
    "fc_gate_dbwd": (c_int, [c_i64, c_int, c_int, c_vp, c_vp, c_vp, c_int, c_vp, c_vp, c_vp, c_vp, c_vp, c_vp]),
    "fc_neighbor_list": (c_i64, [c_i64, c_vp, c_vp, c_vp, ctypes.c_double, c_i64, c_vp, c_vp, c_vp]),
    "fc_neighbor_list_device_workspace": (c_i64, [c_i64]),
    "fc_neighbor_list_device": (c_i64, [c_i64, c_vp, c_vp, c_vp, ctypes.c_double, c_i64, c_vp, c_vp, c_vp, c_vp,
                                        c_i64, c_vp]),
    "fc_neighbor_list_device_noalloc_max_atoms": (c_i64, []),
    "fc_neighbor_list_device_noalloc": (c_i64, [c_i64, c_vp, c_vp, c_vp, ctypes.c_double, c_i64, c_vp, c_vp, c_vp,
                                                c_vp]),
}

EXPORTED_SYMBOLS = tuple(_SIGNATURES)

_lib: Optional[ctypes.CDLL] = None


class HipLibraryError(RuntimeError):
    """The HIP library is missing, or one of its calls returned an error status."""


def load(path: str = LIB_PATH) -> ctypes.CDLL:
    """Load the library once (no GPU work happens at load time)."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(path):
        l4 = os.path.basename(path) == "libflashcart_hip_l4.so"
        raise HipLibraryError(
            f"{path} is missing: build it with `{'FLASHCART_KERNEL_L_MAX=4 ' if l4 else ''}python -m "
            "flashcart_amd.build` (flashcart_amd has no CPU implementation of its kernels)."
        )
    lib = ctypes.CDLL(path)
    for name, (res, args) in _SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    _lib = lib
    return lib


def check(status: int, what: str) -> None:
    if status != 0:
        msg = load().fc_status_string(status).decode()
        raise HipLibraryError(f"{what} failed: {msg} (status {status})")


def ptr(t: Optional[torch.Tensor]) -> Optional[int]:
    return None if t is None else t.data_ptr()


def stream_of(t: torch.Tensor) -> int:
    return torch.cuda.current_stream(t.device).cuda_stream


def require_device(name: str, t: torch.Tensor, dtype: torch.dtype = torch.float32) -> None:
    if not t.is_cuda:
        raise RuntimeError(
            f"flashcart_amd runs its kernels on ROCm devices only; `{name}` is on {t.device}. "
            "Move the model and inputs to a GPU (model.to('cuda'))."
        )
    if t.dtype != dtype:
        raise TypeError(f"`{name}` must be {dtype}, got {t.dtype}.")


def contig(name: str, t: torch.Tensor, dtype: torch.dtype = torch.float32) -> torch.Tensor:
    require_device(name, t, dtype)
    return t if t.is_contiguous() else t.contiguous()


# Per-edge tensors of a molecular-dynamics run change size every step (the edge count drifts by
# ~0.1% per step at 1M edges) and the largest are several GB. Exact-size requests make the
# caching allocator reserve a new segment for each new size until device memory runs out and
# it has to flush (~0.5 s per step once that happens). Rows are therefore allocated in steps of
# 1/8 of a power of two, so one set of segments serves every edge count within ~12% of it.
ROUNDED_ROWS_MIN_BYTES = 64 << 20


def rounded_rows(rows: int) -> int:
    """``rows`` rounded up to a multiple of 2^(floor(log2(rows)) - 3) (at most 12.5% more)."""
    if rows < 16:
        return rows
    q = 1 << (rows.bit_length() - 4)
    return -(-rows // q) * q


def rows_empty(like: torch.Tensor, rows: int, *cols: int, dtype: Optional[torch.dtype] = None) -> torch.Tensor:
    """Uninitialised (rows, *cols) tensor on ``like``'s device: the leading rows of a buffer of
    rounded_rows(rows) rows when it is ROUNDED_ROWS_MIN_BYTES or larger (a contiguous view)."""
    dtype = like.dtype if dtype is None else dtype
    width = 1
    for c in cols:
        width *= int(c)
    rows = int(rows)
    if rows * width * torch.empty((), dtype=dtype).element_size() < ROUNDED_ROWS_MIN_BYTES:
        return like.new_empty((rows, *cols), dtype=dtype)
    return like.new_empty((rounded_rows(rows), *cols), dtype=dtype)[:rows]


def tp_desc(in1_l_max, in2_l_max, out_l_max, in1_features, in2_features, symmetric, shared, reduced,
            alpha_div: Optional[torch.Tensor] = None) -> TPDesc:
    """``alpha_div``: optional one-element float32 device tensor s; the kernels then scale by
    alpha / s, reading s on the device."""
    return TPDesc(int(in1_l_max), int(in2_l_max), int(out_l_max), int(in1_features), int(in2_features),
                  int(bool(symmetric)), int(bool(shared)), int(bool(reduced)), ptr(alpha_div))


def linear_desc(in_l_max: int, out_l_max: int, in_features: int, out_features: int,
                in_paths: Sequence[int], weights: Sequence[torch.Tensor], scale: Sequence[float]):
    """The descriptor of an equivariant linear map: ``LinearDescF64`` when the weights are float64
    (the ``fc_linear_*_f64`` entry points), else ``LinearDesc``."""
    f64 = len(weights) > 0 and weights[0].dtype == torch.float64
    d = LinearDescF64() if f64 else LinearDesc()
    d.in_l_max, d.out_l_max, d.in_features, d.out_features = int(in_l_max), int(out_l_max), int(in_features), int(out_features)
    for l in range(MAX_RANKS):
        d.in_paths[l] = int(in_paths[l]) if l < len(in_paths) else 1
        d.weight[l] = weights[l].data_ptr() if l < len(weights) else None
        d.scale[l] = float(scale[l]) if l < len(scale) else 0.0
    return d


def radial_desc(basis: int, n_radial: int, r_min: float, r_max: float, poly_order: int) -> RadialDesc:
    return RadialDesc(int(basis), int(n_radial), float(r_min), float(r_max), int(poly_order))


def csr_struct(n_nodes: int, n_edges: int, idx_j, rowptr, sender_perm=None, sender_ptr=None,
               n_sender_rows: Optional[int] = None, pair_slot=None, idx_i=None) -> CSR:
    return CSR(int(n_nodes), int(n_edges), ptr(idx_j), ptr(rowptr), ptr(sender_perm), ptr(sender_ptr),
               int(n_nodes if n_sender_rows is None else n_sender_rows), ptr(pair_slot), ptr(idx_i))
